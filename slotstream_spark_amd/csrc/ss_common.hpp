// Device helpers shared by every gfx950 kernel of the slotstream MoE verify path.
//
// Arithmetic that must be bit-identical to the CPU restatement (router logits, softmax, top-k keys,
// acceptance) is written here with an explicit operation order. Every file is compiled with
// -ffp-contract=off, so a*b+c is never fused unless the code says __builtin_fmaf.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SS_DEV __device__ __forceinline__

typedef __bf16 ss_bf16x8 __attribute__((ext_vector_type(8)));
typedef float ss_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t ss_u32x4 __attribute__((ext_vector_type(4)));

// Error bits a kernel may raise in the per-device status word (read back by ssmoe_device_error).
enum {
  SS_ERR_EXPERT_ID = 1,    // an expert id outside [0, E)
  SS_ERR_SLOT = 2,         // a map entry outside [0, n_slots) (an unmapped expert)
  SS_ERR_TOKEN = 4,        // a draft token outside [0, V)
  SS_ERR_NONFINITE = 8,    // non-finite logits reached a p/q decision
};

// ---------------------------------------------------------------- bf16 <-> fp32
SS_DEV float ss_bf16_to_f32(uint32_t b) { return __uint_as_float((b & 0xFFFFu) << 16); }

// Round to nearest even; NaN stays a quiet NaN with its sign.
SS_DEV uint32_t ss_f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) | 0x40u) & 0xFFFFu;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

SS_DEV float ss_round_bf16(float f) { return ss_bf16_to_f32(ss_f32_to_bf16(f)); }

SS_DEV uint32_t ss_pack_bf16(float lo, float hi) { return ss_f32_to_bf16(lo) | (ss_f32_to_bf16(hi) << 16); }

// ---------------------------------------------------------------- exp
// exp(x) in fp32: Cody-Waite reduction x = n*ln2 + r (ln2 split in a 15-bit head, so n*LN2_HI is exact),
// then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2 in Horner form with fused multiply-adds
// (truncation error < 6e-9 relative), then a scale by 2^n built from the exponent bits (two steps near
// the subnormal range so only the last multiply rounds). The CPU restatement runs the same operations.
SS_DEV float ss_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __uint_as_float(0x7F800000u);
  if (x < -103.97208404541015625f) return 0.0f;
  const float n = __builtin_rintf(x * 1.44269502162933349609375f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.428606765330187045037746429443359375e-06f, r);
  float p = 1.98412701138295233249664306640625e-04f;
  p = __builtin_fmaf(p, r, 1.38888892251998186111450195312500e-03f);
  p = __builtin_fmaf(p, r, 8.33333376795053482055664062500000e-03f);
  p = __builtin_fmaf(p, r, 4.16666679084300994873046875000000e-02f);
  p = __builtin_fmaf(p, r, 1.66666671633720397949218750000000e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) {
    p = p * 2.0f;
    ni -= 1;
  } else if (ni < -120) {
    p = p * 5.42101086242752217003726400434970855712890625e-20f;  // 2^-64
    ni += 64;
  }
  return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

// ---------------------------------------------------------------- order-preserving keys
// Positive floats: flip the sign bit; negative: bitwise not; NaN: key 0 (lowest).
// (kernels/topk_stable.py:1-13 semantics: -0.0 sorts just below +0.0.)
SS_DEV uint32_t ss_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0u;
  return (u & 0x80000000u) ? ~u : (u ^ 0x80000000u);
}

// ---------------------------------------------------------------- wave reductions (wave64)
SS_DEV float ss_shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
SS_DEV int ss_shfl_xor_i(int v, int m) { return __shfl_xor(v, m, 64); }

// Butterfly sum over the 64 lanes: lane l adds lane l^32, then l^16, ... l^1. Addition commutes, so
// every lane ends with the same bits; the CPU restatement replays this exact tree.
SS_DEV float ss_wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = v + ss_shfl_xor(v, m);
  return v;
}

SS_DEV float ss_wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, ss_shfl_xor(v, m));
  return v;
}

// ---------------------------------------------------------------- status word
// The word lives in the C-ABI translation unit; kernels receive its device address as an argument.
SS_DEV void ss_raise(int* err, int bit) {
  if (err) __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- affine-4bit record layout
// One expert record, pieces in the reference order (docs/model-and-repack.md:39-53,
// kernels/moe_gemv_affine.py:22-25): gate.w gate.s gate.b up.w up.s up.b down.w down.s down.b.
// w: uint32 [N, K/8] (nibble i of a word at bits 4i, low first); s, b: bf16 [N, K/64].
struct SsRecord {
  int64_t gw, gs, gb, uw, us, ub, dw, ds, db, bytes;
};

static inline __host__ __device__ SsRecord ss_record_layout(int64_t H, int64_t I) {
  SsRecord r;
  const int64_t w_gu = I * H / 2, sb_gu = I * (H / 64) * 2;
  const int64_t w_d = H * I / 2, sb_d = H * (I / 64) * 2;
  r.gw = 0;
  r.gs = r.gw + w_gu;
  r.gb = r.gs + sb_gu;
  r.uw = r.gb + sb_gu;
  r.us = r.uw + w_gu;
  r.ub = r.us + sb_gu;
  r.dw = r.ub + sb_gu;
  r.ds = r.dw + w_d;
  r.db = r.ds + sb_d;
  r.bytes = r.db + sb_d;
  return r;
}

// ---------------------------------------------------------------- MFMA helpers
// v_mfma_f32_16x16x32_bf16 lane layout (CDNA4): A[m][k] sits in lane m + 16*(k/8), element k%8;
// B[k][n] in lane n + 16*(k/8), element k%8; D[m][n] in lane n + 16*(m/4), element m%4.
SS_DEV ss_f32x4 ss_mfma(const ss_u32x4& a, const ss_u32x4& b, const ss_f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(ss_bf16x8, a), __builtin_bit_cast(ss_bf16x8, b), c,
                                                 0, 0, 0);
}

// 8 nibbles of one word -> 8 bf16 values 1 + q/16 (q in the top 4 mantissa bits of 1.0 = 0x3F80), in the pair
// order (q0,q4) (q1,q5) (q2,q6) (q3,q7): one shift and one and-or per pair. The constant part (1.0) is small next
// to the spread of q/16, so the per-group correction (b - 16 s) * sum(x) cancels little of the MFMA dot.
constexpr float kNibbleScale = 16.f;
SS_DEV ss_u32x4 ss_nibbles_to_bf16(uint32_t w) {
  ss_u32x4 b;
  b.x = ((w << 3) & 0x00780078u) | 0x3F803F80u;
  b.y = ((w >> 1) & 0x00780078u) | 0x3F803F80u;
  b.z = ((w >> 5) & 0x00780078u) | 0x3F803F80u;
  b.w = ((w >> 9) & 0x00780078u) | 0x3F803F80u;
  return b;
}
