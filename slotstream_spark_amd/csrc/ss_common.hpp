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
  SS_ERR_TIMEOUT = 16,     // a persistent launch's bounded wait for other workgroups ran out
};

// ---------------------------------------------------------------- global-space access
// Pointers that reach the kernel through the argument struct or LDS are generic (flat) unless cast: flat accesses
// wait on both the vector-memory and LDS counters, so every hot global access goes through a global-space pointer.
#define SS_G __attribute__((address_space(1)))
template <class T>
SS_DEV SS_G T* gp(T* p) {
  return (SS_G T*)p;
}
// 16-byte global load / store through the builtin vector type (HIP's uint4 class does not take address spaces).
SS_DEV uint4 ldg16(const void* p) {
  const ss_u32x4 v = *(const SS_G ss_u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
SS_DEV void stg16(void* p, uint4 v) {
  ss_u32x4 t;
  t.x = v.x;
  t.y = v.y;
  t.z = v.z;
  t.w = v.w;
  *(SS_G ss_u32x4*)p = t;
}

// ---------------------------------------------------------------- bf16 <-> fp32
SS_DEV float ss_bf16_to_f32(uint32_t b) { return __uint_as_float((b & 0xFFFFu) << 16); }

// Round to nearest even; a NaN keeps its sign and top bits with the quiet bit set ((u >> 16) | 0x40), torch's rule.
// gfx950's conversion (v_cvt_pk_bf16_f32) is exactly that rule on every fp32 pattern, NaNs included, so no select
// follows it; ssmoe_bf16_round exports this function so that the rule is tested on the device.
SS_DEV uint32_t ss_f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

SS_DEV float ss_round_bf16(float f) { return ss_bf16_to_f32(ss_f32_to_bf16(f)); }

SS_DEV uint32_t ss_pack_bf16(float lo, float hi) { return ss_f32_to_bf16(lo) | (ss_f32_to_bf16(hi) << 16); }

// ---------------------------------------------------------------- exp
// exp(x) in fp32: Cody-Waite reduction x = n*ln2 + r (ln2 split in a 15-bit head, so n*LN2_HI is exact),
// then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2 in Horner form with fused multiply-adds
// (truncation error < 6e-9 relative), then a scale by 2^n built from the exponent bits (two steps near
// the subnormal range so only the last multiply rounds). The CPU restatement runs the same operations.
// Written without branches (selects only): inside a wave every lane takes the same instructions.
SS_DEV float ss_expf(float x) {
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
  // n is within [-150, 128] for every x the final selects keep; the clamp only keeps the conversion defined.
  int ni = (int)__builtin_fminf(__builtin_fmaxf(n, -160.f), 160.f);
  const bool big = ni > 127, tiny = ni < -120;
  p = big ? p * 2.0f : (tiny ? p * 5.42101086242752217003726400434970855712890625e-20f : p);  // 2^-64
  ni = big ? ni - 1 : (tiny ? ni + 64 : ni);
  float y = p * __uint_as_float((uint32_t)(ni + 127) << 23);
  y = x > 88.72283935546875f ? __uint_as_float(0x7F800000u) : y;
  y = x < -103.97208404541015625f ? 0.0f : y;
  return x != x ? x : y;
}

// ss_expf for x <= 0 (and NaN), with the same bits: there n <= 0, so the clamp's upper bound, the 2^128 range step and
// the overflow select never act and are left out (a softmax of values minus their maximum only needs this range).
SS_DEV float ss_expf_le0(float x) {
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
  int ni = (int)__builtin_fmaxf(n, -160.f);
  const bool tiny = ni < -120;
  p = tiny ? p * 5.42101086242752217003726400434970855712890625e-20f : p;  // 2^-64
  ni = tiny ? ni + 64 : ni;
  float y = p * __uint_as_float((uint32_t)(ni + 127) << 23);
  y = x < -103.97208404541015625f ? 0.0f : y;
  return x != x ? x : y;
}

// ---------------------------------------------------------------- order-preserving keys
// Positive floats: flip the sign bit; negative: bitwise not; NaN: key 0 (lowest).
// (kernels/topk_stable.py:1-13 semantics: -0.0 sorts just below +0.0.)
SS_DEV uint32_t ss_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0u;
  return (u & 0x80000000u) ? ~u : (u ^ 0x80000000u);
}

// Inverse of ss_key for non-NaN values (key 0 maps back to a NaN).
SS_DEV float ss_unkey(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k); }

// ---------------------------------------------------------------- lane exchange (wave64, VALU only)
// ss_xor_lane<M>(v) is v of lane l ^ M for M = 1, 2, 4, 8, from DPP moves inside a row of 16 lanes (GFX9
// encodings): quad_perm xor 1 (0xB1), xor 2 (0x4E) and xor 3 (0x1B); row_half_mirror (0x141, lane l <- l ^ 7);
// row_mirror (0x140, l <- l ^ 15). xor 4 = half_mirror then xor 3; xor 8 = mirror then half_mirror.
// ss_pair<M>(v, lo, hi), M = 16 or 32: gfx950's v_permlane16_swap / v_permlane32_swap of a register with itself,
// which leaves in every lane the values of both partner groups: lo = v[l & ~M], hi = v[l | M].
// Every exchange needs the whole wave active. LDS-routed shuffles (ds_bpermute) cost several times more.
template <int CTRL>
SS_DEV uint32_t ss_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

template <int M>
SS_DEV uint32_t ss_xor_lane(uint32_t v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "DPP exchange inside a row");
  if constexpr (M == 1) return ss_dpp<0xB1>(v);
  if constexpr (M == 2) return ss_dpp<0x4E>(v);
  if constexpr (M == 4) return ss_dpp<0x1B>(ss_dpp<0x141>(v));
  return ss_dpp<0x141>(ss_dpp<0x140>(v));
}

template <int M>
SS_DEV void ss_pair(uint32_t v, uint32_t& lo, uint32_t& hi) {
  static_assert(M == 16 || M == 32, "row-pair exchange");
  if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    lo = r[0];
    hi = r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    lo = r[0];
    hi = r[1];
  }
}

SS_DEV float ss_uf(uint32_t u) { return __uint_as_float(u); }
SS_DEV uint32_t ss_fu(float f) { return __float_as_uint(f); }

// Xor butterfly over the 64 lanes with a commutative operation: lane l combines with lane l^32, then l^16, ...,
// l^1. Because op(a, b) == op(b, a), every lane ends with the same bits, and the CPU restatement replays this
// tree (pairs (l, l^32) first).
template <class Op>
SS_DEV uint32_t ss_butterfly(uint32_t v, Op op) {
  uint32_t lo, hi;
  ss_pair<32>(v, lo, hi);
  v = op(lo, hi);
  ss_pair<16>(v, lo, hi);
  v = op(lo, hi);
  v = op(v, ss_xor_lane<8>(v));
  v = op(v, ss_xor_lane<4>(v));
  v = op(v, ss_xor_lane<2>(v));
  v = op(v, ss_xor_lane<1>(v));
  return v;
}

SS_DEV float ss_wave_sum(float v) {
  return ss_uf(ss_butterfly(ss_fu(v), [](uint32_t a, uint32_t b) { return ss_fu(ss_uf(a) + ss_uf(b)); }));
}

// Two independent ss_wave_sum butterflies with their steps interleaved (each value gets the bits ss_wave_sum gives
// it; the two exchange chains overlap instead of running back to back).
SS_DEV void ss_wave_sum2(float& a, float& b) {
  uint32_t l0, h0, l1, h1;
  ss_pair<32>(ss_fu(a), l0, h0);
  ss_pair<32>(ss_fu(b), l1, h1);
  a = ss_uf(l0) + ss_uf(h0);
  b = ss_uf(l1) + ss_uf(h1);
  ss_pair<16>(ss_fu(a), l0, h0);
  ss_pair<16>(ss_fu(b), l1, h1);
  a = ss_uf(l0) + ss_uf(h0);
  b = ss_uf(l1) + ss_uf(h1);
  a = a + ss_uf(ss_xor_lane<8>(ss_fu(a)));
  b = b + ss_uf(ss_xor_lane<8>(ss_fu(b)));
  a = a + ss_uf(ss_xor_lane<4>(ss_fu(a)));
  b = b + ss_uf(ss_xor_lane<4>(ss_fu(b)));
  a = a + ss_uf(ss_xor_lane<2>(ss_fu(a)));
  b = b + ss_uf(ss_xor_lane<2>(ss_fu(b)));
  a = a + ss_uf(ss_xor_lane<1>(ss_fu(a)));
  b = b + ss_uf(ss_xor_lane<1>(ss_fu(b)));
}

SS_DEV float ss_wave_max(float v) {
  return ss_uf(ss_butterfly(ss_fu(v), [](uint32_t a, uint32_t b) { return ss_fu(fmaxf(ss_uf(a), ss_uf(b))); }));
}

SS_DEV uint32_t ss_wave_max_u32(uint32_t v) {
  return ss_butterfly(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}

SS_DEV uint32_t ss_wave_min_u32(uint32_t v) {
  return ss_butterfly(v, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}

SS_DEV uint32_t ss_wave_or(uint32_t v) {
  return ss_butterfly(v, [](uint32_t a, uint32_t b) { return a | b; });
}

// 64-bit maximum over the wave (both halves exchanged per step).
SS_DEV uint64_t ss_wave_max_u64(uint64_t v) {
  auto mx = [](uint64_t a, uint64_t b) { return a > b ? a : b; };
  auto join = [](uint32_t hi, uint32_t lo) { return ((uint64_t)hi << 32) | lo; };
  uint32_t l0, h0, l1, h1;
  ss_pair<32>((uint32_t)v, l0, h0);
  ss_pair<32>((uint32_t)(v >> 32), l1, h1);
  v = mx(join(l1, l0), join(h1, h0));
  ss_pair<16>((uint32_t)v, l0, h0);
  ss_pair<16>((uint32_t)(v >> 32), l1, h1);
  v = mx(join(l1, l0), join(h1, h0));
  v = mx(v, join(ss_xor_lane<8>((uint32_t)(v >> 32)), ss_xor_lane<8>((uint32_t)v)));
  v = mx(v, join(ss_xor_lane<4>((uint32_t)(v >> 32)), ss_xor_lane<4>((uint32_t)v)));
  v = mx(v, join(ss_xor_lane<2>((uint32_t)(v >> 32)), ss_xor_lane<2>((uint32_t)v)));
  v = mx(v, join(ss_xor_lane<1>((uint32_t)(v >> 32)), ss_xor_lane<1>((uint32_t)v)));
  return v;
}

// Sum of the lanes l, l^16, l^32, l^48 (the four 16-lane rows) in the order (r0 + r1) + (r2 + r3) seen from the
// lane's own row pair: every lane of column l & 15 gets the same bits.
SS_DEV float ss_rows_sum(float v) {
  uint32_t lo, hi;
  ss_pair<16>(ss_fu(v), lo, hi);
  const float s = ss_uf(lo) + ss_uf(hi);
  ss_pair<32>(ss_fu(s), lo, hi);
  return ss_uf(lo) + ss_uf(hi);
}

SS_DEV float ss_readlane_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

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
// order (q0,q4) (q1,q5) (q2,q6) (q3,q7). The constant part (1.0) is small next to the spread of q/16, so the
// per-group correction (b - 16 s) * sum(x) cancels little of the MFMA dot.
constexpr float kNibbleScale = 16.f;
// (x & m) | c, for words that only feed other VALU instructions.
SS_DEV uint32_t ss_and_or(uint32_t x, uint32_t m, uint32_t c) { return (x & m) | c; }
// The same as one v_and_or_b32 (the compiler emits a separate and / or for this pattern). Its result must never be
// an MFMA operand: the compiler does not see an inline-asm write when it inserts the wait states a VALU write needs
// before an MFMA reads the register (one instruction apart, the MFMA read the register's previous value).
SS_DEV uint32_t ss_and_or_v(uint32_t x, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(c));
  return r;
}
// Two and-ors put nibble 2k (a) and 2k+1 (b) at bits 3..6 of byte k with bit 7 set, 0x80 | q << 3 (the low byte of
// bf16 1 + q/16); four byte permutes (compiler-generated, so the wait states before the MFMA are its own) pair each
// with the high byte 0x3F.
SS_DEV ss_u32x4 ss_nibbles_to_bf16(uint32_t w) {
  const uint32_t a = ss_and_or_v(w << 3, 0x78787878u, 0x80808080u);  // q0 q2 q4 q6
  const uint32_t b = ss_and_or_v(w >> 1, 0x78787878u, 0x80808080u);  // q1 q3 q5 q7
  const uint32_t hi = 0x3F3F3F3Fu;
  ss_u32x4 r;
  r.x = __builtin_amdgcn_perm(hi, a, 0x04020400u);  // (q0, q4)
  r.y = __builtin_amdgcn_perm(hi, b, 0x04020400u);  // (q1, q5)
  r.z = __builtin_amdgcn_perm(hi, a, 0x04030401u);  // (q2, q6)
  r.w = __builtin_amdgcn_perm(hi, b, 0x04030401u);  // (q3, q7)
  return r;
}
