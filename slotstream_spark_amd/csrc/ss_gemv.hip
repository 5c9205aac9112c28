// Affine 4-bit GEMV: y[r][n] = sum_k x[r][k] * (q[n][k] * s[n][k/64] + b[n][k/64]) in fp32, the gemv of
// kernels/gemv_affine.py:214-262 for AffineWeight(bits=4, gs=64) (the lm_head is its largest instance, 248,320 x
// 2560). Weights are the MLX affine format: q int32 [N][K/8] (nibble i of a word at bits 4i), s and b bf16
// [N][K/64].
//
// A wave computes one tile of 16 weight rows for up to 4 rows of x with v_mfma_f32_16x16x32_bf16: the weight
// nibbles become bf16 1 + q/16 in registers (B operand, exact), x is staged once per workgroup as bf16 A fragments
// (fp32 x as bf16 high part plus bf16 residual), and each 64-element group adds 16 s * D + (b - 16 s) * sum(x) in
// fp32, the same factoring as the reference (sc * sum(q x) + bi * sum(x), :71-76). The 16 A rows carry (token,
// K half, x part), so one MFMA yields both groups of a 128-element chunk. Row r's result depends on x row r alone,
// so an R-row call equals R one-row calls bit for bit (the reference's invariance rule, kernels/tuning.py:1-10).
//
// The greedy epilogue keeps a running 64-bit argmax key per x row (first maximum, as np.argmax) and a non-finite
// flag in each wave, reduces them over the workgroup and combines workgroups with one atomic max per row (max is
// order-free, so the result does not depend on timing): the acceptance round after the lm_head
// (engine/generate.py:208-229) reads no logits.
#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

namespace {

constexpr int kGR = 4;  // x rows per launch

struct GemvArgs {
  const void* x;  // [R][K] bf16 or fp32
  int R, K, N, ntiles;
  const uint32_t* q;
  const uint16_t* s;
  const uint16_t* b;
  float* y;         // [R][N] or null
  uint64_t* rkey;   // [R] argmax keys, combined with atomic max (zero on entry), or null
  int* rbad;        // [R] non-finite flags, combined with atomic or (with rkey)
  int key_bf16;     // 1: the logits are lin's bf16 result: keys and y take the dot rounded to bf16
  // With rkey: the workgroups count their arrivals on `arrive` (zero on entry); the last one finishes the call when
  // `fin` (the call's last launch): the ids of all R_all rows (ids non-null) or the greedy round (gout non-null),
  // then zeroes every row's key and flag. The last workgroup of every launch zeroes `arrive`.
  int* arrive;
  int fin, R_all;
  uint64_t* rkey0;
  int* rbad0;
  int32_t* ids;
  const int32_t* drafts;
  int32_t* gout;
};

// The greedy round (engine/generate.py:208-229 at temperature 0) from the rows' argmax keys: row i's token is its
// argmax; a row holding a non-finite logit ends the round before it (flag 1); drafts are accepted while equal. out as
// ssmoe_accept_greedy. One thread.
SS_DEV void greedy_decide(const uint64_t* rkey, const int* rbad, const int32_t* drafts, int D, int V, int32_t* out) {
  int na = 0, ne = 0, fl = 0;
  for (int i = 0; i <= D; ++i) {
    if (rbad[i]) {
      fl |= 1;
      break;
    }
    const int tok = (int)(0xFFFFFFFFu - (uint32_t)rkey[i]);
    out[4 + i] = tok;
    ne = i + 1;
    if (i == D) break;
    const int d = drafts[i];
    if (d < 0 || d >= V) fl |= 2;
    if (tok != d) break;
    na = i + 1;
  }
  for (int i = ne; i <= D; ++i) out[4 + i] = -1;
  out[0] = na;
  out[1] = ne;
  out[2] = 0;
  out[3] = fl;
}

SS_DEV float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
SS_DEV float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
// The high or low bf16 of a pair as fp32 in one byte permute (bytes 3, 2 or 1, 0 of the pair to the top, zeros
// below; the selector depends on hi only).
SS_DEV float pick_half(uint32_t pair, int hi) {
  return __uint_as_float(__builtin_amdgcn_perm(pair, pair, hi ? 0x07060C0Cu : 0x05040C0Cu));
}

// bf16 pair (element d, element d+4) of 8 consecutive bf16 held as 4 words (e0e1, e2e3, e4e5, e6e7): the element
// order ss_nibbles_to_bf16 gives the weights.
SS_DEV uint4 perm_pairs(uint4 v) {
  uint4 f;
  f.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
  f.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
  f.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
  f.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  return f;
}

SS_DEV ss_u32x4 as_v(uint4 v) { return ss_u32x4{v.x, v.y, v.z, v.w}; }

SS_DEV bool is_nan(float v) { return v != v; }

// argmax key: the first maximum, NaN counting as the largest (np.argmax).
SS_DEV uint64_t amax_key(float v, int j) {
  const uint32_t k = is_nan(v) ? 0xFFFFFFFFu : ss_key(v == 0.f ? 0.f : v);
  return ((uint64_t)k << 32) | (0xFFFFFFFFu - (uint32_t)j);
}

// x A-fragment entry f = (((j * 4 + i) * 4 + g) * kGR + t) holds elements kb .. kb + 7 of x row t, kb = 128 j +
// 32 g + 8 i, as perm_pairs; fp32 x takes two entries (bf16 high parts, bf16 residuals). gx[G][t] = sum of group
// G of x row t, sequential in element order.
template <int NJG, bool XF32>
SS_DEV void stage_x(const GemvArgs& a, uint4* xfl, float (*gx)[kGR]) {
  const int tid = threadIdx.x;
  const int K = a.K, nt = a.R;
  constexpr int NF = NJG * 16 * kGR;
  constexpr int FPT = NF / 256;
  static_assert(NF % 256 == 0, "whole fragment entries per thread");
  uint4 fv[FPT][XF32 ? 2 : 1];
#pragma unroll
  for (int k = 0; k < FPT; ++k) {
    const int f = tid + 256 * k;
    const int t = f & 3, gg = (f >> 2) & 3, i = (f >> 4) & 3, j = f >> 6;
    const int tt = t < nt ? t : 0;
    const int kb = 128 * j + 32 * gg + 8 * i;
    if (XF32) {
      const float* xp = static_cast<const float*>(a.x) + (size_t)tt * K + kb;
      fv[k][0] = ldg16(xp);
      fv[k][XF32 ? 1 : 0] = ldg16(xp + 4);
    } else {
      fv[k][0] = ldg16(static_cast<const uint16_t*>(a.x) + (size_t)tt * K + kb);
    }
  }
  constexpr int GV = XF32 ? 16 : 8;
  uint4 gv[GV];
  const int q = tid < (K >> 6) * kGR ? tid : 0;
  const int gt = (q & 3) < nt ? (q & 3) : 0;
  const int Gi = q >> 2;
#pragma unroll
  for (int k = 0; k < GV; ++k) {
    if (XF32)
      gv[k] = ldg16(static_cast<const float*>(a.x) + (size_t)gt * K + 64 * Gi + 4 * k);
    else
      gv[k] = ldg16(static_cast<const uint16_t*>(a.x) + (size_t)gt * K + 64 * Gi + 8 * k);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < FPT; ++k) {
    const int f = tid + 256 * k;
    const bool live = (f & 3) < nt;
    if (XF32) {
      const uint4 v0 = fv[k][0], v1 = fv[k][XF32 ? 1 : 0];
      const float e0[4] = {__uint_as_float(v0.x), __uint_as_float(v0.y), __uint_as_float(v0.z), __uint_as_float(v0.w)};
      const float e1[4] = {__uint_as_float(v1.x), __uint_as_float(v1.y), __uint_as_float(v1.z), __uint_as_float(v1.w)};
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t b0 = ss_f32_to_bf16(e0[d]), b1 = ss_f32_to_bf16(e1[d]);
        hw[d] = b0 | (b1 << 16);
        lw[d] = ss_f32_to_bf16(e0[d] - ss_bf16_to_f32(b0)) | (ss_f32_to_bf16(e1[d] - ss_bf16_to_f32(b1)) << 16);
      }
      xfl[2 * f] = make_uint4(live ? hw[0] : 0u, live ? hw[1] : 0u, live ? hw[2] : 0u, live ? hw[3] : 0u);
      xfl[2 * f + 1] = make_uint4(live ? lw[0] : 0u, live ? lw[1] : 0u, live ? lw[2] : 0u, live ? lw[3] : 0u);
    } else {
      const uint4 pv = perm_pairs(fv[k][0]);
      xfl[f] = make_uint4(live ? pv.x : 0u, live ? pv.y : 0u, live ? pv.z : 0u, live ? pv.w : 0u);
    }
  }
  if (tid < (K >> 6) * kGR) {
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < GV; ++k) {
      const uint4 v = gv[k];
      if (XF32) {
        sum = sum + __uint_as_float(v.x);
        sum = sum + __uint_as_float(v.y);
        sum = sum + __uint_as_float(v.z);
        sum = sum + __uint_as_float(v.w);
      } else {
        sum = sum + bf_lo(v.x);
        sum = sum + bf_hi(v.x);
        sum = sum + bf_lo(v.y);
        sum = sum + bf_hi(v.y);
        sum = sum + bf_lo(v.z);
        sum = sum + bf_hi(v.z);
        sum = sum + bf_lo(v.w);
        sum = sum + bf_hi(v.w);
      }
    }
    gx[Gi][q & 3] = (q & 3) < nt ? sum : 0.f;
  }
}

}  // namespace

// Every wave walks the 16-row tiles t = 4 * block + wave, + 4 * grid.
template <int NJG, bool XF32>
__global__ __launch_bounds__(256, 2) void gemv_affine4_kernel(GemvArgs a) {
  constexpr int NXF = NJG * 16 * kGR * (XF32 ? 2 : 1);
  // x fragments, then as many zero entries: a lane whose A row is inactive reads the zeros at the same offsets, so
  // no MFMA operand needs a select.
  __shared__ uint4 xfl[2 * NXF];
  __shared__ float gx[NJG * 2][kGR];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int nt = a.R, K = a.K, N = a.N;
  stage_x<NJG, XF32>(a, xfl, gx);
  for (int i = tid; i < NXF; i += 256) xfl[NXF + i] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();
  const int m = lane & 15, at = m & 3, agrp = m >> 2, ahh = agrp >> 1, apart = agrp & 1;
  const bool a_act = ahh == (g >> 1) && at < nt && (XF32 || apart == 0);
  const uint4* xbase = a_act ? xfl : xfl + NXF;
  const int my_half = g >> 1, my_part = g & 1;
  const int stride = 4 * gridDim.x;
  uint64_t run_key[kGR] = {0, 0, 0, 0};
  uint32_t run_bad = 0;
#pragma unroll 1
  for (int tile = 4 * blockIdx.x + w; tile < a.ntiles; tile += stride) {
    const int row = tile * 16 + n;
    const int rr = row < N ? row : N - 1;
    const uint32_t* qrow = a.q + (size_t)rr * (K >> 3) + 4 * g;
    const uint16_t* srow = a.s + (size_t)rr * (K >> 6);
    const uint16_t* brow = a.b + (size_t)rr * (K >> 6);
    uint4 wv[NJG], sq[NJG / 4], bq[NJG / 4];  // a row's scales and biases: NJG dwords each, as 16-byte words
#pragma unroll
    for (int j = 0; j < NJG; ++j) wv[j] = ldg16(qrow + 16 * j);
#pragma unroll
    for (int c = 0; c < NJG / 4; ++c) {
      sq[c] = ldg16(srow + 8 * c);
      bq[c] = ldg16(brow + 8 * c);
    }
    uint32_t sv[NJG], bv[NJG];
#pragma unroll
    for (int c = 0; c < NJG / 4; ++c) {
      sv[4 * c] = sq[c].x, sv[4 * c + 1] = sq[c].y, sv[4 * c + 2] = sq[c].z, sv[4 * c + 3] = sq[c].w;
      bv[4 * c] = bq[c].x, bv[4 * c + 1] = bq[c].y, bv[4 * c + 2] = bq[c].z, bv[4 * c + 3] = bq[c].w;
    }
    __builtin_amdgcn_sched_barrier(0);
    float acc[kGR] = {0.f, 0.f, 0.f, 0.f};
    constexpr int JB = NJG >= 32 ? 1 : (NJG % 4 == 0 ? 2 : 1);  // chunks whose LDS operands are read ahead
#pragma unroll
    for (int j0 = 0; j0 < NJG; j0 += JB) {
      uint4 av4[JB][4];
      float4 gxv[JB];
#pragma unroll
      for (int jj = 0; jj < JB; ++jj) {
        const int j = j0 + jj;
        const uint4* fp = xbase + (size_t)(((j * 4) * 4 + g) * kGR + at) * (XF32 ? 2 : 1) + (XF32 ? apart : 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) av4[jj][i] = fp[(size_t)i * 16 * (XF32 ? 2 : 1)];
        gxv[jj] = reinterpret_cast<const float4*>(gx)[2 * j + my_half];
      }
#pragma unroll
      for (int jj = 0; jj < JB; ++jj) {
        const int j = j0 + jj;
        ss_f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ss_u32x4 av = as_v(av4[jj][i]);
          const uint32_t wd = i == 0 ? wv[j].x : i == 1 ? wv[j].y : i == 2 ? wv[j].z : wv[j].w;
          d = ss_mfma(av, ss_nibbles_to_bf16(wd), d);
        }
        const float sf = pick_half(sv[j], my_half);
        const float bf = pick_half(bv[j], my_half);
        const float s16 = sf * kNibbleScale;
        const float bp = my_part ? 0.f : __builtin_fmaf(-kNibbleScale, sf, bf);
        const float gxa[kGR] = {gxv[jj].x, gxv[jj].y, gxv[jj].z, gxv[jj].w};
#pragma unroll
        for (int r = 0; r < kGR; ++r) {
          acc[r] = __builtin_fmaf(s16, d[r], acc[r]);
          acc[r] = __builtin_fmaf(bp, gxa[r], acc[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kGR; ++r) {
      acc[r] = ss_rows_sum(acc[r]);
      if (a.key_bf16) acc[r] = ss_round_bf16(acc[r]);
    }
    if (a.y && g == 0 && row < N) {
#pragma unroll
      for (int r = 0; r < kGR; ++r)
        if (r < nt) a.y[(size_t)r * N + row] = acc[r];
    }
    if (a.rkey) {
#pragma unroll
      for (int r = 0; r < kGR; ++r) {
        const bool valid = row < N && r < nt;
        const uint64_t key = valid ? amax_key(acc[r], row) : 0;
        run_key[r] = key > run_key[r] ? key : run_key[r];
        run_bad |= (valid && (__float_as_uint(acc[r]) & 0x7F800000u) == 0x7F800000u) ? 1u << r : 0u;
      }
    }
  }
  if (a.rkey) {
    // The workgroup's maxima: wave, then the four waves in LDS, then one atomic max per x row (max is order-free).
    __shared__ uint64_t wkey[4][kGR];
    __shared__ uint32_t wbad[4];
#pragma unroll
    for (int r = 0; r < kGR; ++r) run_key[r] = ss_wave_max_u64(run_key[r]);
    run_bad = ss_wave_or(run_bad);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < kGR; ++r) wkey[w][r] = run_key[r];
      wbad[w] = run_bad;
    }
    __syncthreads();
    if (tid < nt) {
      uint64_t m = wkey[0][tid];
      uint32_t b = wbad[0];
      for (int ww = 1; ww < 4; ++ww) {
        m = wkey[ww][tid] > m ? wkey[ww][tid] : m;
        b |= wbad[ww];
      }
      __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(a.rkey + tid), (unsigned long long)m,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((b >> tid) & 1u) __hip_atomic_fetch_or(a.rbad + tid, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);  // the combines are performed (acknowledged) before the arrival below
    }
    // Every key, flag and the count are touched only by agent-scope atomics, which are performed at one coherent
    // point: a combine acknowledged before its workgroup's arrival is seen by the last workgroup's loads, with no
    // cache writeback or invalidation.
    __shared__ int s_last;
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(a.arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1;
    __syncthreads();
    if (s_last) {
      if (a.fin) {
        __shared__ uint64_t fkey[64];
        __shared__ int fbad[64];
        if (tid < a.R_all) {
          fkey[tid] = __hip_atomic_load(a.rkey0 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          fbad[tid] = __hip_atomic_load(a.rbad0 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (a.ids) a.ids[tid] = (int32_t)(0xFFFFFFFFu - (uint32_t)fkey[tid]);
          __hip_atomic_store(a.rkey0 + tid, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(a.rbad0 + tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (a.gout && tid == 0) greedy_decide(fkey, fbad, a.drafts, a.R_all - 1, a.N, a.gout);
      }
      if (tid == 0) __hip_atomic_store(a.arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

namespace {

// One resident wave of work per SIMD slot: the grid is the occupancy of this instantiation times the CU count.
template <int NJG, bool XF32>
hipError_t launch_tiles(const GemvArgs& a, hipStream_t st) {
  KernelCfg cfg;
  hipError_t e = kernel_cfg(reinterpret_cast<const void*>(gemv_affine4_kernel<NJG, XF32>), 256, 0, &cfg);
  if (e != hipSuccess) return e;
  const int grid = (cfg.per_cu > 0 ? cfg.per_cu : 1) * cfg.cus;
  const int need = (a.ntiles + 3) / 4;
  hipLaunchKernelGGL((gemv_affine4_kernel<NJG, XF32>), dim3(need < grid ? need : grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int NJG>
hipError_t launch_x(const GemvArgs& a, int x_f32, hipStream_t st) {
  return x_f32 ? launch_tiles<NJG, true>(a, st) : launch_tiles<NJG, false>(a, st);
}

hipError_t launch_chunk(const GemvArgs& a, int x_f32, hipStream_t st) {
  switch (a.K >> 7) {
    case 8: return launch_x<8>(a, x_f32, st);
    case 16: return launch_x<16>(a, x_f32, st);
    case 20: return launch_x<20>(a, x_f32, st);
    case 32: return launch_x<32>(a, x_f32, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool gemv_affine4_shape_ok(int K) { return K == 1024 || K == 2048 || K == 2560 || K == 4096; }

int64_t gemv_tiles(int N) { return ((int64_t)N + 15) / 16; }

hipError_t launch_gemv_affine4(const void* x, int x_f32, int R, int K, const int32_t* q, const uint16_t* s,
                               const uint16_t* b, int N, float* y, hipStream_t st) {
  GemvArgs a{};
  a.K = K;
  a.N = N;
  a.ntiles = (int)gemv_tiles(N);
  a.q = reinterpret_cast<const uint32_t*>(q);
  a.s = s;
  a.b = b;
  const size_t xrow = (size_t)K * (x_f32 ? 4 : 2);
  for (int r0 = 0; r0 < R; r0 += kGR) {
    a.x = static_cast<const uint8_t*>(x) + (size_t)r0 * xrow;
    a.R = R - r0 < kGR ? R - r0 : kGR;
    a.y = y + (size_t)r0 * N;
    hipError_t e = launch_chunk(a, x_f32, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Workspace of the argmax and greedy launches: keys [R] (8 bytes), flags [R], the arrival count; zero before the
// first call, and every call leaves it zero.
int64_t lm_head_greedy_workspace_bytes(int D, int N) {
  (void)N;
  return ((int64_t)(D + 1) * 8 + 255) / 256 * 256 + ((int64_t)(D + 1) * 4 + 255) / 256 * 256 + 256;
}

hipError_t launch_lm_head_greedy(const void* x, int x_f32, int D, int K, const int32_t* q, const uint16_t* s,
                                 const uint16_t* b, int N, const int32_t* drafts, void* work, float* logits,
                                 int32_t* out, hipStream_t st) {
  uint8_t* w = static_cast<uint8_t*>(work);
  uint64_t* rkey = reinterpret_cast<uint64_t*>(w);
  const int64_t ob = ((int64_t)(D + 1) * 8 + 255) / 256 * 256;
  int* rbad = reinterpret_cast<int*>(w + ob);
  const int R = D + 1;
  GemvArgs a{};
  a.arrive = reinterpret_cast<int*>(w + ob + ((int64_t)R * 4 + 255) / 256 * 256);
  a.R_all = R;
  a.rkey0 = rkey;
  a.rbad0 = rbad;
  a.drafts = drafts;
  a.gout = out;
  a.K = K;
  a.N = N;
  a.ntiles = (int)gemv_tiles(N);
  a.q = reinterpret_cast<const uint32_t*>(q);
  a.s = s;
  a.b = b;
  a.key_bf16 = x_f32 ? 0 : 1;  // lin returns the dtype of x
  const size_t xrow = (size_t)K * (x_f32 ? 4 : 2);
  for (int r0 = 0; r0 < R; r0 += kGR) {
    a.x = static_cast<const uint8_t*>(x) + (size_t)r0 * xrow;
    a.R = R - r0 < kGR ? R - r0 : kGR;
    a.y = logits ? logits + (size_t)r0 * N : nullptr;
    a.rkey = rkey + r0;
    a.rbad = rbad + r0;
    a.fin = r0 + kGR >= R;
    hipError_t e = launch_chunk(a, x_f32, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

int64_t lm_head_pq_workspace_bytes(int D, int N) { return (accept_work_floats(D, N) * 4 + 255) / 256 * 256; }

hipError_t launch_lm_head_pq(const void* x, int x_f32, int D, int K, const int32_t* q, const uint16_t* s,
                             const uint16_t* b, int N, const float* draft, const int32_t* drafts, const float* uniforms,
                             float temperature, void* work, float* logits, int32_t* out, int* err, hipStream_t st) {
  GemvArgs a{};
  a.K = K;
  a.N = N;
  a.ntiles = (int)gemv_tiles(N);
  a.q = reinterpret_cast<const uint32_t*>(q);
  a.s = s;
  a.b = b;
  a.key_bf16 = x_f32 ? 0 : 1;  // lin returns the dtype of x
  const size_t xrow = (size_t)K * (x_f32 ? 4 : 2);
  const int R = D + 1;
  for (int r0 = 0; r0 < R; r0 += kGR) {
    a.x = static_cast<const uint8_t*>(x) + (size_t)r0 * xrow;
    a.R = R - r0 < kGR ? R - r0 : kGR;
    a.y = logits + (size_t)r0 * N;
    hipError_t e = launch_chunk(a, x_f32, st);
    if (e != hipSuccess) return e;
  }
  AcceptArgs p{};
  p.target = logits;
  p.draft = draft;
  p.drafts = drafts;
  p.uniforms = uniforms;
  p.D = D;
  p.V = N;
  p.temperature = temperature;
  p.out = out;
  p.work = static_cast<float*>(work);
  p.err = err;
  return launch_accept_pq(p, st);
}

hipError_t launch_lm_head_argmax(const void* x, int x_f32, int R, int K, const int32_t* q, const uint16_t* s,
                                 const uint16_t* b, int N, int round_bf16, void* work, float* logits, int32_t* ids,
                                 hipStream_t st) {
  uint8_t* w = static_cast<uint8_t*>(work);
  uint64_t* rkey = reinterpret_cast<uint64_t*>(w);
  const int64_t ob = ((int64_t)R * 8 + 255) / 256 * 256;
  int* rbad = reinterpret_cast<int*>(w + ob);
  GemvArgs a{};
  a.arrive = reinterpret_cast<int*>(w + ob + ((int64_t)R * 4 + 255) / 256 * 256);
  a.R_all = R;
  a.rkey0 = rkey;
  a.rbad0 = rbad;
  a.ids = ids;
  a.K = K;
  a.N = N;
  a.ntiles = (int)gemv_tiles(N);
  a.q = reinterpret_cast<const uint32_t*>(q);
  a.s = s;
  a.b = b;
  a.key_bf16 = round_bf16 ? 1 : 0;
  const size_t xrow = (size_t)K * (x_f32 ? 4 : 2);
  for (int r0 = 0; r0 < R; r0 += kGR) {
    a.x = static_cast<const uint8_t*>(x) + (size_t)r0 * xrow;
    a.R = R - r0 < kGR ? R - r0 : kGR;
    a.y = logits ? logits + (size_t)r0 * N : nullptr;
    a.rkey = rkey + r0;
    a.rbad = rbad + r0;
    a.fin = r0 + kGR >= R;
    hipError_t e = launch_chunk(a, x_f32, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ss
