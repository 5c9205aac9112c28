// The reference sampler on the device: Sampler.next (engine/sampler.py:76-108) over one row of logits.
//
// The steps and their float32 operations are the reference's, in its order: presence penalty on the raw logits
// (:80-82), argmax at temperature <= 0 (:83-84), division by the temperature (:85), the top-k threshold (:86-88),
// softmax (:89, :67-69), top-p (:90-97), min-p (:98-100) and the inverse-CDF draw with the caller's uniform
// (:101-108). The parameters arrive sanitized (SampleParams.sanitized, :45-64) and the uniform from the sampler's
// splitmix64 stream, both on the host. The order of every sum is defined here (the reference's comes from numpy):
//   * z, the top-p mass and the final total are hierarchical sums: a sub-chunk of 16 entries summed sequentially
//     from 0, the 64 sub-chunk totals of a 1024-entry chunk by the xor butterfly, the chunk totals sequentially;
//   * top-p ranks entry j by rho_j = key(p_j) << 20 | (2^20 - 1 - j) (probability descending, index ascending:
//     the stable argsort of :91); cum(rho) = hierarchical sum of p_i over rho_i > rho; j is kept iff
//     cum(rho_j) < top_p. cum falls as rho grows, so the kept set is rho_j >= r* for the smallest r* with
//     cum(r*) < top_p, found 4 bits at a time from the top (13 rounds, 16 candidates each);
//   * the draw takes the first entry whose hierarchical running sum reaches u * total (u == 0: exceeds 0),
//     chunk, then sub-chunk, then entry, each level falling back to the last nonzero one.
// exp is ss_expf. A total that is not finite and > 0 falls back to the argmax of the raw logits (:105-106).
#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

namespace {

constexpr int kSub = 16;
constexpr int kChunk = 64 * kSub;
constexpr int kPerLane = 16;  // chunk arrays of up to 1024 chunks (V <= 2^20)
constexpr int kRhoBits = 52;  // 32 key bits above 20 index bits

SS_DEV bool is_nan(float v) { return v != v; }

// NaN-largest order-preserving key with -0 == +0 (the order np.sort gives :87).
SS_DEV uint32_t nkey(float v) { return is_nan(v) ? 0xFFFFFFFFu : ss_key(v == 0.f ? 0.f : v); }

SS_DEV uint64_t rho_of(float p, int j) {
  return ((uint64_t)ss_key(p) << 20) | (uint64_t)((1u << 20) - 1u - (uint32_t)j);
}

// argmax key: the first maximum, NaN counting as the largest (np.argmax).
SS_DEV uint64_t amax_key(float v, int j) { return ((uint64_t)nkey(v) << 32) | (0xFFFFFFFFu - (uint32_t)j); }

struct SW {  // workspace views
  float* L;        // [V] logits after penalty / temperature / top-k mask
  float* P;        // [V] probabilities, then the final weights
  float* cmax;     // [nch]
  int* cnan;       // [nch]
  uint64_t* ckey;  // [nch] argmax keys of the penalized logits
  uint64_t* craw;  // [nch] argmax keys of the raw logits
  float* ctot;     // [nch]
  float* tsum;     // [16][nch]
  float* stot;     // [nch][64]
  float* state;    // [16]: 0 kth, 1 pmax, 2..3 r* (u64), 4 total
};

SS_DEV SW sw_of(void* w, int V, int nch) {
  SW s;
  uint8_t* b = static_cast<uint8_t*>(w);
  auto take = [&](size_t bytes) {
    uint8_t* p = b;
    b += (bytes + 255) & ~(size_t)255;
    return p;
  };
  s.L = reinterpret_cast<float*>(take((size_t)V * 4));
  s.P = reinterpret_cast<float*>(take((size_t)V * 4));
  s.cmax = reinterpret_cast<float*>(take((size_t)nch * 4));
  s.cnan = reinterpret_cast<int*>(take((size_t)nch * 4));
  s.ckey = reinterpret_cast<uint64_t*>(take((size_t)nch * 8));
  s.craw = reinterpret_cast<uint64_t*>(take((size_t)nch * 8));
  s.ctot = reinterpret_cast<float*>(take((size_t)nch * 4));
  s.tsum = reinterpret_cast<float*>(take((size_t)16 * nch * 4));
  s.stot = reinterpret_cast<float*>(take((size_t)64 * nch * 4));
  s.state = reinterpret_cast<float*>(take(64));
  return s;
}

size_t sw_bytes(int V, int nch) {
  auto r = [](size_t b) { return (b + 255) & ~(size_t)255; };
  return r((size_t)V * 4) * 2 + r((size_t)nch * 4) * 3 + r((size_t)nch * 8) * 2 + r((size_t)16 * nch * 4) +
         r((size_t)64 * nch * 4) + r(64);
}

struct SampArgs {
  const float* x;
  int V, nch;
  const int32_t* gen;
  int n_gen;
  float temperature, top_p, min_p, pp;
  int top_k;
  const float* u;
  int32_t* out;
  void* work;
};

SS_DEV bool in_sorted(const int32_t* g, int n, int j) {
  int lo = 0, hi = n - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    const int v = g[mid];
    if (v == j) return true;
    if (v < j) lo = mid + 1;
    else hi = mid - 1;
  }
  return false;
}

// Chunk c's hierarchical total of the lane values v[i] (entries c*1024 + 16*lane + i): sequential per lane, then
// the butterfly; `sub` receives the lane's sub-chunk total.
SS_DEV float chunk_sum(const float (&v)[kSub], float& sub) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kSub; ++i) s = s + v[i];
  sub = s;
  return ss_wave_sum(s);
}

// Every lane: ((a[0] + a[1]) + ...) + a[n-1] of a chunk array, from the lanes' registers (entry c in lane c % 64).
SS_DEV float seq_sum(const float* a, int n) {
  const int lane = threadIdx.x & 63;
  float v[kPerLane];
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) v[k] = lane + 64 * k < n ? a[lane + 64 * k] : 0.f;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) {
    if (64 * k >= n) break;
    const int m = n - 64 * k < 64 ? n - 64 * k : 64;
    for (int l = 0; l < m; ++l) s = s + ss_readlane_f(v[k], l);
  }
  return s;
}

SS_DEV uint64_t max_u64_of(const uint64_t* a, int n) {
  const int lane = threadIdx.x & 63;
  uint64_t m = 0;
#pragma unroll
  for (int k = 0; k < kPerLane; ++k)
    if (lane + 64 * k < n) m = a[lane + 64 * k] > m ? a[lane + 64 * k] : m;
  return ss_wave_max_u64(m);
}

}  // namespace

// 1. penalty and temperature; argmax keys of the penalized and of the raw logits.
__global__ __launch_bounds__(64) void samp_prep_kernel(SampArgs a) {
  SW w = sw_of(a.work, a.V, a.nch);
  const int c = blockIdx.x, lane = threadIdx.x;
  uint64_t kp = 0, kr = 0;
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + i * 64 + lane;
    if (j >= a.V) break;
    const float x = a.x[j];
    float l = (a.pp != 0.f && a.n_gen > 0 && in_sorted(a.gen, a.n_gen, j)) ? x - a.pp : x;
    const uint64_t k1 = amax_key(l, j), k2 = amax_key(x, j);
    kp = k1 > kp ? k1 : kp;
    kr = k2 > kr ? k2 : kr;
    if (a.temperature > 0.f) l = l / a.temperature;
    w.L[j] = l;
  }
  kp = ss_wave_max_u64(kp);
  kr = ss_wave_max_u64(kr);
  if (lane == 0) {
    w.ckey[c] = kp;
    w.craw[c] = kr;
  }
}

// Temperature <= 0: the argmax of the penalized logits.
__global__ __launch_bounds__(64) void samp_argmax_kernel(SampArgs a) {
  SW w = sw_of(a.work, a.V, a.nch);
  const uint64_t k = max_u64_of(w.ckey, a.nch);
  if (threadIdx.x == 0) {
    a.out[0] = (int32_t)(0xFFFFFFFFu - (uint32_t)k);
    a.out[1] = 0;
  }
}

// 2. top-k threshold: the top_k-th largest NaN-largest key (counting multiplicity), by a radix select over the
// row, 8 bits per pass; state[0] = its value.
__global__ __launch_bounds__(1024) void samp_kth_kernel(SampArgs a) {
  SW w = sw_of(a.work, a.V, a.nch);
  __shared__ int hist[256];
  __shared__ uint32_t s_prefix;
  __shared__ int s_need;
  const int tid = threadIdx.x;
  if (tid == 0) {
    s_prefix = 0;
    s_need = a.top_k;
  }
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = tid; i < 256; i += 1024) hist[i] = 0;
    __syncthreads();
    const uint32_t prefix = s_prefix;
    const uint32_t hmask = pass == 0 ? 0u : (0xFFFFFFFFu << (shift + 8));
    for (int j = tid; j < a.V; j += 1024) {
      const uint32_t k = nkey(w.L[j]);
      if ((k & hmask) == prefix) atomicAdd(&hist[(k >> shift) & 255], 1);  // integer counts: order-free
    }
    __syncthreads();
    if (tid == 0) {
      int need = s_need, b = 255;
      for (; b > 0; --b) {
        if (hist[b] >= need) break;
        need -= hist[b];
      }
      s_need = need;
      s_prefix = prefix | ((uint32_t)b << shift);
    }
    __syncthreads();
  }
  if (tid == 0) {
    const uint32_t k = s_prefix;
    w.state[0] = k == 0xFFFFFFFFu ? __uint_as_float(0x7FC00000u) : ss_unkey(k);
  }
}

// 3. top-k mask (when has_k) and the chunk maxima / NaN flags of the masked logits.
__global__ __launch_bounds__(64) void samp_max_kernel(SampArgs a, int has_k) {
  SW w = sw_of(a.work, a.V, a.nch);
  const int c = blockIdx.x, lane = threadIdx.x;
  const float kth = has_k ? w.state[0] : 0.f;
  float m = -__builtin_inff();
  int nan = 0;
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + i * 64 + lane;
    if (j >= a.V) break;
    float l = w.L[j];
    if (has_k && l < kth) {
      l = -__builtin_inff();
      w.L[j] = l;
    }
    nan |= is_nan(l);
    m = fmaxf(m, l);
  }
  m = ss_wave_max(m);
  nan = (int)ss_wave_or((uint32_t)nan);
  if (lane == 0) {
    w.cmax[c] = m;
    w.cnan[c] = nan;
  }
}

// 4. e = exp(l - m) into P and the chunk totals (m = NaN when any logit is NaN, as numpy's max).
__global__ __launch_bounds__(64) void samp_exp_kernel(SampArgs a) {
  SW w = sw_of(a.work, a.V, a.nch);
  const int c = blockIdx.x, lane = threadIdx.x;
  float m = -__builtin_inff();
  uint32_t nan = 0;
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) {
    const int q = lane + 64 * k;
    if (q < a.nch) {
      m = fmaxf(m, w.cmax[q]);
      nan |= (uint32_t)w.cnan[q];
    }
  }
  m = ss_wave_max(m);
  if (ss_wave_or(nan)) m = __uint_as_float(0x7FC00000u);
  float v[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    v[i] = j < a.V ? ss_expf(w.L[j] - m) : 0.f;
    if (j < a.V) w.P[j] = v[i];
  }
  float sub;
  const float t = chunk_sum(v, sub);
  if (lane == 0) w.ctot[c] = t;
}

// 5. p = e / z.
__global__ __launch_bounds__(64) void samp_norm_kernel(SampArgs a) {
  SW w = sw_of(a.work, a.V, a.nch);
  const int c = blockIdx.x, lane = threadIdx.x;
  const float z = seq_sum(w.ctot, a.nch);
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + i * 64 + lane;
    if (j < a.V) w.P[j] = w.P[j] / z;
  }
}

// 6. r* = 0 before the top-p rounds (a kernel, not a memset, so the launch sequence is safe to capture).
__global__ void samp_zero_r_kernel(SampArgs a) {
  SW w = sw_of(a.work, a.V, a.nch);
  if (threadIdx.x == 0) *reinterpret_cast<uint64_t*>(w.state + 2) = 0;
}

// 6a. top-p round: chunk c's hierarchical totals of p over rho > r | d << s | (2^s - 1), d = 0..15.
__global__ __launch_bounds__(64) void samp_topp_sums_kernel(SampArgs a, int s) {
  SW w = sw_of(a.work, a.V, a.nch);
  const int c = blockIdx.x, lane = threadIdx.x;
  const uint64_t r = *reinterpret_cast<const uint64_t*>(w.state + 2);
  const uint64_t ones = ((uint64_t)1 << s) - 1;
  float acc[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) acc[d] = 0.f;
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    const float p = j < a.V ? w.P[j] : 0.f;
    const uint64_t rho = j < a.V ? rho_of(p, j) : 0;
#pragma unroll
    for (int d = 0; d < 16; ++d) {
      const uint64_t hi = r | ((uint64_t)d << s) | ones;
      acc[d] = acc[d] + (rho > hi ? p : 0.f);
    }
  }
#pragma unroll
  for (int d = 0; d < 16; ++d) {
    const float t = ss_wave_sum(acc[d]);
    if (lane == 0) w.tsum[d * a.nch + c] = t;
  }
}

// 6b. top-p round: lane d sums candidate d's chunk totals in chunk order; the digit is the smallest d whose mass
// is below top_p (candidate 15 always is: it is the previous round's bound).
__global__ __launch_bounds__(64) void samp_topp_pick_kernel(SampArgs a, int s) {
  SW w = sw_of(a.work, a.V, a.nch);
  const int lane = threadIdx.x;
  const int d = lane < 16 ? lane : 15;
  float cum = 0.f;
  for (int c = 0; c < a.nch; ++c) cum = cum + w.tsum[d * a.nch + c];
  const uint64_t ok = __ballot(lane < 16 && cum < a.top_p);
  const int digit = ok ? (int)__builtin_ctzll(ok) : 15;
  if (lane == 0) {
    uint64_t* rp = reinterpret_cast<uint64_t*>(w.state + 2);
    *rp = *rp | ((uint64_t)digit << s);
  }
}

// 6c. keep rho >= r*; 7. (min_p > 0) chunk maxima of the kept probabilities.
__global__ __launch_bounds__(64) void samp_keep_kernel(SampArgs a, int has_p) {
  SW w = sw_of(a.work, a.V, a.nch);
  const int c = blockIdx.x, lane = threadIdx.x;
  const uint64_t r = has_p ? *reinterpret_cast<const uint64_t*>(w.state + 2) : 0;
  float m = -__builtin_inff();
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + i * 64 + lane;
    if (j >= a.V) break;
    float p = w.P[j];
    if (has_p && !(rho_of(p, j) >= r)) {
      p = 0.f;
      w.P[j] = p;
    }
    m = fmaxf(m, p);
  }
  m = ss_wave_max(m);
  if (lane == 0) w.cmax[c] = m;
}

// 8. min-p cutoff (when min_p > 0) and the hierarchical totals of the final weights.
__global__ __launch_bounds__(64) void samp_total_kernel(SampArgs a, int has_minp) {
  SW w = sw_of(a.work, a.V, a.nch);
  const int c = blockIdx.x, lane = threadIdx.x;
  float cutoff = 0.f;
  if (has_minp) {
    float pm = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < kPerLane; ++k)
      if (lane + 64 * k < a.nch) pm = fmaxf(pm, w.cmax[lane + 64 * k]);
    cutoff = ss_wave_max(pm) * a.min_p;
  }
  float v[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    float p = j < a.V ? w.P[j] : 0.f;
    if (has_minp && p < cutoff) {
      p = 0.f;
      if (j < a.V) w.P[j] = p;
    }
    v[i] = p;
  }
  float sub;
  const float t = chunk_sum(v, sub);
  w.stot[c * 64 + lane] = sub;
  if (lane == 0) w.ctot[c] = t;
}

// 9. the draw (one wave; every lane follows the same scan).
__global__ __launch_bounds__(64) void samp_draw_kernel(SampArgs a) {
  SW w = sw_of(a.work, a.V, a.nch);
  const int lane = threadIdx.x;
  const int nch = a.nch;
  float v[kPerLane];
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) v[k] = lane + 64 * k < nch ? w.ctot[lane + 64 * k] : 0.f;
  float total = 0.f;
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) {
    if (64 * k >= nch) break;
    const int m = nch - 64 * k < 64 ? nch - 64 * k : 64;
    for (int l = 0; l < m; ++l) total = total + ss_readlane_f(v[k], l);
  }
  const bool finite = (__float_as_uint(total) & 0x7F800000u) != 0x7F800000u;
  if (!finite || !(total > 0.f)) {
    const uint64_t k = max_u64_of(w.craw, nch);
    if (lane == 0) {
      a.out[0] = (int32_t)(0xFFFFFFFFu - (uint32_t)k);
      a.out[1] = 1;
    }
    return;
  }
  const float u = *a.u;
  const bool ge = u != 0.f;
  const float target = ge ? u * total : 0.f;
  auto hit = [&](float x) { return ge ? x >= target : x > target; };
  int cs = -1, clast = -1;
  float base = 0.f, run = 0.f;
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) {
    if (64 * k >= nch) break;
    const int m = nch - 64 * k < 64 ? nch - 64 * k : 64;
    for (int l = 0; l < m; ++l) {
      const float t = ss_readlane_f(v[k], l);
      const float nx = run + t;
      if (t > 0.f) clast = 64 * k + l;
      if (cs < 0 && hit(nx)) {
        cs = 64 * k + l;
        base = run;
      }
      run = nx;
    }
  }
  if (cs < 0) {
    cs = clast < 0 ? 0 : clast;
    base = 0.f;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      if (64 * k >= cs) break;
      const int m = cs - 64 * k < 64 ? cs - 64 * k : 64;
      for (int l = 0; l < m; ++l) base = base + ss_readlane_f(v[k], l);
    }
  }
  const float st = w.stot[cs * 64 + lane];
  int bs = -1, blast = -1;
  float sbase = base;
  run = base;
  for (int b = 0; b < 64; ++b) {
    const float t = ss_readlane_f(st, b);
    const float nx = run + t;
    if (t > 0.f) blast = b;
    if (bs < 0 && hit(nx)) {
      bs = b;
      sbase = run;
    }
    run = nx;
  }
  if (bs < 0) {
    bs = blast < 0 ? 0 : blast;
    sbase = base;
    for (int b = 0; b < bs; ++b) sbase = sbase + ss_readlane_f(st, b);
  }
  const int j0 = cs * kChunk + bs * kSub;
  const int jl = j0 + (lane & (kSub - 1));
  const float val = jl < a.V ? w.P[jl] : 0.f;
  int pick = -1, last = -1;
  run = sbase;
  for (int i = 0; i < kSub; ++i) {
    const int j = j0 + i;
    if (j >= a.V) break;
    const float e = ss_readlane_f(val, i);
    if (e > 0.f) last = j;
    run = run + e;
    if (hit(run)) {
      pick = j;
      break;
    }
  }
  if (pick < 0) pick = last >= 0 ? last : (j0 < a.V ? j0 : a.V - 1);
  if (lane == 0) {
    a.out[0] = pick;
    a.out[1] = 0;
  }
}

int64_t sample_workspace_bytes(int V) {
  const int nch = (V + kChunk - 1) / kChunk;
  return (int64_t)sw_bytes(V, nch);
}

hipError_t launch_sample(const float* x, int V, const int32_t* gen, int n_gen, float temperature, float top_p,
                         int top_k, float min_p, float pp, const float* u, void* work, int32_t* out, hipStream_t st) {
  SampArgs a{};
  a.x = x;
  a.V = V;
  a.nch = (V + kChunk - 1) / kChunk;
  a.gen = gen;
  a.n_gen = n_gen;
  a.temperature = temperature;
  a.top_p = top_p;
  a.top_k = top_k;
  a.min_p = min_p;
  a.pp = pp;
  a.u = u;
  a.out = out;
  a.work = work;
  const dim3 g(a.nch), b(64);
  hipLaunchKernelGGL(samp_prep_kernel, g, b, 0, st, a);
  if (!(temperature > 0.f)) {
    hipLaunchKernelGGL(samp_argmax_kernel, dim3(1), b, 0, st, a);
    return hipGetLastError();
  }
  const int has_k = top_k > 0 && top_k < V;
  if (has_k) hipLaunchKernelGGL(samp_kth_kernel, dim3(1), dim3(1024), 0, st, a);
  hipLaunchKernelGGL(samp_max_kernel, g, b, 0, st, a, has_k);
  hipLaunchKernelGGL(samp_exp_kernel, g, b, 0, st, a);
  hipLaunchKernelGGL(samp_norm_kernel, g, b, 0, st, a);
  const int has_p = top_p < 1.f;
  if (has_p) {
    hipLaunchKernelGGL(samp_zero_r_kernel, dim3(1), dim3(64), 0, st, a);
    for (int s = kRhoBits - 4; s >= 0; s -= 4) {
      hipLaunchKernelGGL(samp_topp_sums_kernel, g, b, 0, st, a, s);
      hipLaunchKernelGGL(samp_topp_pick_kernel, dim3(1), b, 0, st, a, s);
    }
  }
  const int has_minp = min_p > 0.f;
  if (has_p || has_minp) hipLaunchKernelGGL(samp_keep_kernel, g, b, 0, st, a, has_p);
  hipLaunchKernelGGL(samp_total_kernel, g, b, 0, st, a, has_minp);
  hipLaunchKernelGGL(samp_draw_kernel, dim3(1), b, 0, st, a);
  return hipGetLastError();
}

}  // namespace ss
