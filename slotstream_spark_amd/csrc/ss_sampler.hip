// The reference sampler on the device: Sampler.next (engine/sampler.py:76-108) over rows of logits.
//
// The steps and their float32 operations are the reference's, in its order: presence penalty on the raw logits
// (:80-82), argmax at temperature <= 0 (:83-84), division by the temperature (:85), the top-k threshold (:86-88),
// softmax (:89, :67-69), top-p (:90-97), min-p (:98-100) and the inverse-CDF draw with the caller's uniform
// (:101-108). The parameters arrive sanitized (SampleParams.sanitized, :45-64) and the uniforms from the sampler's
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
// Entries below the top-k threshold get weight exactly 0 (exp(-inf - m) = 0 for finite m; when m is not finite the
// total is NaN whatever the masked weights are, and the draw takes the fallback).
//
// Every launch covers R rows at once (blockIdx.y). Accept mode is the sampled verify round of _mtp_decode
// (engine/generate.py:208-229) over D+1 rows: row i is reached only if rows 0..i-1 drew their drafts, so its
// penalty set is seen + drafts[0..i) and all rows are drawn together; a last one-wave kernel walks the rows in
// order (a non-finite row ends the round without a draw, :210-212; the round goes on while the token equals the
// draft). The launch sequence depends only on the parameters, so it can be captured in a graph.
#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

namespace {

constexpr int kSub = 16;
constexpr int kChunk = 64 * kSub;
constexpr int kPerLane = 16;  // chunk arrays of up to 1024 chunks (V <= 2^20)
constexpr int kRhoBits = 52;  // 32 key bits above 20 index bits
constexpr int kRounds = kRhoBits / 4;
constexpr int kFlagNonfinite = 1, kFlagBadDraft = 2, kFlagFallback = 8;
constexpr int kSlot = 512;  // nonzero exp entries a top-k chunk lists for the compact top-p search
constexpr int kHistShards = 8;  // copies of each top-k histogram; chunk c adds to copy c % 8 (fewer atomics per bin)

SS_DEV bool is_nan(float v) { return v != v; }
SS_DEV bool is_finite(float v) { return (__float_as_uint(v) & 0x7F800000u) != 0x7F800000u; }

// NaN-largest order-preserving key with -0 == +0 (the order np.sort gives :87).
SS_DEV uint32_t nkey(float v) { return is_nan(v) ? 0xFFFFFFFFu : ss_key(v == 0.f ? 0.f : v); }

SS_DEV uint64_t rho_of(float p, int j) {
  return ((uint64_t)ss_key(p) << 20) | (uint64_t)((1u << 20) - 1u - (uint32_t)j);
}

// argmax key: the first maximum, NaN counting as the largest (np.argmax).
SS_DEV uint64_t amax_key(float v, int j) { return ((uint64_t)nkey(v) << 32) | (0xFFFFFFFFu - (uint32_t)j); }

// Byte offsets of one row's workspace; rows follow each other `bytes` apart.
struct Layout {
  size_t L, P, cmax, cnan, ckey, craw, cbad, etot, ftot, tsum, stot, hist, rr, res, cnz, surv, cres, bytes;
};

__host__ __device__ inline Layout layout_of(int V, int nch) {
  Layout l{};
  size_t o = 0;
  auto take = [&o](size_t b) {
    const size_t p = o;
    o += (b + 255) & ~(size_t)255;
    return p;
  };
  l.L = take((size_t)V * 4);                // logits after penalty and temperature
  l.P = take((size_t)V * 4);                // exp, then probabilities, then the final weights
  l.cmax = take((size_t)nch * 4);           // chunk maxima of the logits, later of the kept probabilities
  l.cnan = take((size_t)nch * 4);
  l.ckey = take((size_t)nch * 8);           // argmax keys of the penalized logits
  l.craw = take((size_t)nch * 8);           // argmax keys of the raw logits
  l.cbad = take((size_t)nch * 4);           // chunk holds a non-finite raw logit
  l.etot = take((size_t)nch * 4);           // chunk totals of exp
  l.ftot = take((size_t)nch * 4);           // chunk totals of the final weights
  l.tsum = take((size_t)2 * 16 * nch * 4);  // top-p candidate masses, two rounds alternating
  l.stot = take((size_t)64 * nch * 4);      // sub-chunk totals of the final weights
  l.hist = take(4 * kHistShards * 256 * 4);  // top-k radix histograms, one per 8-bit pass, kHistShards copies
  l.rr = take((size_t)(kRounds + 1) * 8);   // top-p prefix at the start of each round
  l.res = take(16);                         // token, fallback flag, non-finite row
  l.cnz = take((size_t)nch * 4);            // nonzero exp entries per chunk (top-k rows)
  l.surv = take((size_t)nch * kSlot * 8);   // a chunk's nonzero entries (index << 32 | e bits), up to kSlot
  l.cres = take(16);                        // compact top-p: r* (uint64), then 1 when it was found
  l.bytes = o;
  return l;
}

struct SW {
  float *L, *P, *cmax;
  int* cnan;
  uint64_t *ckey, *craw;
  int* cbad;
  float *etot, *ftot, *tsum, *stot;
  int* hist;
  uint64_t* rr;
  int* res;
  int* cnz;
  uint64_t* surv;
  uint64_t* cres;  // [0] r*, [1] found (1) or not (0)
};

SS_DEV SW sw_of(void* work, int V, int nch, int row) {
  const Layout l = layout_of(V, nch);
  uint8_t* b = static_cast<uint8_t*>(work) + (size_t)row * l.bytes;
  SW s;
  s.L = reinterpret_cast<float*>(b + l.L);
  s.P = reinterpret_cast<float*>(b + l.P);
  s.cmax = reinterpret_cast<float*>(b + l.cmax);
  s.cnan = reinterpret_cast<int*>(b + l.cnan);
  s.ckey = reinterpret_cast<uint64_t*>(b + l.ckey);
  s.craw = reinterpret_cast<uint64_t*>(b + l.craw);
  s.cbad = reinterpret_cast<int*>(b + l.cbad);
  s.etot = reinterpret_cast<float*>(b + l.etot);
  s.ftot = reinterpret_cast<float*>(b + l.ftot);
  s.tsum = reinterpret_cast<float*>(b + l.tsum);
  s.stot = reinterpret_cast<float*>(b + l.stot);
  s.hist = reinterpret_cast<int*>(b + l.hist);
  s.rr = reinterpret_cast<uint64_t*>(b + l.rr);
  s.res = reinterpret_cast<int*>(b + l.res);
  s.cnz = reinterpret_cast<int*>(b + l.cnz);
  s.surv = reinterpret_cast<uint64_t*>(b + l.surv);
  s.cres = reinterpret_cast<uint64_t*>(b + l.cres);
  return s;
}

struct SampArgs {
  const float* x;  // [R, V]
  int V, nch, R;
  const int32_t* gen;  // sorted penalty set
  int n_gen;
  const int32_t* drafts;  // accept mode: [R - 1]; row i also penalizes drafts[0..i)
  float temperature, top_p, min_p, pp;
  int top_k;
  const float* u;  // [R]
  int32_t* out;    // single row: [2] (token, flags); accept mode: [R + 4]
  int accept;
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

SS_DEV bool penalized(const SampArgs& a, int row, int j) {
  if (a.pp == 0.f) return false;
  if (a.n_gen > 0 && in_sorted(a.gen, a.n_gen, j)) return true;
  for (int k = 0; k < row; ++k)
    if (a.drafts[k] == j) return true;
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

// Stages a chunk array [n <= 1024] in LDS for the sequential scans below (one wave, every lane).
// A chunk array into LDS, zero-padded to a multiple of 16 entries (16-byte aligned).
SS_DEV const float* stage(const float* a, int n) {
  __shared__ __attribute__((aligned(16))) float buf[kPerLane * 64];
  const int lane = threadIdx.x & 63;
  float v[kPerLane];
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) v[k] = lane + 64 * k < n ? a[lane + 64 * k] : 0.f;
#pragma unroll
  for (int k = 0; k < kPerLane; ++k)
    if (lane + 64 * k < ((n + 15) & ~15)) buf[lane + 64 * k] = v[k];
  __syncthreads();
  return buf;
}

// ((s + b[0]) + b[1]) + ... + b[n-1] over a zero-padded, 16-byte aligned LDS array: 16 entries read as four
// unconditional 16-byte loads before their in-order adds, the bound applied by selects in the last, partial group.
SS_DEV float lds_seq_sum(const float* b, int n, float s) {
  // whole groups of 16 add without a bound check; only the last, partial group selects
  const float4* b4 = reinterpret_cast<const float4*>(b);
  for (int q = 0; q < n; q += 16) {
    const float4 a0 = b4[q / 4], a1 = b4[q / 4 + 1], a2 = b4[q / 4 + 2], a3 = b4[q / 4 + 3];
    const float t[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                         a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
    if (q + 16 <= n) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s = s + t[i];
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float nx = s + t[i];
        s = q + i < n ? nx : s;
      }
    }
  }
  return s;
}

// Every lane: ((a[0] + a[1]) + ...) + a[n-1] of a chunk array.
SS_DEV float seq_sum(const float* a, int n) { return lds_seq_sum(stage(a, n), n, 0.f); }

SS_DEV uint64_t max_u64_of(const uint64_t* a, int n) {
  const int lane = threadIdx.x & 63;
  uint64_t m = 0;
#pragma unroll
  for (int k = 0; k < kPerLane; ++k)
    if (lane + 64 * k < n) m = a[lane + 64 * k] > m ? a[lane + 64 * k] : m;
  return ss_wave_max_u64(m);
}

// Every lane: the logits' maximum over the chunk maxima (NaN when any chunk holds a NaN, as numpy's max).
SS_DEV float row_max(const SW& w, int nch) {
  const int lane = threadIdx.x & 63;
  float m = -__builtin_inff();
  uint32_t nan = 0;
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) {
    const int q = lane + 64 * k;
    if (q < nch) {
      m = fmaxf(m, w.cmax[q]);
      nan |= (uint32_t)w.cnan[q];
    }
  }
  m = ss_wave_max(m);
  return ss_wave_or(nan) ? __uint_as_float(0x7FC00000u) : m;
}

// One 8-bit radix step of the top-k select, whole wave: the bin of the need-th largest key among those counted in
// `hist` (bins descending, counting multiplicity); need becomes its rank inside the bin. Every lane gets the same.
SS_DEV void select_pass(const int* hist, int& need, uint32_t& prefix, int shift) {
  const int lane = threadIdx.x & 63;
  int hs[kHistShards][4];
#pragma unroll
  for (int c = 0; c < kHistShards; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q) hs[c][q] = hist[256 * c + 255 - 4 * lane - q];
  int h[4], s = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    h[q] = 0;
#pragma unroll
    for (int c = 0; c < kHistShards; ++c) h[q] += hs[c][q];
    s += h[q];
  }
  int incl = s;  // inclusive prefix over lanes = count of keys in bins >= 252 - 4 * lane
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off);
    if (lane >= off) incl += t;
  }
  const int above = incl - s;
  const bool mine = above < need && need <= incl;
  const uint64_t bal = __ballot(mine);
  const int src = bal ? (int)__builtin_ctzll(bal) : 0;
  int b = 0, nn = need - above;
  if (mine) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (h[q] >= nn) {
        b = 255 - 4 * lane - q;
        break;
      }
      nn -= h[q];
    }
  }
  b = __shfl(b, src);
  nn = __shfl(nn, src);
  need = nn;
  prefix |= (uint32_t)b << shift;
}

// One wave: the 4-bit top-p digit of a round from its candidate masses (lane d sums candidate d's chunk totals in
// chunk order): the smallest d whose mass is below top_p (candidate 15 always is: it is the previous round's bound).
// All lanes stage the masses in LDS first, so the loads are in flight together.
// The 16 candidate rows go to dynamic LDS (topp_lds_bytes(nch) at launch) at a zero-padded stride, so a launch
// holds only what its vocabulary needs.
SS_DEV int topp_digit(const float* tsum, int nch, float top_p) {
  constexpr int B = 32;
  extern __shared__ float4 topp_dyn[];
  float* tb = reinterpret_cast<float*>(topp_dyn);
  const int lane = threadIdx.x & 63;
  const int nchp = (nch + 15) & ~15;
  const int n = 16 * nch;
  for (int i = lane; i < 16 * nchp; i += 64) tb[i] = 0.f;
  for (int i0 = 0; i0 < n; i0 += 64 * B) {
    float v[B];
#pragma unroll
    for (int q = 0; q < B; ++q) {
      const int idx = i0 + 64 * q + lane;
      v[q] = idx < n ? tsum[idx] : 0.f;
    }
#pragma unroll
    for (int q = 0; q < B; ++q) {
      const int idx = i0 + 64 * q + lane;
      if (idx < n) {
        const int d = idx / nch;
        tb[d * nchp + (idx - d * nch)] = v[q];
      }
    }
  }
  __syncthreads();
  const float cum = lds_seq_sum(tb + (lane & 15) * nchp, nch, 0.f);
  const uint64_t ok = __ballot(lane < 16 && cum < top_p);
  return ok ? (int)__builtin_ctzll(ok) : 15;
}

}  // namespace

// Clears the top-k histograms of every row.
__global__ __launch_bounds__(256) void samp_begin_kernel(SampArgs a) {
  SW w = sw_of(a.work, a.V, a.nch, blockIdx.x);
  for (int i = threadIdx.x; i < 4 * kHistShards * 256; i += 256) w.hist[i] = 0;
}

// 1. penalty and temperature into L; argmax keys of the penalized and of the raw logits; non-finite flags; chunk
// maxima; (has_k) the first top-k histogram (top 8 key bits).
__global__ __launch_bounds__(64) void samp_prep_kernel(SampArgs a, int has_k) {
  const int c = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  SW w = sw_of(a.work, a.V, a.nch, row);
  const float* x = a.x + (size_t)row * a.V;
  __shared__ int hist[256];
  if (has_k) {
    for (int i = lane; i < 256; i += 64) hist[i] = 0;
    __syncthreads();
  }
  float xv[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    xv[i] = j < a.V ? x[j] : 0.f;
  }
  const bool sampled = a.temperature > 0.f;
  uint64_t kp = 0, kr = 0;
  uint32_t bad = 0, nan = 0;
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    if (j < a.V) {
      const float xx = xv[i];
      bad |= !is_finite(xx);
      float l = penalized(a, row, j) ? xx - a.pp : xx;
      const uint64_t k1 = amax_key(l, j), k2 = amax_key(xx, j);
      kp = k1 > kp ? k1 : kp;
      kr = k2 > kr ? k2 : kr;
      if (sampled) {
        l = l / a.temperature;
        w.L[j] = l;
        m = fmaxf(m, l);
        nan |= is_nan(l);
        if (has_k) atomicAdd(&hist[nkey(l) >> 24], 1);  // integer counts: order-free
      }
    }
  }
  kp = ss_wave_max_u64(kp);
  kr = ss_wave_max_u64(kr);
  bad = ss_wave_or(bad);
  nan = ss_wave_or(nan);
  m = ss_wave_max(m);
  if (lane == 0) {
    w.ckey[c] = kp;
    w.craw[c] = kr;
    w.cbad[c] = (int)bad;
    w.cmax[c] = m;
    w.cnan[c] = (int)nan;
  }
  if (has_k) {
    __syncthreads();
    for (int b = lane; b < 256; b += 64)
      if (hist[b]) atomicAdd(&w.hist[256 * (c % kHistShards) + b], hist[b]);
  }
}

// 2. top-k histogram pass 1..3: keys matching the prefix the earlier passes selected, next 8 bits.
__global__ __launch_bounds__(64) void samp_hist_kernel(SampArgs a, int pass) {
  const int c = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  SW w = sw_of(a.work, a.V, a.nch, row);
  __shared__ int hist[256];
  for (int i = lane; i < 256; i += 64) hist[i] = 0;
  int need = a.top_k;
  uint32_t prefix = 0;
  for (int p = 0; p < pass; ++p) select_pass(w.hist + kHistShards * 256 * p, need, prefix, 24 - 8 * p);
  const int shift = 24 - 8 * pass;
  const uint32_t hmask = 0xFFFFFFFFu << (shift + 8);
  float lv[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    lv[i] = j < a.V ? w.L[j] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    const uint32_t k = nkey(lv[i]);
    if (j < a.V && (k & hmask) == prefix) atomicAdd(&hist[(k >> shift) & 255], 1);
  }
  __syncthreads();
  for (int b = lane; b < 256; b += 64)
    if (hist[b]) atomicAdd(&w.hist[kHistShards * 256 * pass + 256 * (c % kHistShards) + b], hist[b]);
}

// 3. e = exp(l - m) into P (0 below the top-k threshold) and the chunk totals.
__global__ __launch_bounds__(64) void samp_exp_kernel(SampArgs a, int has_k) {
  const int c = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  SW w = sw_of(a.work, a.V, a.nch, row);
  float kth = -__builtin_inff();
  if (has_k) {
    int need = a.top_k;
    uint32_t prefix = 0;
    for (int p = 0; p < 4; ++p) select_pass(w.hist + kHistShards * 256 * p, need, prefix, 24 - 8 * p);
    kth = prefix == 0xFFFFFFFFu ? __uint_as_float(0x7FC00000u) : ss_unkey(prefix);
  }
  const float m = row_max(w, a.nch);
  float v[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    const float l = j < a.V ? w.L[j] : 0.f;
    v[i] = j < a.V ? (l < kth ? 0.f : ss_expf(l - m)) : 0.f;
    if (j < a.V) w.P[j] = v[i];
  }
  float sub;
  const float t = chunk_sum(v, sub);
  if (has_k) {
    // the chunk's nonzero entries in index order (lane-major: entry lane * 16 + i), up to kSlot of them
    int nz = 0;
#pragma unroll
    for (int i = 0; i < kSub; ++i) nz += v[i] != 0.f;
    int incl = nz;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d);
      incl += lane >= d ? o : 0;
    }
    int pos = incl - nz;
#pragma unroll
    for (int i = 0; i < kSub; ++i) {
      if (v[i] != 0.f) {
        if (pos < kSlot) {
          const uint32_t j = (uint32_t)(c * kChunk + lane * kSub + i);
          w.surv[(size_t)c * kSlot + pos] = ((uint64_t)j << 32) | __float_as_uint(v[i]);
        }
        ++pos;
      }
    }
    if (lane == 63) w.cnz[c] = incl;
  }
  if (lane == 0) w.etot[c] = t;
}

// 4'. Compact top-p (top-k rows, one workgroup per row). Only the top-k survivors carry weight, so cum(r) (the
// hierarchical mass of p over rho > r) is a step function of the survivors: with S(m) the masked hierarchical sum of
// the m survivors of largest rho (S grows with m: every partial sum is a monotone function of nonnegative terms),
// the smallest r with cum(r) < top_p is the rho of the m'-th survivor, m' the smallest m with S(m) >= top_p, or 0
// when S(all) < top_p: exactly the r* the 13 radix rounds find. S(m) is formed as the rounds form their masses:
// per chunk, lane b sums sub-chunk b's included entries in index order, the wave butterfly gives the chunk total,
// the chunk totals are summed in order. Four waves evaluate four values of m at a time. Rows with more than
// kCompact survivors, or a non-finite z, leave cres[1] = 0 and the rounds run as before.
constexpr int kCompact = 512;
constexpr int kCompactChunks = 160;  // active chunks the compact search holds (more: the rounds run)

__global__ __launch_bounds__(256) void samp_topp_compact_kernel(SampArgs a) {
  __shared__ int s_cnt[kPerLane * 64];   // nonzero count of active chunk q, then its chunk index
  __shared__ int s_ach[kPerLane * 64];
  __shared__ int s_aoff[kPerLane * 64 + 1];
  __shared__ int s_j[kCompact], s_rank[kCompact];
  __shared__ float s_p[kCompact];
  __shared__ uint64_t s_rho[kCompact];
  __shared__ int s_na, s_ok, s_digit;
  __shared__ __attribute__((aligned(16))) float s_leaf[kCompactChunks * 64];  // leaves; the fallback's masses
  __shared__ __attribute__((aligned(16))) float s_ct[kCompactChunks];
  __shared__ float s_S;
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  SW sw = sw_of(a.work, a.V, a.nch, row);
  const int nch = a.nch;
  // wave 0: the active chunks (nonzero count) in order, their survivor offsets, and whether every count fits
  if (w == 0) {
    int run = 0, na = 0, ok = 1;
    int cv[kPerLane];
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) cv[k] = lane + 64 * k < nch ? sw.cnz[lane + 64 * k] : 0;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      const int v = cv[k];
      ok &= v <= kSlot;
      const uint64_t act = __ballot(v > 0);
      const int before = __popcll(act & ((1ull << lane) - 1ull));
      int incl = v;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d);
        incl += lane >= d ? o : 0;
      }
      if (v > 0) {
        s_ach[na + before] = lane + 64 * k;
        s_aoff[na + before] = run + incl - v;
        s_cnt[na + before] = v;
      }
      run += __shfl(incl, 63);
      na += __popcll(act);
    }
    ok = ss_wave_or((uint32_t)!ok) ? 0 : 1;
    if (lane == 0) {
      s_aoff[na] = run;
      s_na = na;
      s_ok = ok && run <= kCompact && na <= kCompactChunks;
    }
  }
  __syncthreads();
  const int na = s_na;
  const int n = s_aoff[na];
  const float z = seq_sum(sw.etot, nch);  // the z round 0 would form
  if (!s_ok || !(z > 0.f) || !(z < __builtin_inff())) {
    // The 13 radix rounds of samp_topp_kernel inside the workgroup (same masses, digits and order; p = e / z formed
    // as round 0 forms it, P keeps e): r* = the digits at shifts 48, 44, ..., 0. Four waves take the chunks.
    float* tsl = s_leaf;  // [16][nch], nch <= 640
    uint64_t r = 0;
    for (int round = 0; round < kRounds; ++round) {
      const int sft = kRhoBits - 4 - 4 * round;
      const uint64_t r_hi = r >> (sft + 4);
      for (int c = w; c < nch; c += 4) {
        float pv[kSub];
#pragma unroll
        for (int i = 0; i < kSub; ++i) {
          const int j = c * kChunk + lane * kSub + i;
          pv[i] = j < a.V ? sw.P[j] / z : 0.f;
        }
        float acc[16];
#pragma unroll
        for (int d = 0; d < 16; ++d) acc[d] = 0.f;
#pragma unroll
        for (int i = 0; i < kSub; ++i) {
          const int j = c * kChunk + lane * kSub + i;
          const float pp = pv[i];
          if (j < a.V && pp != 0.f) {
            const uint64_t rho = rho_of(pp, j);
            const uint64_t hi = rho >> (sft + 4);
            const int lim = hi > r_hi ? 16 : (hi == r_hi ? (int)((rho >> sft) & 15) : 0);
#pragma unroll
            for (int d = 0; d < 16; ++d) acc[d] = acc[d] + (d < lim ? pp : 0.f);
          }
        }
#pragma unroll
        for (int d = 0; d < 16; ++d) {
          const float t = ss_wave_sum(acc[d]);
          if (lane == 0) tsl[d * nch + c] = t;
        }
      }
      __syncthreads();
      if (w == 0) {
        float cum = 0.f;
        for (int c = 0; c < nch; ++c) cum = cum + tsl[(lane & 15) * nch + c];
        const uint64_t okb = __ballot(lane < 16 && cum < a.top_p);
        if (lane == 0) s_digit = okb ? (int)__builtin_ctzll(okb) : 15;
      }
      __syncthreads();
      r |= (uint64_t)s_digit << sft;
    }
    if (tid == 0) {
      sw.cres[0] = r;
      sw.cres[1] = 1;
    }
    return;
  }
  // gather: survivor q of the row is entry q - aoff[t] of active chunk t (binary search); one batch of loads
  for (int q = tid; q < n; q += 256) {
    int lo = 0, hi = na - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_aoff[mid] <= q) lo = mid;
      else hi = mid - 1;
    }
    const uint64_t e = sw.surv[(size_t)s_ach[lo] * kSlot + (q - s_aoff[lo])];
    const int j = (int)(e >> 32);
    const float pj = __uint_as_float((uint32_t)e) / z;
    s_j[q] = j;
    s_p[q] = pj;
    s_rho[q] = rho_of(pj, j);
  }
  __syncthreads();
  // rank by rho, descending (rho values are distinct: they end in the index)
  for (int q = tid; q < n; q += 256) {
    const uint64_t r = s_rho[q];
    int rk = 0;
    for (int t = 0; t < n; ++t) rk += s_rho[t] > r;
    s_rank[q] = rk;
  }
  __syncthreads();
  // S(m) by the workgroup: leaf (active chunk t, sub-chunk b) = its survivors of rank < m summed in index order
  // (a leaf's survivors are adjacent in the list; its first one sums them), the wave butterfly over each chunk's 64
  // leaves, then the chunk totals in order. The leaf matrix is kept zero between evaluations.
  for (int q = tid; q < na * 64; q += 256) s_leaf[q] = 0.f;
  for (int q = tid; q < n; q += 256) {  // the leaf of survivor q and whether it starts its leaf
    int lo2 = 0, hi2 = na - 1;
    while (lo2 < hi2) {
      const int mid = (lo2 + hi2 + 1) >> 1;
      if (s_aoff[mid] <= q) lo2 = mid;
      else hi2 = mid - 1;
    }
    const int leaf = lo2 * 64 + ((s_j[q] & (kChunk - 1)) >> 4);
    const bool first = q == s_aoff[lo2] || ((s_j[q - 1] & (kChunk - 1)) >> 4) != ((s_j[q] & (kChunk - 1)) >> 4);
    s_cnt[q] = first ? leaf : -1;  // reused: leaf index at a leaf's first survivor, -1 elsewhere
  }
  __syncthreads();
  auto eval = [&](int m) {
    for (int q = tid; q < n; q += 256) {
      const int leaf = s_cnt[q];
      if (leaf >= 0) {
        float v = 0.f;
        for (int r = q; r < n && (r == q || s_cnt[r] < 0); ++r) {
          if (r != q && ((s_j[r] & (kChunk - 1)) >> 4) != ((s_j[q] & (kChunk - 1)) >> 4)) break;
          const float nx = v + s_p[r];
          v = s_rank[r] < m ? nx : v;
        }
        s_leaf[leaf] = v;
      }
    }
    __syncthreads();
    for (int t = w; t < na; t += 4) {
      const float ct = ss_wave_sum(s_leaf[t * 64 + lane]);
      if (lane == 0) s_ct[t] = ct;
    }
    __syncthreads();
    if (tid == 0) {
      float S = 0.f;
      for (int t = 0; t < na; t += 4) {
        const float4 c4 = *reinterpret_cast<const float4*>(s_ct + t);
        const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float nx = S + cv[e];
          S = t + e < na ? nx : S;
        }
      }
      s_S = S;
    }
    __syncthreads();
    return s_S;
  };
  // smallest m in [0, n] with S(m) >= top_p (n + 1 when none): binary search, S(lo) < top_p <= S(hi)
  int lo = 0, hi = n + 1;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (eval(mid) >= a.top_p) hi = mid;
    else lo = mid;
  }
  if (tid == 0) {
    uint64_t rs = 0;
    if (hi <= n)
      for (int q = 0; q < n; ++q)
        if (s_rank[q] == hi - 1) rs = s_rho[q];
    sw.cres[0] = rs;
    sw.cres[1] = 1;
  }
}

// 4. top-p round k: fold the previous round's digit into the prefix r, then chunk c's hierarchical masses of p over
// rho > r | d << s | (2^s - 1), d = 0..15. Round 0 also normalizes p = e / z.
__global__ __launch_bounds__(64) void samp_topp_kernel(SampArgs a, int round, int compact) {
  const int c = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  SW w = sw_of(a.work, a.V, a.nch, row);
  if (compact && w.cres[1]) return;  // r* is known
  const int nch = a.nch;
  const int s = kRhoBits - 4 - 4 * round;
  float pv[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    pv[i] = j < a.V ? w.P[j] : 0.f;
  }
  uint64_t r = 0;
  if (round > 0)
    r = w.rr[round - 1] | ((uint64_t)topp_digit(w.tsum + ((round - 1) & 1) * 16 * nch, nch, a.top_p) << (s + 4));
  if (c == 0 && lane == 0) w.rr[round] = r;
  if (round == 0) {
    const float z = seq_sum(w.etot, nch);
#pragma unroll
    for (int i = 0; i < kSub; ++i) {
      const int j = c * kChunk + lane * kSub + i;
      pv[i] = pv[i] / z;
      if (j < a.V) w.P[j] = pv[i];
    }
  }
  // rho > r | d << s | (2^s - 1) holds for every d when rho is above r in the bits over the round's digit, and for
  // d < t when those bits equal r's and t is rho's digit; p = 0 adds nothing, so zero entries are skipped.
  const uint64_t r_hi = r >> (s + 4);
  float acc[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) acc[d] = 0.f;
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    const float p = pv[i];
    if (j < a.V && p != 0.f) {
      const uint64_t rho = rho_of(p, j);
      const uint64_t hi = rho >> (s + 4);
      const int lim = hi > r_hi ? 16 : (hi == r_hi ? (int)((rho >> s) & 15) : 0);
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[d] = acc[d] + (d < lim ? p : 0.f);
    }
  }
  float* out = w.tsum + (round & 1) * 16 * nch;
#pragma unroll
  for (int d = 0; d < 16; ++d) {
    const float t = ss_wave_sum(acc[d]);
    if (lane == 0) out[d * nch + c] = t;
  }
}

// 5. (has_p) keep rho >= r*; (min_p > 0) chunk maxima of the kept probabilities. `norm`: p = e / z here.
// With `compact` and r* found by samp_topp_compact_kernel, the rounds did not run: r = r* and P still holds e.
__global__ __launch_bounds__(64) void samp_keep_kernel(SampArgs a, int has_p, int norm, int compact) {
  const int c = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  SW w = sw_of(a.work, a.V, a.nch, row);
  const int nch = a.nch;
  float pv[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    pv[i] = j < a.V ? w.P[j] : 0.f;
  }
  uint64_t r = 0;
  if (compact) {
    r = w.cres[0];
    norm = 1;
  } else if (has_p) {
    r = w.rr[kRounds - 1] | (uint64_t)topp_digit(w.tsum + ((kRounds - 1) & 1) * 16 * nch, nch, a.top_p);
  }
  const float z = norm ? seq_sum(w.etot, nch) : 1.f;
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    if (j < a.V) {
      float p = norm ? pv[i] / z : pv[i];
      const bool drop = has_p && !(rho_of(p, j) >= r);
      if (drop) p = 0.f;
      if (drop || norm) w.P[j] = p;
      m = fmaxf(m, p);
    }
  }
  m = ss_wave_max(m);
  if (lane == 0) w.cmax[c] = m;
}

// 6. min-p cutoff (has_minp) and the hierarchical totals of the final weights. `norm`: p = e / z here.
__global__ __launch_bounds__(64) void samp_total_kernel(SampArgs a, int has_minp, int norm) {
  const int c = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  SW w = sw_of(a.work, a.V, a.nch, row);
  float cutoff = 0.f;
  if (has_minp) {
    float pm = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < kPerLane; ++k)
      if (lane + 64 * k < a.nch) pm = fmaxf(pm, w.cmax[lane + 64 * k]);
    cutoff = ss_wave_max(pm) * a.min_p;
  }
  const float z = norm ? seq_sum(w.etot, a.nch) : 1.f;
  float v[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    v[i] = j < a.V ? w.P[j] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + lane * kSub + i;
    float p = norm ? v[i] / z : v[i];
    const bool drop = has_minp && p < cutoff;
    if (drop) p = 0.f;
    if (j < a.V && (drop || norm)) w.P[j] = p;
    v[i] = j < a.V ? p : 0.f;
  }
  float sub;
  const float t = chunk_sum(v, sub);
  w.stot[c * 64 + lane] = sub;
  if (lane == 0) w.ftot[c] = t;
}

// 7. the draw, one wave per row (every lane follows the same scan); greedy rows take the argmax.
__global__ __launch_bounds__(64) void samp_draw_kernel(SampArgs a) {
  const int row = blockIdx.x, lane = threadIdx.x;
  SW w = sw_of(a.work, a.V, a.nch, row);
  const int nch = a.nch;
  auto finish = [&](int tok, int fb, int nonfinite) {
    if (lane != 0) return;
    if (a.accept) {
      w.res[0] = tok;
      w.res[1] = fb;
      w.res[2] = nonfinite;
    } else {
      a.out[0] = tok;
      a.out[1] = fb;
    }
  };
  if (a.accept) {
    uint32_t b = 0;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k)
      if (lane + 64 * k < nch) b |= (uint32_t)w.cbad[lane + 64 * k];
    if (ss_wave_or(b)) {
      finish(-1, 0, 1);
      return;
    }
  }
  if (!(a.temperature > 0.f)) {
    const uint64_t k = max_u64_of(w.ckey, nch);
    finish((int)(0xFFFFFFFFu - (uint32_t)k), 0, 0);
    return;
  }
  const float* ct = stage(w.ftot, nch);  // zero-padded to a multiple of 16
  const float total = lds_seq_sum(ct, nch, 0.f);
  if (!is_finite(total) || !(total > 0.f)) {
    const uint64_t k = max_u64_of(w.craw, nch);
    finish((int)(0xFFFFFFFFu - (uint32_t)k), 1, 0);
    return;
  }
  const float u = a.u[row];
  const bool ge = u != 0.f;
  const float target = ge ? u * total : 0.f;
  auto hit = [&](float x) { return ge ? x >= target : x > target; };
  // The first chunk whose running total hits the target is the count of leading misses: the zero padding adds +0
  // and, following a miss with the same total, cannot be the first hit, so no bound check runs per entry.
  int lead = 0, clast = -1;
  bool alive = true;
  float base = 0.f, run = 0.f;
  const float4* c4 = reinterpret_cast<const float4*>(ct);
  for (int q0 = 0; q0 < nch; q0 += 16) {  // 16 unconditional reads (the padding is zero), then the in-order scan
    const float4 a0 = c4[q0 / 4], a1 = c4[q0 / 4 + 1], a2 = c4[q0 / 4 + 2], a3 = c4[q0 / 4 + 3];
    const float t[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                         a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float nx = run + t[i];
      alive = alive && !hit(nx);
      base = alive ? nx : base;
      lead += alive ? 1 : 0;
      clast = t[i] > 0.f ? q0 + i : clast;
      run = nx;
    }
  }
  int cs = lead < nch ? lead : -1;
  if (cs < 0) {
    cs = clast < 0 ? 0 : clast;
    base = lds_seq_sum(ct, cs, 0.f);
  }
  const float st = w.stot[cs * 64 + lane];
  int slead = 0, blast = -1;
  float sbase = base;
  run = base;
  alive = true;
#pragma unroll 16
  for (int b = 0; b < 64; ++b) {
    const float t = ss_readlane_f(st, b);
    const float nx = run + t;
    blast = t > 0.f ? b : blast;
    alive = alive && !hit(nx);
    sbase = alive ? nx : sbase;
    slead += alive ? 1 : 0;
    run = nx;
  }
  int bs = slead < 64 ? slead : -1;
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
  finish(pick, 0, 0);
}

// 8. accept mode: the round, walking the rows in order (n_accept, n_emit, n_uniform, flags, tokens).
__global__ __launch_bounds__(64) void samp_decide_kernel(SampArgs a) {
  if (threadIdx.x != 0) return;
  const int D = a.R - 1;
  int na = 0, ne = 0, nu = 0, fl = 0;
  for (int i = 0; i <= D; ++i) {
    const SW w = sw_of(a.work, a.V, a.nch, i);
    if (w.res[2]) {
      fl |= kFlagNonfinite;
      break;
    }
    const int tok = w.res[0];
    a.out[4 + i] = tok;
    ne = i + 1;
    if (a.temperature > 0.f) nu = i + 1;
    if (w.res[1]) fl |= kFlagFallback;
    if (i == D) break;
    const int d = a.drafts[i];
    if (d < 0 || d >= a.V) fl |= kFlagBadDraft;
    if (tok != d) break;
    na = i + 1;
  }
  for (int i = ne; i <= D; ++i) a.out[4 + i] = -1;
  a.out[0] = na;
  a.out[1] = ne;
  a.out[2] = nu;
  a.out[3] = fl;
}

namespace {

SampArgs args_of(int V, int R, const int32_t* gen, int n_gen, float temperature, float top_p, int top_k,
                 float min_p, float pp, void* work) {
  SampArgs a{};
  a.V = V;
  a.nch = (V + kChunk - 1) / kChunk;
  a.R = R;
  a.gen = gen;
  a.n_gen = n_gen;
  a.temperature = temperature;
  a.top_p = top_p;
  a.top_k = top_k;
  a.min_p = min_p;
  a.pp = pp;
  a.work = work;
  return a;
}

size_t topp_lds_bytes(int nch) { return (size_t)16 * ((nch + 15) & ~15) * sizeof(float); }

// The rows' launch sequence; which kernels run depends only on the parameters.
void launch_rows(const SampArgs& a, hipStream_t st) {
  const dim3 g(a.nch, a.R), b(64);
  if (!(a.temperature > 0.f)) {
    hipLaunchKernelGGL(samp_prep_kernel, g, b, 0, st, a, 0);
    hipLaunchKernelGGL(samp_draw_kernel, dim3(a.R), b, 0, st, a);
    return;
  }
  const int has_k = a.top_k > 0 && a.top_k < a.V;
  const int has_p = a.top_p < 1.f;
  const int has_minp = a.min_p > 0.f;
  if (has_k) hipLaunchKernelGGL(samp_begin_kernel, dim3(a.R), dim3(256), 0, st, a);
  hipLaunchKernelGGL(samp_prep_kernel, g, b, 0, st, a, has_k);
  if (has_k)
    for (int pass = 1; pass < 4; ++pass) hipLaunchKernelGGL(samp_hist_kernel, g, b, 0, st, a, pass);
  hipLaunchKernelGGL(samp_exp_kernel, g, b, 0, st, a, has_k);
  // top-k rows (k <= kCompact): one workgroup per row finds r* (from the survivors, or by the radix rounds in the
  // workgroup when a row has more); otherwise the 13 rounds run as launches
  const int compact = has_k && has_p && a.top_k <= kCompact && a.nch <= kCompactChunks * 4;
  if (compact) hipLaunchKernelGGL(samp_topp_compact_kernel, dim3(a.R), dim3(256), 0, st, a);
  else if (has_p)
    for (int round = 0; round < kRounds; ++round)
      hipLaunchKernelGGL(samp_topp_kernel, g, b, topp_lds_bytes(a.nch), st, a, round, 0);
  if (has_p || has_minp)
    hipLaunchKernelGGL(samp_keep_kernel, g, b, has_p ? topp_lds_bytes(a.nch) : 0, st, a, has_p, has_p ? 0 : 1,
                       compact);
  hipLaunchKernelGGL(samp_total_kernel, g, b, 0, st, a, has_minp, (has_p || has_minp) ? 0 : 1);
  hipLaunchKernelGGL(samp_draw_kernel, dim3(a.R), b, 0, st, a);
}

}  // namespace

int64_t sample_workspace_bytes(int V) {
  const int nch = (V + kChunk - 1) / kChunk;
  return (int64_t)layout_of(V, nch).bytes;
}

hipError_t launch_sample(const float* x, int V, const int32_t* gen, int n_gen, float temperature, float top_p,
                         int top_k, float min_p, float pp, const float* u, void* work, int32_t* out, hipStream_t st) {
  SampArgs a = args_of(V, 1, gen, n_gen, temperature, top_p, top_k, min_p, pp, work);
  a.x = x;
  a.u = u;
  a.out = out;
  launch_rows(a, st);
  return hipGetLastError();
}

hipError_t launch_accept_sampled(const float* target, const int32_t* drafts, int D, int V, const int32_t* seen,
                                 int n_seen, float temperature, float top_p, int top_k, float min_p, float pp,
                                 const float* uniforms, void* work, int32_t* out, hipStream_t st) {
  SampArgs a = args_of(V, D + 1, seen, n_seen, temperature, top_p, top_k, min_p, pp, work);
  a.x = target;
  a.u = uniforms;
  a.drafts = drafts;
  a.out = out;
  a.accept = 1;
  launch_rows(a, st);
  hipLaunchKernelGGL(samp_decide_kernel, dim3(1), dim3(64), 0, st, a);
  return hipGetLastError();
}

}  // namespace ss
