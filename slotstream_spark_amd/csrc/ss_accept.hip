// Acceptance of one MTP verify round over the vocabulary.
//
// Greedy (engine/generate.py:208-229 with engine/sampler.py:83-84): t_i = argmax(target[i]) (first maximum);
// the round accepts drafts while t_i == draft_i and emits t_0 .. t_good. A row with a non-finite logit stops
// the round before it (generate.py:210-212).
//
// p/q (Leviathan et al. 2023, Alg. 1; not in the reference): p_i = softmax(target_i / T), q_i = softmax(draft_i / T);
// draft x_i is accepted iff u_i * q_i(x_i) < p_i(x_i). The first rejection samples from norm(max(0, p_i - q_i))
// with the next uniform; when every draft is accepted a bonus token is sampled from p_D.
//
// Every reduction has a fixed order, which the CPU restatement replays bit for bit:
//   chunk = 1024 entries = 64 sub-chunks of 16; a sub-chunk total is the sequential fp32 sum of its entries
//   (from 0); a chunk total is the xor-butterfly sum of its 64 sub-chunk totals; a row total is the sequential
//   sum of the chunk totals. Inverse-CDF search: the first chunk whose running total exceeds u*S, then inside
//   it the first sub-chunk (running total started at the chunk's base), then the first entry.
#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

constexpr int kSub = 16;
constexpr int kChunk = 64 * kSub;
constexpr int kMaxRows = 128;        // 2 D + 1 <= 121
constexpr int kArrShards = 32;       // arrival counters: shards of one counter, 128 bytes apart
constexpr int kArrStride = 32;       // ints
constexpr int kArrCounters = 3;      // greedy, p/q sums, p/q residual
constexpr int kHeadFloats = 4096;  // 16 KB: kArrCounters x (kArrShards + 1) x kArrStride ints and spare
static_assert(kArrCounters * (kArrShards + 1) * kArrStride <= kHeadFloats, "header");

// Output header: out[0] n_accept, out[1] n_emit, out[2] uniforms used, out[3] flags, out[4..] tokens.
enum { OUT_NACC = 0, OUT_NEMIT = 1, OUT_NUNI = 2, OUT_FLAGS = 3, OUT_TOK = 4 };
enum { FLAG_NONFINITE = 1, FLAG_BAD_DRAFT = 2, FLAG_RESIDUAL_EMPTY = 4 };

SS_DEV int nchunks_of(int V) { return (V + kChunk - 1) / kChunk; }

int64_t accept_work_floats(int D, int V) {
  const int nch = (V + kChunk - 1) / kChunk;
  const int rows = 2 * D + 1;
  return kHeadFloats + (int64_t)rows * nch * 3 + (int64_t)nch * 65 + 64;
}

// Workspace layout (floats). The header holds the arrival counters of the launches whose last workgroup finishes
// the round; it must be zero before the first call, and every launch sequence leaves it zero.
struct Work {
  int* ctr;         // arrival counters (header)
  float* cmax;      // [rows][nch] chunk maxima (greedy: the maximum's value)
  float* cbad;      // [rows][nch] chunk holds a non-finite value
  float* ctot;      // [rows][nch] chunk totals (greedy: the maximum's index)
  float* stot;      // [nch][64]  sub-chunk totals of the sampled row
  float* rtot;      // [nch]      chunk totals of the sampled row
  float* state;     // [64]
};

SS_DEV Work work_of(float* w, int rows, int nch) {
  Work k;
  k.ctr = reinterpret_cast<int*>(w);
  float* b = w + kHeadFloats;
  k.cmax = b;
  k.cbad = b + (size_t)rows * nch;
  k.ctot = b + (size_t)rows * nch * 2;
  k.stot = b + (size_t)rows * nch * 3;
  k.rtot = k.stot + (size_t)nch * 64;
  k.state = k.rtot + nch;
  return k;
}

template <class T>
SS_DEV void st_ag(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
SS_DEV T ld_ag(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One-wave workgroups: true (in every lane) for the workgroup that arrives last of `total` at counter c. Arrivals
// are counted on up to 32 shards (workgroup `id` on shard id % shards, each shard on its own 128-byte line), and the
// workgroup completing a shard counts on the top counter, so no address takes more than total / 32 + 32 atomics.
// The wave's agent-scope stores are performed before its arrival is counted, and the last workgroup issues its
// agent-scope loads only after it has seen the count, so it reads every other workgroup's results. The last
// workgroup clears the counter (arrival_clear).
SS_DEV int* arrival_ctr(int* ctr, int c, int s) { return ctr + (c * (kArrShards + 1) + s) * kArrStride; }
SS_DEV bool arrive_last(int* ctr, int c, int id, int total) {
  __builtin_amdgcn_s_waitcnt(0);
  int last = 0;
  if ((threadIdx.x & 63) == 0) {
    const int shards = total < kArrShards ? total : kArrShards;
    const int sh = id % shards;
    const int n_sh = total / shards + (sh < total % shards ? 1 : 0);
    if (__hip_atomic_fetch_add(arrival_ctr(ctr, c, sh), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_sh - 1)
      last = __hip_atomic_fetch_add(arrival_ctr(ctr, c, kArrShards), 1, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == shards - 1;
  }
  return __builtin_amdgcn_readfirstlane(last) != 0;
}
SS_DEV void arrival_clear(int* ctr, int c) {
  const int lane = threadIdx.x & 63;
  if (lane <= kArrShards) __hip_atomic_store(arrival_ctr(ctr, c, lane), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

SS_DEV bool finite(float v) { return (__float_as_uint(v) & 0x7F800000u) != 0x7F800000u; }

// Chunk-array entries per lane when one wave loads an array of per-chunk values (lane c % 64, register c / 64).
constexpr int kMaxPerLane = 16;  // V <= 16 * 64 * 1024 entries

// Sequential sums and scans over LDS arrays that are 16-byte aligned and padded with zeros to a multiple of 16
// entries: every 16 entries are read as four unconditional 16-byte loads before their (dependent, in-order) adds,
// and the bound n is applied by selects in the last, partial group.
SS_DEV float lds_seq_sum(const float* v, int n, float s) {
  // whole groups of 16 add without a bound check; only the last, partial group selects
  const float4* v4 = reinterpret_cast<const float4*>(v);
  for (int b = 0; b < n; b += 16) {
    const float4 a0 = v4[b / 4], a1 = v4[b / 4 + 1], a2 = v4[b / 4 + 2], a3 = v4[b / 4 + 3];
    const float t[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                         a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
    if (b + 16 <= n) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s = s + t[i];
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float nx = s + t[i];
        s = b + i < n ? nx : s;
      }
    }
  }
  return s;
}
// Running sum from `start` over v[0..n): the first index whose running sum exceeds `target` (and the running sum
// before it; `start` when there is none), and the last nonzero index. The zero padding adds +0 to the running sum
// and, coming after a miss with the same sum, cannot be the first hit, so no bound check runs per entry: the first
// hit is the count of leading misses.
struct Scan {
  int first, last;
  float base;
};
SS_DEV Scan lds_scan(const float* v, int n, float start, float target) {
  float run = start, base = start;
  int lead = 0, last = -1;
  bool alive = true;
  const float4* v4 = reinterpret_cast<const float4*>(v);
  for (int b = 0; b < n; b += 16) {
    const float4 a0 = v4[b / 4], a1 = v4[b / 4 + 1], a2 = v4[b / 4 + 2], a3 = v4[b / 4 + 3];
    const float t[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                         a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // selects only: every lane holds the same values
      const float nx = run + t[i];
      alive = alive && !(nx > target);
      base = alive ? nx : base;
      lead += alive ? 1 : 0;
      last = t[i] > 0.f ? b + i : last;
      run = nx;
    }
  }
  Scan r;
  r.first = lead < n ? lead : -1;
  r.base = r.first >= 0 ? base : start;
  r.last = last;
  return r;
}

// Stages the same rows of three arrays (as stage_rows_ag) with every load of a batch (Q per lane and array) in
// flight before any store.
template <int Q>
SS_DEV void stage_rows3_ag(const float* s0, const float* s1, const float* s2, int nr, int nch, int nchp, float* d0,
                           float* d1, float* d2) {
  const int lane = threadIdx.x & 63;
  const int n = nr * nch;
  for (int i = lane; i < nr * nchp; i += 64) d0[i] = d1[i] = d2[i] = 0.f;
  for (int b = 0; b < n; b += 64 * Q) {
    float v0[Q], v1[Q], v2[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int i = b + lane + 64 * q;
      const bool in = i < n;
      v0[q] = in ? __hip_atomic_load(const_cast<float*>(s0) + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
      v1[q] = in ? __hip_atomic_load(const_cast<float*>(s1) + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
      v2[q] = in ? __hip_atomic_load(const_cast<float*>(s2) + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
    }
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int i = b + lane + 64 * q;
      if (i < n) {
        const int r = i / nch, o = r * nchp + (i - r * nch);
        d0[o] = v0[q];
        d1[o] = v1[q];
        d2[o] = v2[q];
      }
    }
  }
}

// Stages rows [nr][nch] written by other workgroups (agent-scope loads, 32 per lane in flight) into LDS at a row
// stride of nchp = nch rounded up to 16, the padding zeroed.
SS_DEV void stage_rows_ag(const float* src, int nr, int nch, int nchp, float* lds) {
  const int lane = threadIdx.x & 63;
  const int n = nr * nch;
  for (int i = lane; i < nr * nchp; i += 64) lds[i] = 0.f;
  for (int b = 0; b < n; b += 64 * 32) {
    float v[32];
#pragma unroll
    for (int q = 0; q < 32; ++q) {
      const int i = b + lane + 64 * q;
      v[q] = i < n ? __hip_atomic_load(const_cast<float*>(src) + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
    }
#pragma unroll
    for (int q = 0; q < 32; ++q) {
      const int i = b + lane + 64 * q;
      if (i < n) {
        const int r = i / nch;
        lds[r * nchp + (i - r * nch)] = v[q];
      }
    }
  }
}

// ---------------------------------------------------------------- greedy
// One launch: every (chunk, row) workgroup reduces its chunk to its first maximum and a non-finite flag; the last
// workgroup to arrive reduces the chunks of every row (order-free: the largest (value key, complemented index)),
// decides the round and clears its counter. The order-preserving value key counts +-0 as equal (as np.argmax
// compares); the complemented index makes the first maximum win.
constexpr int kStage = 2048;  // chunk results staged per batch of rows by a finishing workgroup

__global__ __launch_bounds__(64) void greedy_kernel(AcceptArgs a) {
  __shared__ float sv[kStage], si[kStage], sb[kStage];
  __shared__ int s_tok[kMaxRows], s_bad[kMaxRows];
  const int row = blockIdx.y, c = blockIdx.x, lane = threadIdx.x;
  const int nch = gridDim.x, rows = gridDim.y;
  Work k = work_of(a.work, rows, nch);
  {
    const float* x = a.target + (size_t)row * a.V;
    float v[kSub];
#pragma unroll
    for (int i = 0; i < kSub; ++i) {
      const int j = c * kChunk + i * 64 + lane;
      v[i] = j < a.V ? x[j] : 0.f;
    }
    uint64_t bk = 0;
    uint32_t bad = 0;
#pragma unroll
    for (int i = 0; i < kSub; ++i) {
      const int j = c * kChunk + i * 64 + lane;
      if (j < a.V) {
        bad |= !finite(v[i]);
        const uint64_t kv = ((uint64_t)ss_key(v[i] == 0.f ? 0.f : v[i]) << 32) | (0xFFFFFFFFu - (uint32_t)j);
        bk = kv > bk ? kv : bk;
      }
    }
    bk = ss_wave_max_u64(bk);
    bad = ss_wave_or(bad);
    if (lane == 0) {
      const size_t o = (size_t)row * nch + c;
      st_ag(k.cmax + o, ss_unkey((uint32_t)(bk >> 32)));
      st_ag(k.ctot + o, __int_as_float((int)(0xFFFFFFFFu - (uint32_t)bk)));
      st_ag(k.cbad + o, bad ? 1.f : 0.f);
    }
  }
  // The drafts (lane i holds draft i; D <= 60) arrive with this workgroup's own loads rather than after the reduction.
  const int dr = lane < a.D ? a.drafts[lane] : 0;
  if (!arrive_last(k.ctr, 0, row * nch + c, nch * rows)) return;
  arrival_clear(k.ctr, 0);
  const int per = kStage / nch;
  for (int r0 = 0; r0 < rows; r0 += per) {
    const int nr = rows - r0 < per ? rows - r0 : per;
    const size_t o = (size_t)r0 * nch;
    stage_rows3_ag<16>(k.cmax + o, k.ctot + o, k.cbad + o, nr, nch, nch, sv, si, sb);
    __syncthreads();
    for (int rr = 0; rr < nr; ++rr) {
      uint64_t bk = 0;
      uint32_t b = 0;
      for (int cc = lane; cc < nch; cc += 64) {
        const float v = sv[rr * nch + cc];
        const int ix = __float_as_int(si[rr * nch + cc]);
        b |= sb[rr * nch + cc] != 0.f ? 1u : 0u;
        const uint64_t kv = ((uint64_t)ss_key(v == 0.f ? 0.f : v) << 32) | (0xFFFFFFFFu - (uint32_t)ix);
        bk = kv > bk ? kv : bk;
      }
      bk = ss_wave_max_u64(bk);
      b = ss_wave_or(b);
      if (lane == 0) {
        s_tok[r0 + rr] = (int)(0xFFFFFFFFu - (uint32_t)bk);
        s_bad[r0 + rr] = (int)b;
      }
    }
    __syncthreads();
  }
  __shared__ int s_dr[64];
  if (lane < a.D) s_dr[lane] = dr;
  __syncthreads();
  if (lane == 0) {
    const int D = a.D;
    int good = 0, emit = 0, flags = 0;
    for (int i = 0; i <= D; ++i) {
      if (s_bad[i]) {
        flags |= FLAG_NONFINITE;
        break;
      }
      const int t = s_tok[i];
      a.out[OUT_TOK + emit++] = t;
      if (i < D && t == s_dr[i]) {
        ++good;
        continue;
      }
      break;
    }
    for (int i = emit; i <= D; ++i) a.out[OUT_TOK + i] = -1;
    a.out[OUT_NACC] = good;
    a.out[OUT_NEMIT] = emit;
    a.out[OUT_NUNI] = 0;
    a.out[OUT_FLAGS] = flags;
  }
}

hipError_t launch_accept_greedy(const AcceptArgs& a, hipStream_t st) {
  const int nch = (a.V + kChunk - 1) / kChunk;
  hipLaunchKernelGGL(greedy_kernel, dim3(nch, a.D + 1), dim3(64), 0, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------- p/q
// Three launches: (1) chunk maxima of l / T and non-finite flags; (2) e = exp(l / T - m) chunk totals, then the
// last workgroup forms each row's total (sequential over its chunk totals), maximum and flag and decides the
// drafts; (3) the chunk and sub-chunk totals of the sampled distribution, then the last workgroup searches them and
// writes the round. Logical rows: target i -> i (0..D), draft i -> D + 1 + i.
SS_DEV const float* row_ptr(const AcceptArgs& a, int row) {
  return row <= a.D ? a.target + (size_t)row * a.V : a.draft + (size_t)(row - a.D - 1) * a.V;
}

__global__ __launch_bounds__(64) void pq_max_kernel(AcceptArgs a) {
  const int row = blockIdx.y, c = blockIdx.x, lane = threadIdx.x;
  const int nch = gridDim.x, rows = gridDim.y;
  Work k = work_of(a.work, rows, nch);
  if (a.tkey && row <= a.D) {
    // formed by the lm_head GEMV: the same maximum (order-free), key 0 = a chunk of NaNs only (fmaxf's -inf)
    if (lane == 0) {
      const uint32_t key = a.tkey[row * nch + c];
      k.cmax[row * nch + c] = key ? ss_unkey(key) : -__builtin_inff();
      k.cbad[row * nch + c] = a.tbad[row * nch + c] ? 1.f : 0.f;
    }
    return;
  }
  const float* x = row_ptr(a, row);
  float v[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + i * 64 + lane;
    v[i] = j < a.V ? x[j] : 0.f;
  }
  float m = -__builtin_inff();
  int bad = 0;
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + i * 64 + lane;
    if (j < a.V) {
      bad |= !finite(v[i]);
      m = fmaxf(m, v[i] / a.temperature);
    }
  }
  m = ss_wave_max(m);
  bad = (int)ss_wave_or((uint32_t)bad);
  if (lane == 0) {
    k.cmax[row * nch + c] = m;
    k.cbad[row * nch + c] = bad ? 1.f : 0.f;
  }
}

__global__ __launch_bounds__(256) void pq_sum_kernel(AcceptArgs a) {
  __shared__ float lds[64 * (kSub + 1)];
  __shared__ __attribute__((aligned(16))) float sv[kStage], sm[kStage], sb[kStage];
  __shared__ float zrow[kMaxRows], mrow[kMaxRows];
  __shared__ int brow[kMaxRows];
  __shared__ float s_m;
  const int row = blockIdx.y, c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nch = gridDim.x, rows = gridDim.y;
  Work k = work_of(a.work, rows, nch);
  {
    // wave 0: the row maximum over the chunk maxima (order-free); all waves: a quarter of the chunk each
    const float* x = row_ptr(a, row);
    constexpr int NQ = kSub / 4;
    float xv[NQ];
#pragma unroll
    for (int ii = 0; ii < NQ; ++ii) {
      const int j = c * kChunk + (w * NQ + ii) * 64 + lane;
      xv[ii] = j < a.V ? x[j] : 0.f;
    }
    if (w == 0) {
      float cm[kMaxPerLane];
#pragma unroll
      for (int q = 0; q < kMaxPerLane; ++q) {
        const int cc = lane + 64 * q;
        cm[q] = cc < nch ? k.cmax[row * nch + cc] : -__builtin_inff();
      }
      float m = -__builtin_inff();
#pragma unroll
      for (int q = 0; q < kMaxPerLane; ++q) m = fmaxf(m, cm[q]);
      m = ss_wave_max(m);
      if (lane == 0) s_m = m;
    }
    __syncthreads();
    const float m = s_m;
    // e = exp(l/T - m) staged with a 17-float stride per sub-chunk of 16
#pragma unroll
    for (int ii = 0; ii < NQ; ++ii) {
      const int e = (w * NQ + ii) * 64 + lane;
      const int j = c * kChunk + e;
      lds[(e >> 4) * (kSub + 1) + (e & (kSub - 1))] = j < a.V ? ss_expf(xv[ii] / a.temperature - m) : 0.f;
    }
    __syncthreads();
    if (w != 0) return;
    float s = 0.f;
    for (int i = 0; i < kSub; ++i) s = s + lds[lane * (kSub + 1) + i];
    s = ss_wave_sum(s);
    if (lane == 0) st_ag(k.ctot + (size_t)row * nch + c, s);
  }
  // The drafts (lane i holds draft i; D <= 60) arrive with this workgroup's own loads, so the finishing workgroup
  // requests the draft positions' logits and the uniforms together with its staging.
  const int xi = lane < a.D ? a.drafts[lane] : 0;
  if (!arrive_last(k.ctr, 1, row * nch + c, nch * rows)) return;
  arrival_clear(k.ctr, 1);
  const bool xok = lane < a.D && xi >= 0 && xi < a.V;
  const float lt = xok ? a.target[(size_t)lane * a.V + xi] : 0.f;
  const float lq = xok ? a.draft[(size_t)lane * a.V + xi] : 0.f;
  const float uu = lane < a.D ? a.uniforms[lane] : 0.f;
  // Per row: the total (sequential over its chunk totals, from 0), the maximum and the non-finite flag.
  const int nchp = (nch + 15) & ~15;
  const int per = kStage / nchp;
  for (int r0 = 0; r0 < rows; r0 += per) {
    const int nr = rows - r0 < per ? rows - r0 : per;
    const size_t o = (size_t)r0 * nch;
    // 17 per lane: one batch for the seven rows of a depth-3 round at V = 151,936 (1,043 chunks), and 88 VGPRs,
    // which keep five workgroups per CU (as the LDS does)
    stage_rows3_ag<17>(k.ctot + o, k.cmax + o, k.cbad + o, nr, nch, nchp, sv, sm, sb);
    __syncthreads();
    // the maximum and flag of each row across the wave (order-free: a +-0 difference in m changes no exp(x - m));
    // the totals, which keep their order, lane r taking row r
    for (int rr = 0; rr < nr; ++rr) {
      float m = -__builtin_inff(), b = 0.f;
      for (int cc = lane; cc < nch; cc += 64) {
        m = fmaxf(m, sm[rr * nchp + cc]);
        b = fmaxf(b, sb[rr * nchp + cc]);  // flags are 0 or 1
      }
      m = ss_wave_max(m);
      b = ss_wave_max(b);
      if (lane == 0) {
        mrow[r0 + rr] = m;
        brow[r0 + rr] = b != 0.f;
      }
    }
    for (int rr = lane; rr < nr; rr += 64) zrow[r0 + rr] = lds_seq_sum(sv + rr * nchp, nch, 0.f);
    __syncthreads();
  }
  // the drafts, the draft positions' logits and the uniforms
  __shared__ int s_x[64];
  __shared__ float s_lt[64], s_lq[64], s_u[64];
  if (lane < a.D) {
    s_x[lane] = xi;
    s_lt[lane] = lt;
    s_lq[lane] = lq;
    s_u[lane] = uu;
  }
  __syncthreads();
  if (lane == 0) {
    const int D = a.D;
    int good = 0, flags = 0, stop = 0;
    int srow = D, sdraft = -1;
    for (int i = 0; i < D; ++i) {
      const int dr = D + 1 + i;
      if (brow[i] || brow[dr]) {
        flags |= FLAG_NONFINITE;
        stop = 1;
        break;
      }
      const int x = s_x[i];
      if (x < 0 || x >= a.V) {
        flags |= FLAG_BAD_DRAFT;
        ss_raise(a.err, SS_ERR_TOKEN);
        srow = i;
        sdraft = dr;
        break;
      }
      const float p = ss_expf(s_lt[i] / a.temperature - mrow[i]) / zrow[i];
      const float q = ss_expf(s_lq[i] / a.temperature - mrow[dr]) / zrow[dr];
      if (s_u[i] * q < p) {
        ++good;
        continue;
      }
      srow = i;
      sdraft = dr;
      break;
    }
    if (!stop && sdraft < 0 && brow[D]) {
      flags |= FLAG_NONFINITE;
      stop = 1;
    }
    k.state[0] = __int_as_float(srow);
    k.state[1] = __int_as_float(sdraft);
    k.state[2] = __int_as_float(good + (sdraft >= 0 ? 1 : 0));
    k.state[3] = __int_as_float(stop);
    k.state[4] = __int_as_float(good);
    k.state[5] = __int_as_float(flags);
    k.state[6] = zrow[srow];
    k.state[7] = sdraft >= 0 ? zrow[sdraft] : 0.f;
    k.state[8] = mrow[srow];
    k.state[9] = sdraft >= 0 ? mrow[sdraft] : 0.f;
  }
}

// The round's state as the p/q sums launch left it, read with one batch of loads.
struct PqState {
  int srow, sdraft, uidx, stop, good, flags;
  float zs, zd, ms, md;
};
SS_DEV PqState pq_state(const float* st) {
  float v[10];
#pragma unroll
  for (int i = 0; i < 10; ++i) v[i] = st[i];
  PqState r;
  r.srow = __float_as_int(v[0]);
  r.sdraft = __float_as_int(v[1]);
  r.uidx = __float_as_int(v[2]);
  r.stop = __float_as_int(v[3]);
  r.good = __float_as_int(v[4]);
  r.flags = __float_as_int(v[5]);
  r.zs = v[6];
  r.zd = v[7];
  r.ms = v[8];
  r.md = v[9];
  return r;
}

// Value of entry j of the sampled distribution: p_j, or max(0, p_j - q_j) after a rejection.
SS_DEV float sample_value(const AcceptArgs& a, const PqState& st, int j) {
  const float p = ss_expf(a.target[(size_t)st.srow * a.V + j] / a.temperature - st.ms) / st.zs;
  if (st.sdraft < 0) return p;
  const float q = ss_expf(a.draft[(size_t)(st.sdraft - a.D - 1) * a.V + j] / a.temperature - st.md) / st.zd;
  const float d = p - q;
  return d > 0.f ? d : 0.f;
}

// Inverse-CDF search by the finishing workgroup. Every lane forms the same running sums (index order, from the
// chunk's base) from LDS broadcast reads: the chunk, then the sub-chunk, then the entry, each falling back to the
// last nonzero one.
SS_DEV void pq_search(const AcceptArgs& a, const Work& k, const PqState& st, int nch, float* srt) {
  __shared__ __attribute__((aligned(16))) float s_st[64];
  __shared__ float s_val[kSub];
  __shared__ int s_dr[64];
  const int lane = threadIdx.x;
  const int good = st.good;
  int flags = st.flags;
  const int stop = st.stop;
  const int uidx = st.uidx;
  // the accepted drafts, requested with the first loads rather than one round trip each at the end
  for (int i = lane; i < good; i += 64) s_dr[i] = a.drafts[i];
  int emit = good;
  int pick = -1;
  if (!stop) {
    const float u = a.uniforms[uidx];
    stage_rows_ag(k.rtot, 1, nch, (nch + 15) & ~15, srt);
    __syncthreads();
    const float S = lds_seq_sum(srt, nch, 0.f);
    if (!(S > 0.f)) flags |= FLAG_RESIDUAL_EMPTY;
    const float target = u * S;
    // chunk: the first whose running total exceeds the target (else the last nonzero one, based at its prefix)
    const Scan ch = lds_scan(srt, nch, 0.f, target);
    int cs = ch.first;
    float base = ch.base;
    if (cs < 0) {
      cs = ch.last < 0 ? 0 : ch.last;
      base = lds_seq_sum(srt, cs, 0.f);
    }
    __syncthreads();
    s_st[lane] = __hip_atomic_load(k.stot + cs * 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const Scan sc = lds_scan(s_st, 64, base, target);
    int bs = sc.first;
    float sbase = sc.base;
    if (bs < 0) {
      bs = sc.last < 0 ? 0 : sc.last;
      sbase = lds_seq_sum(s_st, bs, base);
    }
    const int j0 = cs * kChunk + bs * kSub;
    if (lane < kSub) s_val[lane] = j0 + lane < a.V ? sample_value(a, st, j0 + lane) : 0.f;
    __syncthreads();
    int last = -1;
    float run = sbase;
    for (int i = 0; i < kSub; ++i) {
      const int j = j0 + i;
      if (j >= a.V) break;
      const float v = s_val[i];
      if (v > 0.f) last = j;
      run = run + v;
      if (run > target) {
        pick = j;
        break;
      }
    }
    if (pick < 0) pick = last >= 0 ? last : min(j0, a.V - 1);
  }
  __syncthreads();
  if (lane == 0) {
    for (int i = 0; i < good; ++i) a.out[OUT_TOK + i] = s_dr[i];
    if (!stop) a.out[OUT_TOK + emit++] = pick;
    for (int i = emit; i <= a.D; ++i) a.out[OUT_TOK + i] = -1;
    a.out[OUT_NACC] = good;
    a.out[OUT_NEMIT] = emit;
    a.out[OUT_NUNI] = stop ? uidx : uidx + 1;
    a.out[OUT_FLAGS] = flags;
  }
}

// Four waves per chunk compute the sampled distribution's values (its divisions and exps are the chunk's latency);
// wave 0 then forms the sub-chunk and chunk totals and, in the last workgroup, runs the search.
__global__ __launch_bounds__(256) void pq_residual_kernel(AcceptArgs a) {
  __shared__ __attribute__((aligned(16))) float lds[kMaxPerLane * 64 + 64];
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nch = gridDim.x;
  Work k = work_of(a.work, 2 * a.D + 1, nch);
  const PqState st = pq_state(k.state);
  const bool run = !st.stop;
  if (run) {
#pragma unroll
    for (int ii = 0; ii < kSub / 4; ++ii) {
      const int e = (w * (kSub / 4) + ii) * 64 + lane;
      const int j = c * kChunk + e;
      lds[(e >> 4) * (kSub + 1) + (e & (kSub - 1))] = j < a.V ? sample_value(a, st, j) : 0.f;
    }
  }
  __syncthreads();
  if (w != 0) return;
  if (run) {
    float s = 0.f;
    for (int i = 0; i < kSub; ++i) s = s + lds[lane * (kSub + 1) + i];
    st_ag(k.stot + c * 64 + lane, s);
    s = ss_wave_sum(s);
    if (lane == 0) st_ag(k.rtot + c, s);
  }
  if (!arrive_last(k.ctr, 2, c, nch)) return;
  arrival_clear(k.ctr, 2);
  pq_search(a, k, st, nch, lds);
}

hipError_t launch_accept_pq(const AcceptArgs& a, hipStream_t st) {
  const int nch = (a.V + kChunk - 1) / kChunk;
  const int rows = 2 * a.D + 1;
  hipLaunchKernelGGL(pq_max_kernel, dim3(nch, rows), dim3(64), 0, st, a);
  hipLaunchKernelGGL(pq_sum_kernel, dim3(nch, rows), dim3(256), 0, st, a);
  hipLaunchKernelGGL(pq_residual_kernel, dim3(nch), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace ss
