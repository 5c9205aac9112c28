// Acceptance of one MTP verify round over the vocabulary.
//
// Greedy (engine/generate.py:208-229 with engine/sampler.py:83-84): t_i = argmax(target[i]) (first maximum);
// the round accepts drafts while t_i == draft_i and emits t_0 .. t_good. A row with a non-finite logit stops
// the round before it (generate.py:210-212).
//
// p/q (Leviathan et al. 2023, Alg. 1; not in the reference): p_i = softmax(target_i / T), q_i = softmax(draft_i / T);
// draft x_i is accepted iff u_i * q_i(x_i) < p_i(x_i). The first rejection samples from norm(max(0, p_i - q_i))
// with the next uniform; when every draft is accepted a bonus token is sampled from p_D. Its sums are in a
// lane-parallel fixed order, described with the p/q kernels below, which the CPU restatement replays bit for bit.
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
  return kHeadFloats + (int64_t)rows * nch * 7 + (int64_t)nch * 3 + 64;
}

// Workspace layout (floats). The header holds the arrival counters of the launches whose last workgroup finishes
// the round; it must be zero before the first call, and every launch sequence leaves it zero.
// The one-launch p/q round hands its chunk results over as 64-bit words tagged with the launch: the high half is
// the tag (bits 32-62; bit 63 of wd0 is the chunk's non-finite flag), the low half the float. The tag is the
// workspace's launch epoch + 1 (mod 2^31); the epoch (header int kEpochInt, never reset) is advanced once every
// workgroup has published, so words left by an earlier launch never match.
constexpr int kEpochInt = 3200;
static_assert(kArrCounters * (kArrShards + 1) * kArrStride <= kEpochInt && kEpochInt < kHeadFloats, "epoch word");
struct Work {
  int* ctr;         // arrival counters and the epoch (header)
  uint64_t* wd0;    // [rows][nch] tagged chunk maxima (one-launch round)
  uint64_t* wd1;    // [rows][nch] tagged chunk totals (one-launch round)
  uint64_t* wr;     // [nch]       tagged chunk totals of the sampled values (one-launch round)
  float* cmax;      // [rows][nch] chunk maxima (greedy: the maximum's value)
  float* cbad;      // [rows][nch] chunk holds a non-finite value
  float* ctot;      // [rows][nch] chunk totals (greedy: the maximum's index)
  float* rtot;      // [nch]       chunk totals of the sampled values
  float* state;     // [64]
};

SS_DEV Work work_of(float* w, int rows, int nch) {
  Work k;
  k.ctr = reinterpret_cast<int*>(w);
  float* b = w + kHeadFloats;  // 16 KB into the 256-byte aligned workspace: 8-byte aligned
  k.wd0 = reinterpret_cast<uint64_t*>(b);
  k.wd1 = k.wd0 + (size_t)rows * nch;
  k.wr = k.wd1 + (size_t)rows * nch;
  float* f = reinterpret_cast<float*>(k.wr + nch);
  k.cmax = f;
  k.cbad = f + (size_t)rows * nch;
  k.ctot = f + (size_t)rows * nch * 2;
  k.rtot = f + (size_t)rows * nch * 3;
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

// Stages rows [nr][nch] of three arrays written by other workgroups (agent-scope loads, every load of a batch, Q per
// lane and array, in flight before any store) into LDS at a row stride of nchp (nch rounded up to 16).
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


// ---------------------------------------------------------------- p/q
// Leviathan et al. 2023, Alg. 1 (no reference counterpart), with every sum in a lane-parallel fixed order that the
// CPU restatement (or_accept_pq) replays bit for bit:
//   wave_scan: the inclusive prefix of one nonnegative value per lane: Hillis-Steele steps d = 1, 2, 4, 8 inside each
//   row of 16 lanes (R), then rows 1 and 3 add the last lane of the row before (R_15, R_47), then rows 2 and 3 add
//   lane 31's value of that step (R_31 + R_15); every addition is (own + other).
//   lane layout of n values, k per lane: lane l holds values k l .. k l + k - 1; its local sum is sequential from 0;
//   the layout's total is the last lane's prefix.
// Per row and 1024-entry chunk c (lane l: entries 16 l .. 16 l + 15): y = x * (1 / T), m_c = max y, e = exp(y - m_c),
// s_c = the layout total of e (k = 16). Per row: M = max m_c, g_c = exp(m_c - M), Z = the layout total of s_c g_c
// (k = ceil(nch / 64)), a_c = g_c / Z, p_j = e_j a_c. Draft x_i is accepted iff u_i q_i(x_i) < p_i(x_i); the first
// rejection samples from max(0, p_i - q_i), every draft accepted from p_D: wave_descend over the chunk totals of the
// sampled values, then over the chosen chunk's entries. A non-finite row the round reaches stops it.
// Logical rows: target i -> i (0..D), draft i -> D + 1 + i.
//
// Two forms, the same bits: pq_round_kernel, one persistent launch, when every unit (target row i with draft row i,
// or the bonus target row D, over one chunk) has a wave of a resident grid: the unit's e values stay in registers;
// the chunk parts are published as tagged words, which every workgroup polls directly (no counter) before it forms
// the row statistics and the decision itself; after a rejection the waves of the sampled row form its values and
// publish their chunk totals the same way, every such wave finds the chunk of the sample and the wave holding it
// finds the entry; with every draft accepted the bonus row is sampled as the proposal draw samples (chunk by its mass
// s_c a_c, entry by e against (t - base) / a_c), with no second hand-off. Otherwise two launches: pq_sum_kernel
// (chunk parts; the last workgroup decides) and pq_residual_kernel (chunk totals of the sampled values; the last
// workgroup searches).

// DPP (GFX9 encodings): row_shr:d = 0x110 + d reads lane l - d of the same row (0 past the row's start, bound_ctrl);
// row_bcast:15 = 0x142 gives rows 1 and 3 (row_mask 0xA) lane 15 / 47; row_bcast:31 = 0x143 gives rows 2 and 3
// (row_mask 0xC) lane 31. Rows a step leaves out read 0, and v + 0 = v for v >= +0. VALU only, whole wave active.
template <int CTRL, int ROWS, bool BOUND>
SS_DEV float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, BOUND));
}
SS_DEV float wave_scan(float v) {
  v = v + dpp_f<0x111, 0xF, true>(v);
  v = v + dpp_f<0x112, 0xF, true>(v);
  v = v + dpp_f<0x114, 0xF, true>(v);
  v = v + dpp_f<0x118, 0xF, true>(v);
  v = v + dpp_f<0x142, 0xA, false>(v);
  v = v + dpp_f<0x143, 0xC, false>(v);
  return v;
}

// The layout total of v (k per lane, n values): every lane returns it.
template <int KMAX>
SS_DEV float wave_total(const float (&v)[KMAX], int k, int n) {
  const int lane = threadIdx.x & 63;
  float L = 0.f;
#pragma unroll
  for (int i = 0; i < KMAX; ++i)
    if (i < k && k * lane + i < n) L = L + v[i];
  return ss_readlane_f(wave_scan(L), 63);
}

// The search over a lane layout for target t (whole wave, uniform result): the first lane holding values whose
// prefix exceeds t (else the last lane with a nonzero local sum, else lane 0), then inside it the first value whose
// running sum from the lane's exclusive prefix exceeds t (else its last nonzero value, else its first); *base
// receives the running sum before the chosen value. Returns the value's index, at most n - 1.
template <int KMAX>
SS_DEV int wave_descend(const float (&v)[KMAX], int k, int n, float t, float* base) {
  const int lane = threadIdx.x & 63;
  float L = 0.f;
#pragma unroll
  for (int i = 0; i < KMAX; ++i)
    if (i < k && k * lane + i < n) L = L + v[i];
  const float P = wave_scan(L);
  const uint64_t gt = __ballot(P > t && k * lane < n);  // lanes holding values only
  int ls;
  if (gt) {
    ls = __builtin_ctzll(gt);
  } else {
    const uint64_t nz = __ballot(L > 0.f);
    ls = nz ? 63 - __builtin_clzll(nz) : 0;
  }
  const float e = ls > 0 ? ss_readlane_f(P, ls - 1) : 0.f;
  // Branch-free inside the lane: the running sums R_i = e + v_0 + .. + v_i (sequential; an entry past n adds
  // nothing), the first valid i with R_i > t, else the last valid nonzero value, else 0; the base is R before it.
  float R[KMAX];
  float run = e;
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    const bool in = i < k && k * lane + i < n;
    run = in ? run + v[i] : run;
    R[i] = run;
  }
  int pick = -1, last = -1;
#pragma unroll
  for (int i = KMAX - 1; i >= 0; --i) {
    const bool in = i < k && k * lane + i < n;
    pick = in && R[i] > t ? i : pick;
  }
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    const bool in = i < k && k * lane + i < n;
    last = in && v[i] > 0.f ? i : last;
  }
  pick = pick >= 0 ? pick : (last >= 0 ? last : 0);
  float bse = e;
#pragma unroll
  for (int i = 1; i < KMAX; ++i) bse = pick == i ? R[i - 1] : bse;
  const int pb = __builtin_amdgcn_readlane(pick, ls);
  *base = ss_readlane_f(bse, ls);
  const int idx = k * ls + pb;
  return idx < n ? idx : n - 1;
}

// One chunk of one row in a wave: lane l holds entries j0 .. j0 + 15 of v (j0 = 1024 c + 16 l; entries >= V
// excluded), which become e; returns m_c, s_c and the non-finite flag.
struct ChunkPart {
  float m, s;
  int bad;
};
SS_DEV ChunkPart chunk_part(float (&v)[kSub], int j0, int V, float invT) {
  float m = -__builtin_inff();
  uint32_t bad = 0;
  const int nv = V - j0;  // entries of this lane inside the row (every one in all but the last chunk)
#pragma unroll
  for (int e = 0; e < kSub; ++e) {
    const bool in = e < nv;
    bad |= in && (__float_as_uint(v[e]) & 0x7F800000u) == 0x7F800000u;
    v[e] = v[e] * invT;
    m = in ? fmaxf(m, v[e]) : m;
  }
  ChunkPart r;
  r.m = ss_wave_max(m);
  r.bad = (int)ss_wave_or(bad);
  float sub = 0.f;
#pragma unroll
  for (int e = 0; e < kSub; ++e) {
    v[e] = e < nv ? ss_expf_le0(v[e] - r.m) : 0.f;  // v - m <= 0 (NaN aside)
    sub = sub + v[e];
  }
  r.s = ss_readlane_f(wave_scan(sub), 63);
  return r;
}

// Statistics of NR rows (interleaved, so that their dependent chains overlap) from their staged chunk parts (LDS at
// row r: m at sm + r nchp, s at sv + r nchp, flags at sb + r nchp), one wave; rows r[q] with q >= nr are skipped.
// M, Z and the flag go to mrow, zrow, brow; sv receives a_c in place of s_c.
// KM: chunks per lane the code is built for (kc = ceil(nch / 64) <= KM; KM == kc lets every loop bound be constant).
template <int NR, int KM>
SS_DEV void rows_stats(float* sv, const float* sm, const float* sb, const int (&r)[NR], int nr, int nch, int nchp,
                       float* mrow, float* zrow, int* brow) {
  const int lane = threadIdx.x & 63, kc = KM < kMaxPerLane ? KM : (nch + 63) >> 6;
  float mv[NR][KM], g[NR][KM], m[NR], b[NR], L[NR];
#pragma unroll
  for (int q = 0; q < NR; ++q) {
    m[q] = -__builtin_inff();
    b[q] = 0.f;
    L[q] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < KM; ++i) {
    const int c = kc * lane + i;
    const bool in = i < kc && c < nch;  // i < kc: the same in every lane
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      const int o = (q < nr ? r[q] : 0) * nchp + c;
      mv[q][i] = in ? sm[o] : -__builtin_inff();
      if (in) {
        m[q] = fmaxf(m[q], mv[q][i]);
        b[q] = fmaxf(b[q], sb[o]);  // flags are 0 or 1
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NR; ++q) {
    m[q] = ss_wave_max(m[q]);
    b[q] = ss_wave_max(b[q]);
  }
#pragma unroll
  for (int i = 0; i < KM; ++i) {
    if (i < kc) {
      const int c = kc * lane + i;
#pragma unroll
      for (int q = 0; q < NR; ++q) {
        g[q][i] = ss_expf_le0(mv[q][i] - m[q]);  // m_c - M <= 0
        if (c < nch) L[q] = L[q] + sv[(q < nr ? r[q] : 0) * nchp + c] * g[q][i];
      }
    }
  }
  float z[NR];
#pragma unroll
  for (int q = 0; q < NR; ++q) z[q] = ss_readlane_f(wave_scan(L[q]), 63);
#pragma unroll
  for (int i = 0; i < KM; ++i) {
    const int c = kc * lane + i;
    if (i < kc && c < nch) {
#pragma unroll
      for (int q = 0; q < NR; ++q)
        if (q < nr) sv[r[q] * nchp + c] = g[q][i] / z[q];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < NR; ++q)
      if (q < nr) {
        mrow[r[q]] = m[q];
        zrow[r[q]] = z[q];
        brow[r[q]] = b[q] != 0.f;
      }
  }
}

// The round's decision, by one wave: lane i < D holds draft i's p_i(x_i), q_i(x_i) (exp(l x invT - m_c) a_c of
// target row i and draft row i at the draft's chunk: the values the sampled distribution would take there), its
// uniform, whether either row is non-finite and whether the draft is outside [0, V). The first draft that is not
// accepted ends the round: a non-finite row stops it, a draft outside [0, V) is flagged (and raised) and rejected,
// otherwise it is rejected; with every draft accepted, a non-finite row D stops it. Every lane returns the state.
struct PqState {
  int srow, sdraft, uidx, stop, good, flags;
  float ms, zs, md, zd;
};
SS_DEV float p_at(float l, float invT, float mc, float ac) { return ss_expf(l * invT - mc) * ac; }
SS_DEV PqState pq_decide(const AcceptArgs& a, bool bad_i, bool xbad_i, float p, float q, float u, const float* mrow,
                         const float* zrow, const int* brow, bool raise) {
  const int lane = threadIdx.x & 63, D = a.D;
  const bool acc = lane < D && !bad_i && !xbad_i && u * q < p;
  const uint64_t nacc = __ballot(lane < D && !acc);
  const int f = nacc ? __builtin_ctzll(nacc) : D;
  int flags = 0, stop = 0, srow = D, sdraft = -1;
  if (f < D) {
    const bool bf = __builtin_amdgcn_readlane((int)bad_i, f) != 0;
    const bool xf = __builtin_amdgcn_readlane((int)xbad_i, f) != 0;
    if (bf) {
      flags |= FLAG_NONFINITE;
      stop = 1;
    } else {
      if (xf) {
        flags |= FLAG_BAD_DRAFT;
        if (raise && lane == 0) ss_raise(a.err, SS_ERR_TOKEN);
      }
      srow = f;
      sdraft = D + 1 + f;
    }
  } else if (brow[D]) {
    flags |= FLAG_NONFINITE;
    stop = 1;
  }
  PqState st;
  st.srow = srow;
  st.sdraft = sdraft;
  st.good = f;
  st.uidx = f + (sdraft >= 0 ? 1 : 0);
  st.stop = stop;
  st.flags = flags;
  st.ms = mrow[srow];
  st.zs = zrow[srow];
  st.md = sdraft >= 0 ? mrow[sdraft] : 0.f;
  st.zd = sdraft >= 0 ? zrow[sdraft] : 1.f;
  return st;
}

// Per draft i (lane i of wave 0): the draft, the target and draft logits at it, and the uniform.
struct PqIn {
  int x[64];
  float lt[64], lq[64], u[64];
};

// Writes the round: the accepted drafts, then the sampled token unless the round stopped.
SS_DEV void pq_write_out(const AcceptArgs& a, const PqState& st, const int* drafts, int pick, int flags) {
  int emit = st.good;
  for (int i = 0; i < st.good; ++i) a.out[OUT_TOK + i] = drafts[i];
  if (!st.stop) a.out[OUT_TOK + emit++] = pick;
  for (int i = emit; i <= a.D; ++i) a.out[OUT_TOK + i] = -1;
  a.out[OUT_NACC] = st.good;
  a.out[OUT_NEMIT] = emit;
  a.out[OUT_NUNI] = st.stop ? st.uidx : st.uidx + 1;
  a.out[OUT_FLAGS] = flags;
}

// Lane l's 16 entries j0 .. j0 + 15 of row x (zeros past V), as four 16-byte loads when the row allows them.
SS_DEV void load16(const float* x, int j0, int V, bool vec, float (&v)[kSub]) {
  if (vec && j0 + kSub <= V) {
    const float4* p = reinterpret_cast<const float4*>(x + j0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 t = p[q];
      v[4 * q] = t.x;
      v[4 * q + 1] = t.y;
      v[4 * q + 2] = t.z;
      v[4 * q + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < kSub; ++e) v[e] = j0 + e < V ? x[j0 + e] : 0.f;
  }
}

// The sampled distribution's value from e of the target and draft rows and their a_c.
SS_DEV float sampled_value(float et, float ed, float at, float ad, bool rejected) {
  const float p = et * at;
  if (!rejected) return p;
  const float d = p - ed * ad;
  return d > 0.f ? d : 0.f;
}

// A tagged word's tag and value.
SS_DEV uint32_t tag_of(uint64_t w) { return (uint32_t)(w >> 32) & 0x7FFFFFFFu; }
SS_DEV float val_of(uint64_t w) { return __uint_as_float((uint32_t)w); }
SS_DEV uint64_t tagged(uint32_t tag, float v) { return ((uint64_t)tag << 32) | __float_as_uint(v); }
constexpr int kSpin = 1 << 22;  // bound of every wait for tagged words (then SS_ERR_TIMEOUT and on)

// ---------------------------------------------------------------- greedy, one launch
// Used when every (row, chunk) unit has a wave of a resident grid: each wave forms its chunk's first maximum (the
// greedy_kernel key: order key of the value, +-0 equal, then the complemented index) and non-finite flag and
// publishes them as two tagged words; workgroup 0 polls them, reduces each row (order-free), decides and writes the
// round. No counter and no arrival: the epoch is advanced by workgroup 0 once every word has been seen.
__global__ __launch_bounds__(256) void greedy_round_kernel(AcceptArgs a, int units) {
  __shared__ uint32_t s_epoch;
  __shared__ int s_tok[kMaxRows], s_bad[kMaxRows];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int D = a.D, V = a.V, nch = nchunks_of(V), rows = D + 1;
  Work k = work_of(a.work, 2 * D + 1, nch);
  const int gw = blockIdx.x * 4 + w;
  const bool has = gw < units;
  const int row = has ? gw / nch : 0, c = has ? gw - row * nch : 0;
  const int j0 = c * kChunk + kSub * lane;
  const bool vec = (V & 3) == 0 && (reinterpret_cast<uintptr_t>(a.target) & 15) == 0;
  float v[kSub];
  if (has) load16(a.target + (size_t)row * V, j0, V, vec, v);
  // the drafts (lane i: draft i), with the first loads
  const int dr = w == 0 && blockIdx.x == 0 && lane < D ? a.drafts[lane] : 0;
  if (tid == 0) s_epoch = (uint32_t)ld_ag(k.ctr + kEpochInt);
  __syncthreads();
  const uint32_t epoch = s_epoch;
  const uint32_t tag = (epoch + 1u) & 0x7FFFFFFFu;
  if (has) {
    uint64_t bk = 0;
    uint32_t bad = 0;
    const int nv = V - j0;
#pragma unroll
    for (int e = 0; e < kSub; ++e) {
      const bool in = e < nv;
      bad |= in && (__float_as_uint(v[e]) & 0x7F800000u) == 0x7F800000u;
      const uint64_t kv = ((uint64_t)ss_key(v[e] == 0.f ? 0.f : v[e]) << 32) | (0xFFFFFFFFu - (uint32_t)(j0 + e));
      bk = in && kv > bk ? kv : bk;
    }
    bk = ss_wave_max_u64(bk);
    bad = ss_wave_or(bad);
    if (lane == 0) {
      const size_t o = (size_t)row * nch + c;
      st_ag(k.wd0 + o, ((uint64_t)(tag | (bad ? 0x80000000u : 0u)) << 32) | (uint32_t)(bk >> 32));
      st_ag(k.wd1 + o, ((uint64_t)tag << 32) | (uint32_t)bk);
    }
  }
  if (blockIdx.x != 0) return;
  // workgroup 0: wave w reduces rows w, w + 4, .. once all their chunk words carry this launch's tag
  for (int r = w; r < rows; r += 4) {
    uint64_t bk = 0;
    uint32_t bad = 0;
    for (int it = 0;; ++it) {
      int ok = 1;
      bk = 0;
      bad = 0;
      uint64_t w0[kMaxPerLane], w1[kMaxPerLane];  // every load of the poll in flight before any is used
#pragma unroll
      for (int q = 0; q < kMaxPerLane; ++q) {
        const int cc = lane + 64 * q;
        w0[q] = cc < nch ? ld_ag(k.wd0 + (size_t)r * nch + cc) : 0;
        w1[q] = cc < nch ? ld_ag(k.wd1 + (size_t)r * nch + cc) : 0;
      }
#pragma unroll
      for (int q = 0; q < kMaxPerLane; ++q) {
        if (lane + 64 * q >= nch) continue;
        ok &= tag_of(w0[q]) == tag && tag_of(w1[q]) == tag;
        const uint64_t kv = ((uint64_t)(uint32_t)w0[q] << 32) | (uint32_t)w1[q];
        bk = kv > bk ? kv : bk;
        bad |= (uint32_t)(w0[q] >> 63);
      }
      if (__all(ok)) break;
      if (it >= kSpin) {
        if (lane == 0) ss_raise(a.err, SS_ERR_TIMEOUT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    bk = ss_wave_max_u64(bk);
    bad = ss_wave_or(bad);
    if (lane == 0) {
      s_tok[r] = (int)(0xFFFFFFFFu - (uint32_t)bk);
      s_bad[r] = (int)bad;
    }
  }
  __shared__ int s_dr[64];
  if (w == 0 && lane < D) s_dr[lane] = dr;
  __syncthreads();
  if (tid == 0) {
    // every workgroup has published, so every one has read the epoch
    st_ag(k.ctr + kEpochInt, (int)(epoch + 1u));
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

constexpr int kFastUnits = 1024;                            // units of the one-launch round (one wave each)
constexpr int kFastStage = 2 * kFastUnits + 15 * kMaxRows;  // rows x nchp chunk parts staged per workgroup

template <int KM>
__global__ __launch_bounds__(256) void pq_round_kernel(AcceptArgs a, int units) {
  __shared__ __attribute__((aligned(16))) float sv[kFastStage], sm[kFastStage], sb[kFastStage], sc[kFastStage];
  __shared__ float mrow[kMaxRows], zrow[kMaxRows];
  __shared__ int brow[kMaxRows];
  __shared__ PqIn s_in;
  __shared__ PqState s_st;
  __shared__ uint64_t s_tr[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int D = a.D, V = a.V, nch = nchunks_of(V), rows = 2 * D + 1, nchp = (nch + 15) & ~15;
  const int kc = KM < kMaxPerLane ? KM : (nch + 63) >> 6;  // chunks per lane of the chunk layout
  const float invT = 1.0f / a.temperature;
  // phase stamps, kept in LDS and written at the exit: slot k by thread 0, slots 8 + k by lane 0 of a sampled-row wave
#define PQ_TRACE(k, who)                                               \
  do {                                                                 \
    if (a.trace && (who)) s_tr[k] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
  if (tid < 16) s_tr[tid] = 0;
  PQ_TRACE(0, tid == 0);
  Work k = work_of(a.work, rows, nch);
  const int gw = blockIdx.x * 4 + w;
  const bool has = gw < units;
  const int ui = has ? gw / nch : 0, c = has ? gw - ui * nch : 0;
  const int j0 = c * kChunk + kSub * lane;
  const bool vec = (V & 3) == 0 && (reinterpret_cast<uintptr_t>(a.target) & 15) == 0 &&
                   (D == 0 || (reinterpret_cast<uintptr_t>(a.draft) & 15) == 0);
  // the unit's logits (target row ui; draft row ui when ui < D), and the drafts, their logits and the uniforms
  float vt[kSub], vd[kSub];
  if (has) load16(a.target + (size_t)ui * V, j0, V, vec, vt);
  if (has && ui < D) load16(a.draft + (size_t)ui * V, j0, V, vec, vd);
  if (w == 0) {
    const int xi = lane < D ? a.drafts[lane] : 0;
    const bool xok = lane < D && xi >= 0 && xi < V;
    s_in.x[lane] = xi;
    s_in.lt[lane] = xok ? a.target[(size_t)lane * V + xi] : 0.f;
    s_in.lq[lane] = xok ? a.draft[(size_t)lane * V + xi] : 0.f;
    s_in.u[lane] = lane <= D ? a.uniforms[lane] : 0.f;
  }
  // The epoch, read once per workgroup (with the loads above in flight) and shared, so that every thread's tag was
  // read before any wave of the workgroup publishes.
  __shared__ uint32_t s_epoch;
  if (tid == 0) s_epoch = (uint32_t)ld_ag(k.ctr + kEpochInt);
  __syncthreads();
  const uint32_t epoch = s_epoch;
  const uint32_t tag = (epoch + 1u) & 0x7FFFFFFFu;
  // phase 1: the unit's chunk parts (vt, vd become e), published as tagged words
  if (a.trace && tid == 0) {
    __builtin_amdgcn_s_waitcnt(0);  // traced launches only: the stamp after this wave's loads have landed
    s_tr[12] = __builtin_amdgcn_s_memrealtime();
  }
  if (has) {
    const ChunkPart pt = chunk_part(vt, j0, V, invT);
    PQ_TRACE(13, tid == 0);
    if (lane == 0) {
      const size_t o = (size_t)ui * nch + c;
      st_ag(k.wd0 + o, tagged(tag | (pt.bad ? 0x80000000u : 0u), pt.m));
      st_ag(k.wd1 + o, tagged(tag, pt.s));
    }
    if (ui < D) {
      const ChunkPart pd = chunk_part(vd, j0, V, invT);
      if (lane == 0) {
        const size_t o = (size_t)(D + 1 + ui) * nch + c;
        st_ag(k.wd0 + o, tagged(tag | (pd.bad ? 0x80000000u : 0u), pd.m));
        st_ag(k.wd1 + o, tagged(tag, pd.s));
      }
    }
  }
  PQ_TRACE(1, tid == 0);
  // phase 2: every workgroup polls every row's chunk words until all carry this launch's tag (rows x nch <= 2048:
  // eight pairs per thread), stages them, forms the row statistics and decides
  {
    const int n = rows * nch;
    uint64_t w0[8], w1[8];
    for (int it = 0;; ++it) {
      int ok = 1;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int i = tid + 256 * q;
        w0[q] = i < n ? ld_ag(k.wd0 + i) : 0;
        w1[q] = i < n ? ld_ag(k.wd1 + i) : 0;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (tid + 256 * q < n) ok &= tag_of(w0[q]) == tag && tag_of(w1[q]) == tag;
      if (__syncthreads_and(ok)) break;
      if (it >= kSpin) {
        if (tid == 0) ss_raise(a.err, SS_ERR_TIMEOUT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    // every workgroup has published, so every one has read the epoch: the next launch's tag may follow
    if (blockIdx.x == 0 && tid == 0) st_ag(k.ctr + kEpochInt, (int)(epoch + 1u));
    PQ_TRACE(2, tid == 0);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int i = tid + 256 * q;
      if (i < n) {
        const int r = i / nch, o = r * nchp + (i - r * nch);
        sv[o] = sc[o] = val_of(w1[q]);
        sm[o] = val_of(w0[q]);
        sb[o] = (w0[q] >> 63) ? 1.f : 0.f;
      }
    }
    __syncthreads();
    PQ_TRACE(3, tid == 0);
    for (int r0 = w; r0 < rows; r0 += 8) {
      const int rr[2] = {r0, r0 + 4};
      rows_stats<2, KM>(sv, sm, sb, rr, r0 + 4 < rows ? 2 : 1, nch, nchp, mrow, zrow, brow);
    }
    __syncthreads();
    PQ_TRACE(4, tid == 0);
    if (w == 0) {
      const int xi = s_in.x[lane];
      const bool xbad = lane < D && (xi < 0 || xi >= V);
      const int cx = lane < D && !xbad ? xi >> 10 : 0;
      const int ti = lane < D ? lane : 0, di = lane < D ? D + 1 + lane : 0;
      const bool bad = lane < D && (brow[ti] || brow[di]);
      const float p = p_at(s_in.lt[lane], invT, sm[ti * nchp + cx], sv[ti * nchp + cx]);
      const float q = p_at(s_in.lq[lane], invT, sm[di * nchp + cx], sv[di * nchp + cx]);
      const PqState st = pq_decide(a, bad, xbad, p, q, s_in.u[lane], mrow, zrow, brow, blockIdx.x == 0);
      if (lane == 0) s_st = st;
    }
    __syncthreads();
    PQ_TRACE(5, tid == 0);
  }
  const PqState st = s_st;
  if (st.stop) {
    if (blockIdx.x == 0 && tid == 0) pq_write_out(a, st, s_in.x, -1, st.flags);
  } else if (has && ui == D && st.sdraft < 0) {
    // every draft accepted: the bonus row's sample as the proposal draw takes it (chunk by mass s_c a_c, then the
    // entry from the holding wave's e values), with no second hand-off
    float rv[KM];
#pragma unroll
    for (int i = 0; i < KM; ++i) {
      const int cc = kc * lane + i;
      rv[i] = i < kc && cc < nch ? sc[D * nchp + cc] * sv[D * nchp + cc] : 0.f;
    }
    int flags = st.flags;
    const float S = wave_total(rv, kc, nch);
    if (!(S > 0.f)) flags |= FLAG_RESIDUAL_EMPTY;
    const float t = s_in.u[st.uidx] * S;
    float cbase;
    const int cs = wave_descend(rv, kc, nch, t, &cbase);
    PQ_TRACE(10, lane == 0);
    if (c == cs) {
      const int n_in = V - cs * kChunk < kChunk ? V - cs * kChunk : kChunk;
      float ebase;
      const int e = wave_descend(vt, kSub, n_in, (t - cbase) / sv[D * nchp + cs], &ebase);
      if (lane == 0) pq_write_out(a, st, s_in.x, cs * kChunk + e, flags);
      PQ_TRACE(11, lane == 0);
    }
  } else if (has && ui == st.srow && st.sdraft >= 0) {
    // phase 3: the sampled row's values (in place of vt) and this chunk's total
    const float at = sv[st.srow * nchp + c], ad = sv[st.sdraft * nchp + c];
#pragma unroll
    for (int e = 0; e < kSub; ++e) vt[e] = j0 + e < V ? sampled_value(vt[e], vd[e], at, ad, true) : 0.f;
    const float ct = wave_total(vt, kSub, kChunk);
    if (lane == 0) st_ag(k.wr + c, tagged(tag, ct));
    PQ_TRACE(8, lane == 0);
    // phase 4: every wave of the row polls the chunk totals, finds the chunk of the sample; the wave holding it
    // finds the entry
    float rv[KM];
    for (int it = 0;; ++it) {
      int ok = 1;
#pragma unroll
      for (int i = 0; i < KM; ++i) {
        const int cc = kc * lane + i;
        const bool in = i < kc && cc < nch;
        const uint64_t wv = in ? ld_ag(k.wr + cc) : 0;
        ok &= !in || tag_of(wv) == tag;
        rv[i] = in ? val_of(wv) : 0.f;
      }
      if (__all(ok)) break;
      if (it >= kSpin) {
        if (lane == 0) ss_raise(a.err, SS_ERR_TIMEOUT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    PQ_TRACE(9, lane == 0);
    int flags = st.flags;
    const float S = wave_total(rv, kc, nch);
    if (!(S > 0.f)) flags |= FLAG_RESIDUAL_EMPTY;
    const float t = s_in.u[st.uidx] * S;
    float cbase;
    const int cs = wave_descend(rv, kc, nch, t, &cbase);
    PQ_TRACE(10, lane == 0);
    if (c == cs) {
      const int n_in = V - cs * kChunk < kChunk ? V - cs * kChunk : kChunk;
      float ebase;
      const int e = wave_descend(vt, kSub, n_in, t - cbase, &ebase);
      if (lane == 0) pq_write_out(a, st, s_in.x, cs * kChunk + e, flags);
      PQ_TRACE(11, lane == 0);
    }
  }
  __syncthreads();
  PQ_TRACE(6, tid == 0);
  if (a.trace && tid < 16) a.trace[(size_t)blockIdx.x * 16 + tid] = s_tr[tid];
#undef PQ_TRACE
}

// Two-launch form, first launch: each (chunk, row) workgroup forms its chunk part (four waves, a quarter of the
// chunk each, staged in the sub-chunk layout of stride 17); the last workgroup forms every row's statistics and
// decides the drafts; the round's state goes to the workspace.
__global__ __launch_bounds__(256) void pq_sum_kernel(AcceptArgs a) {
  __shared__ float lds[64 * (kSub + 1)];
  __shared__ __attribute__((aligned(16))) float sv[kStage], sm[kStage], sb[kStage];
  __shared__ float zrow[kMaxRows], mrow[kMaxRows];
  __shared__ int brow[kMaxRows];
  __shared__ float s_m[4];
  __shared__ int s_b[4];
  const int row = blockIdx.y, c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nch = gridDim.x, rows = gridDim.y;
  const float invT = 1.0f / a.temperature;
  Work k = work_of(a.work, rows, nch);
  {
    const float* x = row < a.D + 1 ? a.target + (size_t)row * a.V : a.draft + (size_t)(row - a.D - 1) * a.V;
    constexpr int NQ = kSub / 4;
    float yv[NQ];
    float m = -__builtin_inff();
    uint32_t bad = 0;
#pragma unroll
    for (int ii = 0; ii < NQ; ++ii) {
      const int j = c * kChunk + (w * NQ + ii) * 64 + lane;
      const float v = j < a.V ? x[j] : 0.f;
      yv[ii] = v * invT;
      if (j < a.V) {
        bad |= !finite(v);
        m = fmaxf(m, yv[ii]);
      }
    }
    m = ss_wave_max(m);
    bad = ss_wave_or(bad);
    if (lane == 0) {
      s_m[w] = m;
      s_b[w] = (int)bad;
    }
    __syncthreads();
    const float mc = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
#pragma unroll
    for (int ii = 0; ii < NQ; ++ii) {
      const int e = (w * NQ + ii) * 64 + lane;
      const int j = c * kChunk + e;
      lds[(e >> 4) * (kSub + 1) + (e & (kSub - 1))] = j < a.V ? ss_expf(yv[ii] - mc) : 0.f;
    }
    __syncthreads();
    if (w != 0) return;
    float s = 0.f;
    for (int i = 0; i < kSub; ++i) s = s + lds[lane * (kSub + 1) + i];
    s = ss_readlane_f(wave_scan(s), 63);
    if (lane == 0) {
      const size_t o = (size_t)row * nch + c;
      st_ag(k.cmax + o, mc);
      st_ag(k.ctot + o, s);
      st_ag(k.cbad + o, (s_b[0] | s_b[1] | s_b[2] | s_b[3]) ? 1.f : 0.f);
    }
  }
  // The drafts (lane i holds draft i; D <= 60) arrive with this workgroup's own loads, so the finishing workgroup
  // requests the draft positions' logits and the uniforms together with its staging.
  const int xi = lane < a.D ? a.drafts[lane] : 0;
  if (!arrive_last(k.ctr, 1, row * nch + c, nch * rows)) return;
  arrival_clear(k.ctr, 1);
  const bool xok = lane < a.D && xi >= 0 && xi < a.V;
  const int cx = xok ? xi >> 10 : 0;
  const float lt = xok ? a.target[(size_t)lane * a.V + xi] : 0.f;
  const float lq = xok ? a.draft[(size_t)lane * a.V + xi] : 0.f;
  const float mt = lane < a.D ? ld_ag(k.cmax + (size_t)lane * nch + cx) : 0.f;
  const float md = lane < a.D ? ld_ag(k.cmax + (size_t)(a.D + 1 + lane) * nch + cx) : 0.f;
  const float uu = lane <= a.D ? a.uniforms[lane] : 0.f;
  // Per row: M, Z and the flag.
  const int nchp = (nch + 15) & ~15;
  const int per = kStage / nchp;
  for (int r0 = 0; r0 < rows; r0 += per) {
    const int nr = rows - r0 < per ? rows - r0 : per;
    const size_t o = (size_t)r0 * nch;
    // 17 per lane: one batch for the seven rows of a depth-3 round at V = 151,936 (1,043 chunks)
    stage_rows3_ag<17>(k.ctot + o, k.cmax + o, k.cbad + o, nr, nch, nchp, sv, sm, sb);
    __syncthreads();
    for (int rr = 0; rr < nr; rr += 2) {
      const int ri[2] = {rr, rr + 1};
      rows_stats<2, kMaxPerLane>(sv, sm, sb, ri, rr + 1 < nr ? 2 : 1, nch, nchp, mrow + r0, zrow + r0, brow + r0);
    }
    __syncthreads();
  }
  {
    // a_c at the draft's chunk, as rows_stats forms it: exp(m_c - M) / Z
    const int ti = lane < a.D ? lane : 0, di = lane < a.D ? a.D + 1 + lane : 0;
    const bool xbad = lane < a.D && !xok;
    const bool bad = lane < a.D && (brow[ti] || brow[di]);
    const float p = p_at(lt, invT, mt, ss_expf_le0(mt - mrow[ti]) / zrow[ti]);
    const float q = p_at(lq, invT, md, ss_expf_le0(md - mrow[di]) / zrow[di]);
    const PqState st = pq_decide(a, bad, xbad, p, q, uu, mrow, zrow, brow, true);
    if (lane == 0) {
      k.state[0] = __int_as_float(st.srow);
      k.state[1] = __int_as_float(st.sdraft);
      k.state[2] = __int_as_float(st.uidx);
      k.state[3] = __int_as_float(st.stop);
      k.state[4] = __int_as_float(st.good);
      k.state[5] = __int_as_float(st.flags);
      k.state[6] = st.ms;
      k.state[7] = st.zs;
      k.state[8] = st.md;
      k.state[9] = st.zd;
    }
  }
}

// The round's state as pq_sum_kernel left it, read with one batch of loads.
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
  r.ms = v[6];
  r.zs = v[7];
  r.md = v[8];
  r.zd = v[9];
  return r;
}

// e of entry j of a row from its logit and its chunk's maximum.
SS_DEV float e_of(float x, float invT, float mc) { return ss_expf(x * invT - mc); }

// Two-launch form, second launch: each chunk's workgroup forms the sampled values of its chunk (a_c from the
// chunk's maxima and the sampled rows' M and Z, as row_stats forms it) and their total; the last workgroup finds
// the chunk of the sample over the totals, then recomputes that chunk's values and finds the entry.
__global__ __launch_bounds__(256) void pq_residual_kernel(AcceptArgs a) {
  __shared__ float lds[64 * (kSub + 1)];
  __shared__ int s_dr[64];
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nch = gridDim.x;
  const int V = a.V, D = a.D;
  const float invT = 1.0f / a.temperature;
  Work k = work_of(a.work, 2 * D + 1, nch);
  const PqState st = pq_state(k.state);
  const bool rej = st.sdraft >= 0;
  const float* xt = a.target + (size_t)st.srow * V;
  const float* xd = rej ? a.draft + (size_t)(st.sdraft - D - 1) * V : xt;
  if (!st.stop && !rej) {
    // every draft accepted: the chunk's mass s_c a_c (the proposal draw's form)
    if (tid == 0) {
      const float mt = ld_ag(k.cmax + (size_t)st.srow * nch + c);
      st_ag(k.rtot + c, ld_ag(k.ctot + (size_t)st.srow * nch + c) * (ss_expf_le0(mt - st.ms) / st.zs));
    }
  } else if (!st.stop) {
    const float mt = ld_ag(k.cmax + (size_t)st.srow * nch + c);
    const float md = ld_ag(k.cmax + (size_t)st.sdraft * nch + c);
    const float at = ss_expf_le0(mt - st.ms) / st.zs, ad = ss_expf_le0(md - st.md) / st.zd;
#pragma unroll
    for (int ii = 0; ii < kSub / 4; ++ii) {
      const int e = (w * (kSub / 4) + ii) * 64 + lane;
      const int j = c * kChunk + e;
      float v = 0.f;
      if (j < V) v = sampled_value(e_of(xt[j], invT, mt), rej ? e_of(xd[j], invT, md) : 0.f, at, ad, rej);
      lds[(e >> 4) * (kSub + 1) + (e & (kSub - 1))] = v;
    }
  }
  __syncthreads();
  if (w != 0) return;
  if (!st.stop && rej) {
    float s = 0.f;
    for (int i = 0; i < kSub; ++i) s = s + lds[lane * (kSub + 1) + i];
    s = ss_readlane_f(wave_scan(s), 63);
    if (lane == 0) st_ag(k.rtot + c, s);
  }
  for (int i = lane; i < st.good; i += 64) s_dr[i] = a.drafts[i];
  if (!arrive_last(k.ctr, 2, c, nch)) return;
  arrival_clear(k.ctr, 2);
  int pick = -1, flags = st.flags;
  if (!st.stop) {
    const int kc = (nch + 63) >> 6;
    float rv[kMaxPerLane];
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      const int cc = kc * lane + i;
      rv[i] = i < kc && cc < nch ? ld_ag(k.rtot + cc) : 0.f;
    }
    const float S = wave_total(rv, kc, nch);
    if (!(S > 0.f)) flags |= FLAG_RESIDUAL_EMPTY;
    const float t = a.uniforms[st.uidx] * S;
    float cbase;
    const int cs = wave_descend(rv, kc, nch, t, &cbase);
    // the values of chunk cs, lane l holding entries 16 l .. 16 l + 15: the sampled values after a rejection, e
    // (against (t - base) / a_cs) with every draft accepted
    const float mt = ld_ag(k.cmax + (size_t)st.srow * nch + cs);
    const float md = rej ? ld_ag(k.cmax + (size_t)st.sdraft * nch + cs) : 0.f;
    const float at = ss_expf_le0(mt - st.ms) / st.zs, ad = rej ? ss_expf_le0(md - st.md) / st.zd : 0.f;
    const int j0 = cs * kChunk + kSub * lane;
    float vt[kSub];
#pragma unroll
    for (int e = 0; e < kSub; ++e) {
      const int j = j0 + e;
      const float et = j < V ? e_of(xt[j], invT, mt) : 0.f;
      vt[e] = !rej ? et : j < V ? sampled_value(et, e_of(xd[j], invT, md), at, ad, true) : 0.f;
    }
    const int n_in = V - cs * kChunk < kChunk ? V - cs * kChunk : kChunk;
    float ebase;
    pick = cs * kChunk + wave_descend(vt, kSub, n_in, rej ? t - cbase : (t - cbase) / at, &ebase);
  }
  if (lane == 0) pq_write_out(a, st, s_dr, pick, flags);
}

// ---------------------------------------------------------------- draws from softmax(x / T)
// The proposal draw of the p/q round (ssmoe_sample_rows), one persistent launch per group of rows whose (row, chunk)
// units have a wave each: the chunk parts as in the p/q round (tagged words), the row statistics in every
// workgroup, then each row's chunk by wave_descend over the chunk masses r_c = s_c a_c (one rounding) and, in the
// wave holding the chosen chunk, the entry by wave_descend over its e values (registers) with target
// (t - base) / a_c. One hand-off in all. A row with a non-finite logit still yields an index in [0, V), of no meaning.
int64_t draw_work_floats(int R, int V) {
  const int nch = (V + kChunk - 1) / kChunk;
  return kHeadFloats + (int64_t)R * nch * 7 + (int64_t)nch * 3 + 64;
}

struct DrawArgs {
  const float* x;  // [R, V]
  const float* u;  // [R]
  int32_t* tokens;
  float* work;
  int* err;
  int R, V;
  float temperature;
};

constexpr int kDrawStage = 2048;  // R x nchp chunk parts staged per workgroup (R nch <= 1024, R <= 64)

template <int KM>
__global__ __launch_bounds__(256) void draw_rows_kernel(DrawArgs a, int units) {
  __shared__ __attribute__((aligned(16))) float sv[kDrawStage], sm[kDrawStage], sb[kDrawStage], sc[kDrawStage];
  __shared__ float mrow[64], zrow[64];
  __shared__ int brow[64];
  __shared__ uint32_t s_epoch;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int R = a.R, V = a.V, nch = nchunks_of(V), nchp = (nch + 15) & ~15;
  const int kc = KM < kMaxPerLane ? KM : (nch + 63) >> 6;
  const float invT = 1.0f / a.temperature;
  Work k = work_of(a.work, R, nch);
  const int gw = blockIdx.x * 4 + w;
  const bool has = gw < units;
  const int ui = has ? gw / nch : 0, c = has ? gw - ui * nch : 0;
  const int j0 = c * kChunk + kSub * lane;
  const bool vec = (V & 3) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0;
  float v[kSub];
  if (has) load16(a.x + (size_t)ui * V, j0, V, vec, v);
  const float u = has ? a.u[ui] : 0.f;
  if (tid == 0) s_epoch = (uint32_t)ld_ag(k.ctr + kEpochInt);
  __syncthreads();
  const uint32_t epoch = s_epoch;
  const uint32_t tag = (epoch + 1u) & 0x7FFFFFFFu;
  if (has) {
    const ChunkPart pt = chunk_part(v, j0, V, invT);
    if (lane == 0) {
      const size_t o = (size_t)ui * nch + c;
      st_ag(k.wd0 + o, tagged(tag | (pt.bad ? 0x80000000u : 0u), pt.m));
      st_ag(k.wd1 + o, tagged(tag, pt.s));
    }
  }
  // every workgroup polls every row's chunk words (R nch <= 1024: four pairs per thread)
  const int n = R * nch;
  uint64_t w0[4], w1[4];
  for (int it = 0;; ++it) {
    int ok = 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = tid + 256 * q;
      w0[q] = i < n ? ld_ag(k.wd0 + i) : 0;
      w1[q] = i < n ? ld_ag(k.wd1 + i) : 0;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (tid + 256 * q < n) ok &= tag_of(w0[q]) == tag && tag_of(w1[q]) == tag;
    if (__syncthreads_and(ok)) break;
    if (it >= kSpin) {
      if (tid == 0) ss_raise(a.err, SS_ERR_TIMEOUT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (blockIdx.x == 0 && tid == 0) st_ag(k.ctr + kEpochInt, (int)(epoch + 1u));
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = tid + 256 * q;
    if (i < n) {
      const int r = i / nch, o = r * nchp + (i - r * nch);
      sv[o] = sc[o] = val_of(w1[q]);
      sm[o] = val_of(w0[q]);
      sb[o] = (w0[q] >> 63) ? 1.f : 0.f;
    }
  }
  __syncthreads();
  for (int r0 = w; r0 < R; r0 += 8) {
    const int rr[2] = {r0, r0 + 4};
    rows_stats<2, KM>(sv, sm, sb, rr, r0 + 4 < R ? 2 : 1, nch, nchp, mrow, zrow, brow);
  }
  __syncthreads();
  if (!has) return;
  // the row's chunk: masses r_c = s_c a_c in the chunk layout
  float rv[KM];
#pragma unroll
  for (int i = 0; i < KM; ++i) {
    const int cc = kc * lane + i;
    rv[i] = i < kc && cc < nch ? sc[ui * nchp + cc] * sv[ui * nchp + cc] : 0.f;
  }
  const float t = u * wave_total(rv, kc, nch);
  float cbase;
  const int cs = wave_descend(rv, kc, nch, t, &cbase);
  if (c != cs) return;
  const int n_in = V - cs * kChunk < kChunk ? V - cs * kChunk : kChunk;
  float eb;
  const int e = wave_descend(v, kSub, n_in, (t - cbase) / sv[ui * nchp + cs], &eb);
  if (lane == 0) a.tokens[ui] = cs * kChunk + e;
}

hipError_t launch_draw_rows(const float* x, int R, int V, float temperature, const float* u, void* work,
                            int32_t* tokens, int* err, hipStream_t st) {
  const int nch = (V + kChunk - 1) / kChunk;
  const int kc = (nch + 63) >> 6;
  auto kern = kc == 1 ? draw_rows_kernel<1> : kc == 2 ? draw_rows_kernel<2> : kc == 3 ? draw_rows_kernel<3>
            : kc == 4 ? draw_rows_kernel<4> : draw_rows_kernel<kMaxPerLane>;
  KernelCfg cfg;
  hipError_t e = kernel_cfg(reinterpret_cast<const void*>(kern), 256, 0, &cfg);
  if (e != hipSuccess) return e;
  // rows per launch: every unit a wave of a grid resident at once (one workgroup per CU at most)
  const int cap = 4 * cfg.cus < kFastUnits ? 4 * cfg.cus : kFastUnits;
  const int per = cap / nch < 64 ? cap / nch : 64;
  if (cfg.per_cu < 1 || per < 1) return hipErrorInvalidConfiguration;
  for (int r0 = 0; r0 < R; r0 += per) {
    DrawArgs d;
    d.R = R - r0 < per ? R - r0 : per;
    d.V = V;
    d.x = x + (size_t)r0 * V;
    d.u = u + r0;
    d.tokens = tokens + r0;
    d.work = static_cast<float*>(work);
    d.err = err;
    d.temperature = temperature;
    const int units = d.R * nch;
    hipLaunchKernelGGL(kern, dim3((units + 3) / 4), dim3(256), 0, st, d, units);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_accept_greedy(const AcceptArgs& a, hipStream_t st) {
  const int nch = (a.V + kChunk - 1) / kChunk;
  const int units = (a.D + 1) * nch;
  KernelCfg cfg;
  hipError_t e = kernel_cfg(reinterpret_cast<const void*>(greedy_round_kernel), 256, 0, &cfg);
  if (e != hipSuccess) return e;
  const int grid = (units + 3) / 4;
  if (units <= kFastUnits && cfg.per_cu >= 1 && grid <= cfg.cus) {
    hipLaunchKernelGGL(greedy_round_kernel, dim3(grid), dim3(256), 0, st, a, units);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(greedy_kernel, dim3(nch, a.D + 1), dim3(64), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_accept_pq(const AcceptArgs& a, hipStream_t st) {
  const int nch = (a.V + kChunk - 1) / kChunk;
  const int rows = 2 * a.D + 1;
  const int units = (a.D + 1) * nch;
  // One launch when every unit has a wave of a grid that is resident at once (one workgroup per CU at most).
  const int kc = (nch + 63) >> 6;
  auto kern = kc == 1 ? pq_round_kernel<1> : kc == 2 ? pq_round_kernel<2> : kc == 3 ? pq_round_kernel<3>
            : kc == 4 ? pq_round_kernel<4> : pq_round_kernel<kMaxPerLane>;
  KernelCfg cfg;
  hipError_t e = kernel_cfg(reinterpret_cast<const void*>(kern), 256, 0, &cfg);
  if (e != hipSuccess) return e;
  const int grid = (units + 3) / 4;
  if (units <= kFastUnits && cfg.per_cu >= 1 && grid <= cfg.cus) {
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, st, a, units);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(pq_sum_kernel, dim3(nch, rows), dim3(256), 0, st, a);
  hipLaunchKernelGGL(pq_residual_kernel, dim3(nch), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace ss
