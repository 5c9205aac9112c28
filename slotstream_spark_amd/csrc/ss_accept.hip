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

// Output header: out[0] n_accept, out[1] n_emit, out[2] uniforms used, out[3] flags, out[4..] tokens.
enum { OUT_NACC = 0, OUT_NEMIT = 1, OUT_NUNI = 2, OUT_FLAGS = 3, OUT_TOK = 4 };
enum { FLAG_NONFINITE = 1, FLAG_BAD_DRAFT = 2, FLAG_RESIDUAL_EMPTY = 4 };

SS_DEV int nchunks_of(int V) { return (V + kChunk - 1) / kChunk; }

int64_t accept_work_floats(int D, int V) {
  const int nch = (V + kChunk - 1) / kChunk;
  const int rows = 2 * D + 1;
  return (int64_t)rows * nch * 3 + (int64_t)nch * 65 + 64;
}

// Workspace layout (floats).
struct Work {
  float* cmax;   // [rows][nch]
  float* cbad;   // [rows][nch]
  float* ctot;   // [rows][nch]
  float* stot;   // [nch][64]  sub-chunk totals of the sampled row
  float* rtot;   // [nch]      chunk totals of the sampled row
  float* state;  // [64]
};

SS_DEV Work work_of(float* w, int rows, int nch) {
  Work k;
  k.cmax = w;
  k.cbad = w + (size_t)rows * nch;
  k.ctot = w + (size_t)rows * nch * 2;
  k.stot = w + (size_t)rows * nch * 3;
  k.rtot = k.stot + (size_t)nch * 64;
  k.state = k.rtot + nch;
  return k;
}

SS_DEV bool finite(float v) { return (__float_as_uint(v) & 0x7F800000u) != 0x7F800000u; }

// Wave-wide helpers over per-chunk arrays of n <= 64 * kMaxPerLane entries (called by all 64 lanes; every lane
// returns the same value). Entry c is loaded by lane c % 64 into register c / 64, so all loads are in flight at
// once; a sum that must keep its sequential order is then formed in index order from the lanes' registers.
constexpr int kMaxPerLane = 16;  // V <= 16 * 64 * 1024 entries
struct WaveVals {
  float v[kMaxPerLane];
};
SS_DEV WaveVals wave_load(const float* arr, int n) {
  WaveVals w;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < kMaxPerLane; ++k) {
    const int c = lane + 64 * k;
    w.v[k] = c < n ? arr[c] : 0.f;
  }
  return w;
}
// ((v[0] + v[1]) + ...) + v[n-1] from 0.f, fp32, in index order.
SS_DEV float wave_seq_sum(const WaveVals& w, int n) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxPerLane; ++k) {
    if (64 * k >= n) break;
    const int m = n - 64 * k < 64 ? n - 64 * k : 64;
    for (int l = 0; l < m; ++l) s = s + ss_readlane_f(w.v[k], l);
  }
  return s;
}
SS_DEV float wave_max_of(const WaveVals& w, int n) {
  const int lane = threadIdx.x & 63;
  float m = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < kMaxPerLane; ++k) m = lane + 64 * k < n ? fmaxf(m, w.v[k]) : m;
  return ss_wave_max(m);
}
SS_DEV bool wave_any_nonzero(const WaveVals& w, int n) {
  const int lane = threadIdx.x & 63;
  uint32_t b = 0;
#pragma unroll
  for (int k = 0; k < kMaxPerLane; ++k) b |= (lane + 64 * k < n && w.v[k] != 0.f) ? 1u : 0u;
  return ss_wave_or(b) != 0u;
}

// ---------------------------------------------------------------- greedy
__global__ __launch_bounds__(64) void greedy_chunk_kernel(const float* __restrict__ target, int V, float* work) {
  const int row = blockIdx.y, c = blockIdx.x, lane = threadIdx.x;
  const int nch = gridDim.x, rows = gridDim.y;
  Work k = work_of(work, rows, nch);
  const float* x = target + (size_t)row * V;
  // (value, first index) as one 64-bit key: order-preserving value key (+-0 equal, as np.argmax compares) above
  // the complemented index; a row holding a non-finite value is flagged and never decided on.
  uint64_t bk = 0;
  uint32_t bad = 0;
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + i * 64 + lane;
    if (j >= V) break;
    const float v = x[j];
    bad |= !finite(v);
    const uint64_t kv = ((uint64_t)ss_key(v == 0.f ? 0.f : v) << 32) | (0xFFFFFFFFu - (uint32_t)j);
    bk = kv > bk ? kv : bk;
  }
  bk = ss_wave_max_u64(bk);
  bad = ss_wave_or(bad);
  const int bi = (int)(0xFFFFFFFFu - (uint32_t)bk);
  const float best = ss_unkey((uint32_t)(bk >> 32));
  if (lane == 0) {
    k.cmax[row * nch + c] = best;
    k.ctot[row * nch + c] = __int_as_float(bi);
    k.cbad[row * nch + c] = bad ? 1.f : 0.f;
  }
}

__global__ __launch_bounds__(64) void greedy_finish_kernel(const int32_t* __restrict__ drafts, int D, int nch,
                                                           float* work, int32_t* out) {
  const int lane = threadIdx.x;
  Work k = work_of(work, D + 1, nch);
  __shared__ int tok[64];
  __shared__ int bad[64];
  // Row i's first maximum over its chunk maxima: the largest (value key, complemented index) over the wave.
  for (int row = 0; row <= D; ++row) {
    uint64_t bk = 0;
    uint32_t b = 0;
#pragma unroll
    for (int q = 0; q < kMaxPerLane; ++q) {
      const int c = lane + 64 * q;
      if (c < nch) {
        const float v = k.cmax[row * nch + c];
        const int i = __float_as_int(k.ctot[row * nch + c]);
        b |= k.cbad[row * nch + c] != 0.f ? 1u : 0u;
        const uint64_t kv = ((uint64_t)ss_key(v == 0.f ? 0.f : v) << 32) | (0xFFFFFFFFu - (uint32_t)i);
        bk = kv > bk ? kv : bk;
      }
    }
    bk = ss_wave_max_u64(bk);
    b = ss_wave_or(b);
    if (lane == 0) {
      tok[row] = (int)(0xFFFFFFFFu - (uint32_t)bk);
      bad[row] = (int)b;
    }
  }
  __syncthreads();
  if (lane == 0) {
    int good = 0, emit = 0, flags = 0;
    for (int i = 0; i <= D; ++i) {
      if (bad[i]) {
        flags |= FLAG_NONFINITE;
        break;
      }
      out[OUT_TOK + emit++] = tok[i];
      if (i < D && tok[i] == drafts[i]) {
        ++good;
        continue;
      }
      break;
    }
    for (int i = emit; i <= D; ++i) out[OUT_TOK + i] = -1;
    out[OUT_NACC] = good;
    out[OUT_NEMIT] = emit;
    out[OUT_NUNI] = 0;
    out[OUT_FLAGS] = flags;
  }
}

hipError_t launch_accept_greedy(const AcceptArgs& a, hipStream_t st) {
  const int nch = (a.V + kChunk - 1) / kChunk;
  hipLaunchKernelGGL(greedy_chunk_kernel, dim3(nch, a.D + 1), dim3(64), 0, st, a.target, a.V, a.work);
  hipLaunchKernelGGL(greedy_finish_kernel, dim3(1), dim3(64), 0, st, a.drafts, a.D, nch, a.work, a.out);
  return hipGetLastError();
}

// ---------------------------------------------------------------- p/q
// Logical rows: target i -> i (0..D), draft i -> D + 1 + i.
SS_DEV const float* row_ptr(const AcceptArgs& a, int row) {
  return row <= a.D ? a.target + (size_t)row * a.V : a.draft + (size_t)(row - a.D - 1) * a.V;
}

__global__ __launch_bounds__(64) void pq_max_kernel(AcceptArgs a) {
  const int row = blockIdx.y, c = blockIdx.x, lane = threadIdx.x;
  const int nch = gridDim.x, rows = gridDim.y;
  Work k = work_of(a.work, rows, nch);
  const float* x = row_ptr(a, row);
  float m = -__builtin_inff();
  int bad = 0;
  for (int i = 0; i < kSub; ++i) {
    const int j = c * kChunk + i * 64 + lane;
    if (j >= a.V) break;
    const float v = x[j];
    bad |= !finite(v);
    m = fmaxf(m, v / a.temperature);
  }
  m = ss_wave_max(m);
  bad = (int)ss_wave_or((uint32_t)bad);
  if (lane == 0) {
    k.cmax[row * nch + c] = m;
    k.cbad[row * nch + c] = bad ? 1.f : 0.f;
  }
}

// Row maximum over the chunk maxima (order-free), by the whole wave.
SS_DEV float row_max(const Work& k, int row, int nch) { return wave_max_of(wave_load(k.cmax + (size_t)row * nch, nch), nch); }

// Stage one chunk of a row (as e = exp(l/T - m)) into LDS with a 65-float stride per sub-chunk.
SS_DEV void stage_exp(const AcceptArgs& a, int row, int c, float m, float* lds) {
  const float* x = row_ptr(a, row);
  const int lane = threadIdx.x;
  for (int i = 0; i < kSub; ++i) {
    const int e = i * 64 + lane;
    const int j = c * kChunk + e;
    float v = 0.f;
    if (j < a.V) v = ss_expf(x[j] / a.temperature - m);
    lds[(e >> 4) * (kSub + 1) + (e & (kSub - 1))] = v;
  }
}

__global__ __launch_bounds__(64) void pq_sum_kernel(AcceptArgs a) {
  __shared__ float lds[64 * (kSub + 1)];
  const int row = blockIdx.y, c = blockIdx.x, lane = threadIdx.x;
  const int nch = gridDim.x, rows = gridDim.y;
  Work k = work_of(a.work, rows, nch);
  const float m = row_max(k, row, nch);
  stage_exp(a, row, c, m, lds);
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < kSub; ++i) s = s + lds[lane * (kSub + 1) + i];
  s = ss_wave_sum(s);
  if (lane == 0) k.ctot[row * nch + c] = s;
}

// state: [0] sample target row, [1] sample draft row (-1 = plain p), [2] uniform index, [3] stop (no sample),
//        [4..] per-row Z and m for the two sampled rows.
__global__ __launch_bounds__(64) void pq_decide_kernel(AcceptArgs a, int nch) {
  // Run by the whole wave (every lane computes the same values); lane 0 writes the state.
  const int rows = 2 * a.D + 1;
  Work k = work_of(a.work, rows, nch);
  auto row_sum = [&](int row) { return wave_seq_sum(wave_load(k.ctot + (size_t)row * nch, nch), nch); };
  auto row_bad = [&](int row) { return wave_any_nonzero(wave_load(k.cbad + (size_t)row * nch, nch), nch); };
  int good = 0, flags = 0, stop = 0;
  int srow = a.D, sdraft = -1;
  for (int i = 0; i < a.D; ++i) {
    const int dr = a.D + 1 + i;
    if (row_bad(i) || row_bad(dr)) {
      flags |= FLAG_NONFINITE;
      stop = 1;
      break;
    }
    const int x = a.drafts[i];
    if (x < 0 || x >= a.V) {
      flags |= FLAG_BAD_DRAFT;
      if (threadIdx.x == 0) ss_raise(a.err, SS_ERR_TOKEN);
      srow = i;
      sdraft = dr;
      break;
    }
    const float zp = row_sum(i), zq = row_sum(dr);
    const float mp = row_max(k, i, nch), mq = row_max(k, dr, nch);
    const float p = ss_expf(a.target[(size_t)i * a.V + x] / a.temperature - mp) / zp;
    const float q = ss_expf(a.draft[(size_t)i * a.V + x] / a.temperature - mq) / zq;
    if (a.uniforms[i] * q < p) {
      ++good;
      continue;
    }
    srow = i;
    sdraft = dr;
    break;
  }
  if (!stop && sdraft < 0 && row_bad(a.D)) {
    flags |= FLAG_NONFINITE;
    stop = 1;
  }
  const float zp = row_sum(srow);
  const float zq = sdraft >= 0 ? row_sum(sdraft) : 0.f;
  const float ms = row_max(k, srow, nch);
  const float md = sdraft >= 0 ? row_max(k, sdraft, nch) : 0.f;
  if (threadIdx.x == 0) {
    k.state[0] = __int_as_float(srow);
    k.state[1] = __int_as_float(sdraft);
    k.state[2] = __int_as_float(good + (sdraft >= 0 ? 1 : 0));
    k.state[3] = __int_as_float(stop);
    k.state[4] = __int_as_float(good);
    k.state[5] = __int_as_float(flags);
    k.state[6] = zp;
    k.state[7] = zq;
    k.state[8] = ms;
    k.state[9] = md;
  }
}

// Value of entry j of the sampled distribution: p_j, or max(0, p_j - q_j) after a rejection.
SS_DEV float sample_value(const AcceptArgs& a, const float* st, int j) {
  const int srow = __float_as_int(st[0]), sdraft = __float_as_int(st[1]);
  const float p = ss_expf(a.target[(size_t)srow * a.V + j] / a.temperature - st[8]) / st[6];
  if (sdraft < 0) return p;
  const float q = ss_expf(a.draft[(size_t)(sdraft - a.D - 1) * a.V + j] / a.temperature - st[9]) / st[7];
  const float d = p - q;
  return d > 0.f ? d : 0.f;
}

__global__ __launch_bounds__(64) void pq_residual_kernel(AcceptArgs a) {
  __shared__ float lds[64 * (kSub + 1)];
  const int c = blockIdx.x, lane = threadIdx.x, nch = gridDim.x;
  Work k = work_of(a.work, 2 * a.D + 1, nch);
  if (__float_as_int(k.state[3])) return;
  for (int i = 0; i < kSub; ++i) {
    const int e = i * 64 + lane;
    const int j = c * kChunk + e;
    lds[(e >> 4) * (kSub + 1) + (e & (kSub - 1))] = j < a.V ? sample_value(a, k.state, j) : 0.f;
  }
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < kSub; ++i) s = s + lds[lane * (kSub + 1) + i];
  k.stot[c * 64 + lane] = s;
  s = ss_wave_sum(s);
  if (lane == 0) k.rtot[c] = s;
}

// Inverse-CDF search, by the whole wave: the running sums keep their sequential order (index order, from the
// chunk's base), formed from the lanes' registers; every lane follows the same scan.
__global__ __launch_bounds__(64) void pq_search_kernel(AcceptArgs a, int nch) {
  Work k = work_of(a.work, 2 * a.D + 1, nch);
  const int lane = threadIdx.x;
  const int good = __float_as_int(k.state[4]);
  int flags = __float_as_int(k.state[5]);
  const int stop = __float_as_int(k.state[3]);
  const int uidx = __float_as_int(k.state[2]);
  int emit = good;
  int pick = -1;
  if (!stop) {
    const WaveVals rt = wave_load(k.rtot, nch);
    const float S = wave_seq_sum(rt, nch);
    if (!(S > 0.f)) flags |= FLAG_RESIDUAL_EMPTY;
    const float target = a.uniforms[uidx] * S;
    // chunk: the first whose running total exceeds the target (else the last nonzero one, based at its prefix)
    int cs = -1, clast = -1;
    float base = 0.f, run = 0.f;
#pragma unroll
    for (int q = 0; q < kMaxPerLane; ++q) {
      if (64 * q >= nch) break;
      const int m = nch - 64 * q < 64 ? nch - 64 * q : 64;
      for (int l = 0; l < m; ++l) {
        const float t = ss_readlane_f(rt.v[q], l);
        const float nx = run + t;
        if (t > 0.f) clast = 64 * q + l;
        if (cs < 0 && nx > target) {
          cs = 64 * q + l;
          base = run;
        }
        run = nx;
      }
    }
    if (cs < 0) {
      cs = clast < 0 ? 0 : clast;
      base = 0.f;
#pragma unroll
      for (int q = 0; q < kMaxPerLane; ++q) {
        if (64 * q >= cs) break;
        const int m = cs - 64 * q < 64 ? cs - 64 * q : 64;
        for (int l = 0; l < m; ++l) base = base + ss_readlane_f(rt.v[q], l);
      }
    }
    // sub-chunk: lane b holds the sub-chunk total b of chunk cs
    const float st_b = k.stot[cs * 64 + lane];
    int bs = -1, blast = -1;
    float sbase = base;
    run = base;
    for (int b = 0; b < 64; ++b) {
      const float t = ss_readlane_f(st_b, b);
      const float nx = run + t;
      if (t > 0.f) blast = b;
      if (bs < 0 && nx > target) {
        bs = b;
        sbase = run;
      }
      run = nx;
    }
    if (bs < 0) {
      bs = blast < 0 ? 0 : blast;
      sbase = base;
      for (int b = 0; b < bs; ++b) sbase = sbase + ss_readlane_f(st_b, b);
    }
    // entry: lane i < 16 holds the value of entry i of sub-chunk bs
    const int j0 = cs * kChunk + bs * kSub;
    const int jl = j0 + (lane & (kSub - 1));
    const float val = jl < a.V ? sample_value(a, k.state, jl) : 0.f;
    int last = -1;
    run = sbase;
    for (int i = 0; i < kSub; ++i) {
      const int j = j0 + i;
      if (j >= a.V) break;
      const float v = ss_readlane_f(val, i);
      if (v > 0.f) last = j;
      run = run + v;
      if (run > target) {
        pick = j;
        break;
      }
    }
    if (pick < 0) pick = last >= 0 ? last : min(j0, a.V - 1);
  }
  if (lane == 0) {
    for (int i = 0; i < good; ++i) a.out[OUT_TOK + i] = a.drafts[i];
    if (!stop) a.out[OUT_TOK + emit++] = pick;
    for (int i = emit; i <= a.D; ++i) a.out[OUT_TOK + i] = -1;
    a.out[OUT_NACC] = good;
    a.out[OUT_NEMIT] = emit;
    a.out[OUT_NUNI] = stop ? uidx : uidx + 1;
    a.out[OUT_FLAGS] = flags;
  }
}

hipError_t launch_accept_pq(const AcceptArgs& a, hipStream_t st) {
  const int nch = (a.V + kChunk - 1) / kChunk;
  const int rows = 2 * a.D + 1;
  hipLaunchKernelGGL(pq_max_kernel, dim3(nch, rows), dim3(64), 0, st, a);
  hipLaunchKernelGGL(pq_sum_kernel, dim3(nch, rows), dim3(64), 0, st, a);
  hipLaunchKernelGGL(pq_decide_kernel, dim3(1), dim3(64), 0, st, a, nch);
  hipLaunchKernelGGL(pq_residual_kernel, dim3(nch), dim3(64), 0, st, a);
  hipLaunchKernelGGL(pq_search_kernel, dim3(1), dim3(64), 0, st, a, nch);
  return hipGetLastError();
}

}  // namespace ss
