// Router of the MoE layer and the stable top-k.
//
//  * dense_rows_kernel: bf16 GEMV rows (router gate, shared-expert gate/up, shared_expert_gate) with a fixed fp32
//    operation order, so the CPU restatement reproduces every bit (model/layers.py:339, :62-76;
//    reference_torch.py:121, :132-133).
//  * router_topk_kernel: fp32 softmax of the bf16 logits (+ optional routing bias), top-k with ties to the lower
//    index, renormalisation in rank order (model/layers.py:340-347; reference_torch.py:122-124).
//  * topk_stable_kernel: kernels/topk_stable.py:29-113 (order-preserving keys, NaN lowest, k <= 16 sorted by
//    (value desc, index asc), larger k by index, rows shorter than k padded with -1 / -inf).
#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

constexpr int kDenseTB = 4;  // tokens staged per pass

struct SegPack {
  DenseSeg s[4];
  int nseg;
};

__global__ __launch_bounds__(256) void dense_rows_kernel(const uint16_t* __restrict__ x, int T, int H, SegPack segs,
                                                         int total_rows) {
  extern __shared__ uint4 xs[];  // [kDenseTB][H / 8]
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int h8 = H >> 3;
  const int nj = (H + 511) >> 9;
  for (int t0 = 0; t0 < T; t0 += kDenseTB) {
    const int nt = min(kDenseTB, T - t0);
    __syncthreads();
    for (int i = threadIdx.x; i < nt * h8; i += blockDim.x)
      xs[i] = reinterpret_cast<const uint4*>(x + (size_t)(t0 + i / h8) * H)[i % h8];
    __syncthreads();
    for (int row = blockIdx.x * 4 + wid; row < total_rows; row += gridDim.x * 4) {
      int r = row, si = 0;
      while (si < segs.nseg - 1 && r >= segs.s[si].n) {
        r -= segs.s[si].n;
        ++si;
      }
      const uint4* wrow = reinterpret_cast<const uint4*>(segs.s[si].w + (size_t)r * H);
      float acc[kDenseTB] = {0.f, 0.f, 0.f, 0.f};
      for (int j = 0; j < nj; ++j) {
        const int k8 = 64 * j + lane;
        if (k8 >= h8) break;
        const uint4 wv = wrow[k8];
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int t = 0; t < kDenseTB; ++t) {
          if (t >= nt) break;
          const uint4 xv = xs[t * h8 + k8];
          const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
          float a = acc[t];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float wf = __uint_as_float((e & 1) ? (ww[e >> 1] & 0xFFFF0000u) : (ww[e >> 1] << 16));
            const float xf = __uint_as_float((e & 1) ? (xx[e >> 1] & 0xFFFF0000u) : (xx[e >> 1] << 16));
            a = __builtin_fmaf(xf, wf, a);
          }
          acc[t] = a;
        }
      }
#pragma unroll
      for (int t = 0; t < kDenseTB; ++t) {
        if (t >= nt) break;
        const float v = ss_wave_sum(acc[t]);
        if (lane == 0) segs.s[si].out[(size_t)(t0 + t) * segs.s[si].out_ld + r] = (uint16_t)ss_f32_to_bf16(v);
      }
    }
  }
}

hipError_t launch_dense_rows(const uint16_t* x, int T, int H, const DenseSeg* segs, int nseg, hipStream_t st) {
  SegPack p{};
  int total = 0;
  for (int i = 0; i < nseg; ++i) {
    p.s[i] = segs[i];
    total += segs[i].n;
  }
  p.nseg = nseg;
  const int grid = (total + 3) / 4;
  const size_t lds = (size_t)kDenseTB * H * 2;
  hipLaunchKernelGGL(dense_rows_kernel, dim3(grid), dim3(256), lds, st, x, T, H, p, total);
  return hipGetLastError();
}

// ---------------------------------------------------------------- router tail
__global__ __launch_bounds__(64) void router_topk_kernel(const uint16_t* __restrict__ logits,
                                                         const float* __restrict__ bias, float* __restrict__ probs,
                                                         int32_t* __restrict__ ids, float* __restrict__ weights, int E,
                                                         int K) {
  extern __shared__ float sm[];  // E floats, then E taken flags (bytes)
  uint8_t* taken = reinterpret_cast<uint8_t*>(sm + E);
  __shared__ float tv[64];
  __shared__ int ti[64];
  const int t = blockIdx.x, lane = threadIdx.x;
  const uint16_t* lg = logits + (size_t)t * E;
  float m = -__builtin_inff();
  for (int e = lane; e < E; e += 64) {
    float s = ss_bf16_to_f32(lg[e]);
    if (bias) s = s + bias[e];
    sm[e] = s;
    taken[e] = 0;
    m = fmaxf(m, s);
  }
  m = ss_wave_max(m);
  float acc = 0.f;
  for (int e = lane; e < E; e += 64) {
    const float v = ss_expf(sm[e] - m);
    sm[e] = v;
    acc = acc + v;
  }
  const float z = ss_wave_sum(acc);
  for (int e = lane; e < E; e += 64) {
    const float p = sm[e] / z;
    sm[e] = p;
    if (probs) probs[(size_t)t * E + e] = p;
  }
  __syncthreads();
  for (int r = 0; r < K; ++r) {
    // (key, lowest index) as one 64-bit key: key above the complemented index, 0 for taken entries.
    uint64_t best = 0;
    for (int e = lane; e < E; e += 64) {
      if (taken[e]) continue;
      const uint64_t kv = ((uint64_t)ss_key(sm[e]) << 32) | (0xFFFFFFFFu - (uint32_t)e);
      best = kv > best ? kv : best;
    }
    best = ss_wave_max_u64(best);
    const int bi = (int)(0xFFFFFFFFu - (uint32_t)best);
    if (lane == 0) {
      taken[bi] = 1;
      ti[r] = bi;
      tv[r] = sm[bi];
    }
    __syncthreads();
  }
  if (lane == 0) {
    float s = 0.f;
    for (int r = 0; r < K; ++r) s = s + tv[r];
    for (int r = 0; r < K; ++r) {
      ids[(size_t)t * K + r] = ti[r];
      weights[(size_t)t * K + r] = tv[r] / s;
    }
  }
}

// The same router tail with the scores in registers: one wave per token (four per block), lane l holding entries
// l + 64 i (E <= 64 NV). The operations and their order are those of router_topk_kernel: max, exp(s - m) summed per
// lane in i order then by the butterfly, one division per entry; each top-k round takes the largest
// (key + 1) over the untaken entries and, among lanes holding it, the lowest index; the weights divide by the
// rank-order sum of the selected probabilities.
template <int NV>
__global__ __launch_bounds__(256) void router_topk_reg_kernel(const uint16_t* __restrict__ logits,
                                                              const float* __restrict__ bias, float* __restrict__ probs,
                                                              int32_t* __restrict__ ids, float* __restrict__ weights,
                                                              int T, int E, int K) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const uint16_t* lg = logits + (size_t)t * E;
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = lane + 64 * i;
    float sc = ss_bf16_to_f32(lg[e < E ? e : 0]);
    if (bias) sc = sc + bias[e < E ? e : 0];
    v[i] = sc;
  }
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < NV; ++i) m = lane + 64 * i < E ? fmaxf(m, v[i]) : m;
  m = ss_wave_max(m);
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    v[i] = ss_expf(v[i] - m);
    acc = acc + (lane + 64 * i < E ? v[i] : 0.f);
  }
  const float z = ss_wave_sum(acc);
  uint32_t kp[NV];  // key + 1 of a present, untaken entry; 0 once taken or absent
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = lane + 64 * i;
    v[i] = v[i] / z;
    kp[i] = e < E ? ss_key(v[i]) + 1u : 0u;
    if (probs && e < E) probs[(size_t)t * E + e] = v[i];
  }
  float mine = 0.f, sum = 0.f;
  int my_id = 0;
#pragma unroll 1
  for (int r = 0; r < K; ++r) {
    uint32_t lm = kp[0];
#pragma unroll
    for (int i = 1; i < NV; ++i) lm = kp[i] > lm ? kp[i] : lm;
    const uint32_t mx = ss_wave_max_u32(lm);
    int li = NV;
#pragma unroll
    for (int i = NV - 1; i >= 0; --i) li = kp[i] == mx ? i : li;
    const uint32_t code = (uint32_t)(li * 64 + lane);  // the entry index where this lane holds mx
    const uint64_t holders = __ballot(li < NV);
    uint32_t best;
    if (__popcll(holders) == 1)
      best = (uint32_t)__builtin_amdgcn_readlane((int)code, (int)__builtin_ctzll(holders));
    else
      best = ss_wave_min_u32(code);
    const int bi = __builtin_amdgcn_readfirstlane((int)best);
    const int wl = bi & 63, wi = bi >> 6;
    float pl = v[0];
#pragma unroll
    for (int i = 1; i < NV; ++i) pl = i == wi ? v[i] : pl;
    const float pv = ss_readlane_f(pl, wl);
#pragma unroll
    for (int i = 0; i < NV; ++i) kp[i] = (lane == wl && i == wi) ? 0u : kp[i];
    sum = sum + pv;
    mine = lane == r ? pv : mine;
    my_id = lane == r ? bi : my_id;
  }
  if (lane < K) {
    ids[(size_t)t * K + lane] = my_id;
    weights[(size_t)t * K + lane] = mine / sum;
  }
}

hipError_t launch_router_topk(const uint16_t* logits, const float* bias, float* probs, int32_t* ids, float* weights,
                              int T, int E, int K, hipStream_t st) {
  if (E <= 512 && K <= 64) {
    const dim3 grid((unsigned)((T + 3) / 4));
    if (E <= 128)
      hipLaunchKernelGGL(router_topk_reg_kernel<2>, grid, dim3(256), 0, st, logits, bias, probs, ids, weights, T, E, K);
    else if (E <= 256)
      hipLaunchKernelGGL(router_topk_reg_kernel<4>, grid, dim3(256), 0, st, logits, bias, probs, ids, weights, T, E, K);
    else
      hipLaunchKernelGGL(router_topk_reg_kernel<8>, grid, dim3(256), 0, st, logits, bias, probs, ids, weights, T, E, K);
    return hipGetLastError();
  }
  const size_t lds = (size_t)E * 4 + (size_t)E;
  hipLaunchKernelGGL(router_topk_kernel, dim3(T), dim3(64), lds, st, logits, bias, probs, ids, weights, E, K);
  return hipGetLastError();
}

// ---------------------------------------------------------------- topk_stable
// One block of 256 threads per row; thread t owns the contiguous index range [t*C, (t+1)*C).
constexpr int kTopkThreads = 256;

__global__ __launch_bounds__(kTopkThreads) void topk_stable_kernel(const float* __restrict__ scores,
                                                                   const int32_t* __restrict__ n_valid,
                                                                   int32_t* __restrict__ out_idx,
                                                                   float* __restrict__ out_val, int N, int k) {
  __shared__ int hist[256];
  __shared__ int scan_a[kTopkThreads], scan_b[kTopkThreads];
  __shared__ uint32_t s_prefix;
  __shared__ int s_need;
  __shared__ uint32_t sel_key[16];
  __shared__ int sel_idx[16];
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* x = scores + (size_t)row * N;
  int nv = N;
  if (n_valid) nv = min(max(n_valid[row], 0), N);
  const int C = (N + kTopkThreads - 1) / kTopkThreads;
  const int lo = min(tid * C, nv), hi = min(lo + C, nv);
  const int want = min(k, nv);  // entries that can be selected
  // Radix select of the want-th largest key, 8 bits per pass from the top.
  uint32_t prefix = 0;
  int need = want;
  if (want > 0) {
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      const uint32_t mask_hi = pass == 0 ? 0u : (0xFFFFFFFFu << (shift + 8));
      hist[tid] = 0;
      __syncthreads();
      for (int i = lo; i < hi; ++i) {
        const uint32_t key = ss_key(x[i]);
        if ((key & mask_hi) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
      }
      __syncthreads();
      if (tid == 0) {
        int cum = 0, d = 255;
        for (; d > 0; --d) {
          if (cum + hist[d] >= need) break;
          cum += hist[d];
        }
        s_prefix = prefix | ((uint32_t)d << shift);
        s_need = need - cum;
      }
      __syncthreads();
      prefix = s_prefix;
      need = s_need;
      __syncthreads();
    }
  }
  const uint32_t thr = prefix;
  // Count greater / equal per thread, then exclusive scans (thread 0, fixed order).
  int ng = 0, ne = 0;
  if (want > 0) {
    for (int i = lo; i < hi; ++i) {
      const uint32_t key = ss_key(x[i]);
      ng += key > thr;
      ne += key == thr;
    }
  }
  scan_a[tid] = ng;
  scan_b[tid] = ne;
  __syncthreads();
  if (tid == 0) {
    int a = 0, b = 0;
    for (int i = 0; i < kTopkThreads; ++i) {
      const int va = scan_a[i], vb = scan_b[i];
      scan_a[i] = a;
      scan_b[i] = b;
      a += va;
      b += vb;
    }
    s_need = a;  // total greater
  }
  __syncthreads();
  const int total_greater = s_need;
  const int budget = want - total_greater;
  // Selected count per thread (greater, plus ties whose tie rank is inside the budget).
  int tie = scan_b[tid], nsel = 0;
  if (want > 0) {
    for (int i = lo; i < hi; ++i) {
      const uint32_t key = ss_key(x[i]);
      if (key > thr) {
        ++nsel;
      } else if (key == thr) {
        if (tie < budget) ++nsel;
        ++tie;
      }
    }
  }
  __syncthreads();
  scan_a[tid] = nsel;
  __syncthreads();
  if (tid == 0) {
    int a = 0;
    for (int i = 0; i < kTopkThreads; ++i) {
      const int v = scan_a[i];
      scan_a[i] = a;
      a += v;
    }
  }
  __syncthreads();
  int pos = scan_a[tid];
  tie = scan_b[tid];
  int32_t* oi = out_idx + (size_t)row * k;
  float* ov = out_val ? out_val + (size_t)row * k : nullptr;
  const bool by_value = k <= 16;
  if (want > 0) {
    for (int i = lo; i < hi; ++i) {
      const uint32_t key = ss_key(x[i]);
      bool sel = false;
      if (key > thr) {
        sel = true;
      } else if (key == thr) {
        sel = tie < budget;
        ++tie;
      }
      if (!sel) continue;
      if (by_value) {
        sel_key[pos] = key;
        sel_idx[pos] = i;
      } else {
        oi[pos] = i;
        if (ov) ov[pos] = x[i];
      }
      ++pos;
    }
  }
  __syncthreads();
  if (tid == 0) {
    if (by_value) {
      // Insertion sort of the selected entries by (key desc, index asc); they arrive in index order.
      for (int a = 1; a < want; ++a) {
        const uint32_t kk = sel_key[a];
        const int ii = sel_idx[a];
        int b = a - 1;
        while (b >= 0 && (sel_key[b] < kk || (sel_key[b] == kk && sel_idx[b] > ii))) {
          sel_key[b + 1] = sel_key[b];
          sel_idx[b + 1] = sel_idx[b];
          --b;
        }
        sel_key[b + 1] = kk;
        sel_idx[b + 1] = ii;
      }
      for (int a = 0; a < want; ++a) {
        oi[a] = sel_idx[a];
        if (ov) ov[a] = x[sel_idx[a]];
      }
    }
    for (int a = want; a < k; ++a) {
      oi[a] = -1;
      if (ov) ov[a] = -__builtin_inff();
    }
  }
}

hipError_t launch_topk_stable(const float* scores, const int32_t* n_valid, int32_t* idx, float* val, int R, int N,
                              int k, hipStream_t st) {
  hipLaunchKernelGGL(topk_stable_kernel, dim3(R), dim3(kTopkThreads), 0, st, scores, n_valid, idx, val, N, k);
  return hipGetLastError();
}

// ---------------------------------------------------------------- shared expert elementwise chain
// hs[t, i] = bf16(bf16(silu(g)) * u) with g = proj[t, i], u = proj[t, Is + i] (bf16), and sgl[t] = proj[t, 2 Is]:
// the rounding of F.silu and of the bf16 product in the reference's shared expert (model/layers.py:398-402,
// reference_torch.py:132-133), whose gate, up and shared_expert_gate projections arrive as one bf16 GEMM output
// with row stride ld.
__global__ __launch_bounds__(256) void shared_hs_kernel(const uint16_t* __restrict__ proj, int64_t ld, int T, int Is,
                                                        uint16_t* __restrict__ hs, uint16_t* __restrict__ sgl) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)T * Is) return;
  const int64_t t = idx / Is, i = idx - t * Is;
  const uint16_t* row = proj + t * ld;
  const float gv = ss_bf16_to_f32(row[i]), uv = ss_bf16_to_f32(row[Is + i]);
  const float sv = ss_round_bf16(gv / (1.f + ss_expf(-gv)));
  hs[idx] = (uint16_t)ss_f32_to_bf16(sv * uv);
  if (i == 0) sgl[t] = row[2 * Is];
}

hipError_t launch_shared_hs(const uint16_t* proj, int64_t ld, int T, int Is, uint16_t* hs, uint16_t* sgl,
                            hipStream_t st) {
  const int64_t n = (int64_t)T * Is;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(shared_hs_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, proj, ld, T, Is, hs, sgl);
  return hipGetLastError();
}

// y = bf16(bf16(routed) + bf16(bf16(sigmoid(sgl)) * sh)): routed.to(bf16) + sigmoid(x w_sg) * sh with the reference's
// bf16 rounding of each op (model/layers.py:398-402). Four elements per thread.
__global__ __launch_bounds__(256) void combine_shared_kernel(const float* __restrict__ routed,
                                                             const uint16_t* __restrict__ sh,
                                                             const uint16_t* __restrict__ sgl, uint16_t* __restrict__ y,
                                                             int T, int H) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int h4 = H >> 2;
  if (idx >= (int64_t)T * h4) return;
  const int64_t t = idx / h4;
  const float sg = ss_round_bf16(1.f / (1.f + ss_expf(-ss_bf16_to_f32(sgl[t]))));
  const float4 r = reinterpret_cast<const float4*>(routed)[idx];
  const uint2 s2 = reinterpret_cast<const uint2*>(sh)[idx];
  const float rv[4] = {r.x, r.y, r.z, r.w};
  const uint32_t sv[4] = {s2.x & 0xFFFFu, s2.x >> 16, s2.y & 0xFFFFu, s2.y >> 16};
  uint32_t o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float sh2 = ss_round_bf16(sg * ss_bf16_to_f32(sv[c]));
    o[c] = ss_f32_to_bf16(ss_round_bf16(rv[c]) + sh2);
  }
  reinterpret_cast<uint2*>(y)[idx] = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
}

hipError_t launch_combine_shared(const float* routed, const uint16_t* sh, const uint16_t* sgl, uint16_t* y, int T,
                                 int H, hipStream_t st) {
  const int64_t n = (int64_t)T * (H / 4);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_shared_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, routed, sh, sgl, y, T,
                     H);
  return hipGetLastError();
}

// ---------------------------------------------------------------- residual stream and RMSNorm between layers
// s = bf16(resid + y): the residual add of GraphSet._moe (runtime/graphs.py:169) with one stream and unit injection;
// mixed = bf16((s * r) * w), r = 1 / sqrt(sum(s^2) / H + eps): rmsnorm (model/reference_torch.py:30-38) with the
// reduction order fixed. One wave per row: lane l accumulates s^2 over elements 512 j + 8 l .. 512 j + 8 l + 7,
// j = 0, 1, ..., with fma from 0, then the xor butterfly. y == nullptr: s = resid (no add, nothing stored). The
// second pass reads s back from stream_out (the lane's own stores), so stream_out may be resid itself.
__global__ __launch_bounds__(256) void residual_rmsnorm_kernel(const uint16_t* resid, const uint16_t* __restrict__ y,
                                                               const uint16_t* __restrict__ w, float eps, int R, int H,
                                                               uint16_t* stream_out, uint16_t* __restrict__ mixed) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= R) return;  // whole waves; no workgroup barrier follows
  const int h8 = H >> 3;
  const uint4* xs = reinterpret_cast<const uint4*>(resid + (size_t)row * H);
  uint4* so = y ? reinterpret_cast<uint4*>(stream_out + (size_t)row * H) : nullptr;
  float acc = 0.f;
  for (int k8 = lane; k8 < h8; k8 += 64) {
    const uint4 a = xs[k8];
    uint32_t v[4] = {a.x, a.y, a.z, a.w};
    if (y) {
      const uint4 b = reinterpret_cast<const uint4*>(y + (size_t)row * H)[k8];
      const uint32_t bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t lo = ss_f32_to_bf16(ss_bf16_to_f32(v[c] & 0xFFFFu) + ss_bf16_to_f32(bv[c] & 0xFFFFu));
        const uint32_t hi = ss_f32_to_bf16(ss_bf16_to_f32(v[c] >> 16) + ss_bf16_to_f32(bv[c] >> 16));
        v[c] = lo | (hi << 16);
      }
      so[k8] = make_uint4(v[0], v[1], v[2], v[3]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float e0 = ss_bf16_to_f32(v[c] & 0xFFFFu), e1 = ss_bf16_to_f32(v[c] >> 16);
      acc = fmaf(e0, e0, acc);
      acc = fmaf(e1, e1, acc);
    }
  }
  const float r = 1.f / sqrtf(ss_wave_sum(acc) / (float)H + eps);
  const uint4* src = y ? reinterpret_cast<const uint4*>(so) : xs;
  const uint4* ws = w ? reinterpret_cast<const uint4*>(w) : nullptr;
  uint4* mo = reinterpret_cast<uint4*>(mixed + (size_t)row * H);
  for (int k8 = lane; k8 < h8; k8 += 64) {
    const uint4 a = src[k8];
    const uint32_t v[4] = {a.x, a.y, a.z, a.w};
    uint32_t wv[4] = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0 pairs
    if (ws) {
      const uint4 b = ws[k8];
      wv[0] = b.x, wv[1] = b.y, wv[2] = b.z, wv[3] = b.w;
    }
    uint32_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t lo = ss_f32_to_bf16((ss_bf16_to_f32(v[c] & 0xFFFFu) * r) * ss_bf16_to_f32(wv[c] & 0xFFFFu));
      const uint32_t hi = ss_f32_to_bf16((ss_bf16_to_f32(v[c] >> 16) * r) * ss_bf16_to_f32(wv[c] >> 16));
      o[c] = lo | (hi << 16);
    }
    mo[k8] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

hipError_t launch_residual_rmsnorm(const uint16_t* resid, const uint16_t* y, const uint16_t* w, float eps, int R,
                                   int H, uint16_t* stream_out, uint16_t* mixed, hipStream_t st) {
  if (R == 0) return hipSuccess;
  hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3((unsigned)((R + 3) / 4)), dim3(256), 0, st, resid, y, w, eps, R, H,
                     stream_out, mixed);
  return hipGetLastError();
}

}  // namespace ss
