// Prefill MoE: rows sorted into expert-contiguous blocks, a grouped bf16 MFMA GEMM over affine-4bit records
// dequantized into LDS, and the rank-order combine.
//
// Semantics follow kernels/moe_align.py:11-48, kernels/fused_moe_affine.py:39-172 (the reference's prefill path):
//  * moe_align: a stable counting sort of the rows by local expert (rows outside [0, num_local) are skipped); each
//    expert's rows padded to block_m with the sentinel R; every block of block_m positions belongs to one expert.
//    Computed without atomics in any order-dependent place: ranks inside a 256-row chunk by comparison, chunk
//    offsets by a sequential scan per expert.
//  * gate/up: h[r, n] = bf16(silu(g) * u), g = sum_k x[tok(r), k] * bf16(q*s + b)[n, k] with bf16 products and
//    fp32 accumulation (the dequantized weight is rounded to bf16 as the reference's _wtile does; q*s is exact
//    in fp32, so one rounding of q*s + b, fused or not, gives the same value).
//  * down: out_rows[r, n] = (sum_k h[r, k] * bf16(q*s + b)[n, k]) * row_weight[r], fp32.
//  * combine: out[t] = ((o[t,0] + o[t,1]) + ...) + o[t,K-1], sequential fp32.
// Tiles are constants of the kernel (64 rows x 64 columns x 64 K), never functions of R.
#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

// ---------------------------------------------------------------- moe_align
constexpr int kAlignChunk = 256;

int64_t padded_rows(int64_t R, int num_local, int block_m) {
  const int64_t n = R + (int64_t)num_local * (block_m - 1);
  return (n + block_m - 1) / block_m * block_m;
}

// scratch ints: rank [R], chunk offsets [nchunk][num_local], pad_start [num_local + 1], totals [num_local]
int64_t align_scratch_ints(int64_t R, int num_local) {
  const int64_t nch = (R + kAlignChunk - 1) / kAlignChunk;
  return R + nch * num_local + 2 * (int64_t)num_local + 1;
}

SS_DEV int align_key(const int32_t* le, int64_t i, int64_t R, int nl) {
  if (i >= R) return nl + 1;
  const int v = le[i];
  return (v >= 0 && v < nl) ? v : nl;
}

// Per chunk: the rank of each row among the earlier rows of the chunk with the same key, and per-key counts.
__global__ __launch_bounds__(kAlignChunk) void align_count_kernel(const int32_t* __restrict__ le, int64_t R, int nl,
                                                                  int32_t* __restrict__ rank,
                                                                  int32_t* __restrict__ chunk_cnt) {
  extern __shared__ int sm_cnt[];  // [nl]
  __shared__ int keys[kAlignChunk];
  const int tid = threadIdx.x;
  const int64_t i = (int64_t)blockIdx.x * kAlignChunk + tid;
  const int key = align_key(le, i, R, nl);
  keys[tid] = key;
  for (int e = tid; e < nl; e += kAlignChunk) sm_cnt[e] = 0;
  __syncthreads();
  int r = 0;
#pragma unroll 8
  for (int j = 0; j < kAlignChunk; ++j) r += (j < tid && keys[j] == key) ? 1 : 0;
  if (i < R) rank[i] = r;
  if (key < nl) atomicAdd(&sm_cnt[key], 1);  // integer counts: any order gives the same totals
  __syncthreads();
  for (int e = tid; e < nl; e += kAlignChunk) chunk_cnt[(int64_t)blockIdx.x * nl + e] = sm_cnt[e];
}

// One workgroup: exclusive chunk offsets per key (sequential over chunks), padded expert ranges, block experts,
// the sentinel padding and num_padded.
__global__ __launch_bounds__(1024) void align_scan_kernel(int64_t R, int nl, int bm, int nch, int64_t P,
                                                          int32_t* __restrict__ chunk_cnt, int32_t* __restrict__ pad,
                                                          int32_t* __restrict__ sorted_rows,
                                                          int32_t* __restrict__ block_expert,
                                                          int32_t* __restrict__ num_padded) {
  extern __shared__ int sm[];  // pad_start [nl + 1], total [nl]
  int* ps = sm;
  int* tot = sm + nl + 1;
  const int tid = threadIdx.x;
  for (int e = tid; e < nl; e += 1024) {
    int run = 0;
    for (int c = 0; c < nch; ++c) {
      const int v = chunk_cnt[(int64_t)c * nl + e];
      chunk_cnt[(int64_t)c * nl + e] = run;
      run += v;
    }
    tot[e] = run;
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int e = 0; e < nl; ++e) {
      ps[e] = run;
      run += (tot[e] + bm - 1) / bm * bm;
    }
    ps[nl] = run;
    *num_padded = run;
  }
  __syncthreads();
  for (int e = tid; e <= nl; e += 1024) pad[e] = ps[e];
  const int64_t nb = P / bm;
  for (int64_t q = tid; q < nb; q += 1024) {
    const int64_t pos = q * bm;
    // expert whose padded range holds pos: the last e with ps[e] <= pos (binary search), -1 past the end
    int lo = 0, hi = nl;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (ps[mid] <= pos) lo = mid;
      else hi = mid - 1;
    }
    const int e = pos < ps[nl] ? lo : -1;
    block_expert[q] = e;
    for (int m = 0; m < bm; ++m) {
      const int64_t p = pos + m;
      if (e < 0 || p - ps[e] >= tot[e]) sorted_rows[p] = (int32_t)R;
    }
  }
}

__global__ __launch_bounds__(kAlignChunk) void align_scatter_kernel(const int32_t* __restrict__ le, int64_t R, int nl,
                                                                    const int32_t* __restrict__ rank,
                                                                    const int32_t* __restrict__ chunk_off,
                                                                    const int32_t* __restrict__ pad,
                                                                    int32_t* __restrict__ sorted_rows) {
  const int64_t i = (int64_t)blockIdx.x * kAlignChunk + threadIdx.x;
  const int key = align_key(le, i, R, nl);
  if (key < nl) sorted_rows[pad[key] + chunk_off[(int64_t)blockIdx.x * nl + key] + rank[i]] = (int32_t)i;
}

hipError_t launch_moe_align(const AlignArgs& a, hipStream_t st) {
  const int nch = (int)((a.R + kAlignChunk - 1) / kAlignChunk);
  int32_t* rank = a.scratch;
  int32_t* chunk = rank + a.R;
  int32_t* pad = chunk + (int64_t)nch * a.num_local;
  const int64_t P = padded_rows(a.R, a.num_local, a.block_m);
  if (nch > 0)
    hipLaunchKernelGGL(align_count_kernel, dim3(nch), dim3(kAlignChunk), (size_t)a.num_local * 4, st, a.local_expert,
                       a.R, a.num_local, rank, chunk);
  hipLaunchKernelGGL(align_scan_kernel, dim3(1), dim3(1024), (size_t)(2 * a.num_local + 1) * 4, st, a.R, a.num_local,
                     a.block_m, nch, P, chunk, pad, a.sorted_rows, a.block_expert, a.num_padded);
  if (nch > 0)
    hipLaunchKernelGGL(align_scatter_kernel, dim3(nch), dim3(kAlignChunk), 0, st, a.local_expert, a.R, a.num_local,
                       rank, chunk, pad, a.sorted_rows);
  return hipGetLastError();
}

// ---------------------------------------------------------------- grouped GEMM tiles
constexpr int kBM = 64;      // rows per block (the moe_align block)
constexpr int kBN = 64;      // output columns per block and matrix
constexpr int kBK = 64;      // K per step: one quantisation group
constexpr int kLdsRow = 72;  // bf16 per LDS row (64 + 8 padding: rows 144 B apart spread the banks)

// v or zero, selected component by component (a select of whole vectors can turn into a load through a
// selected private/global address).
SS_DEV uint4 zero_if(bool z, uint4 v) {
  return make_uint4(z ? 0u : v.x, z ? 0u : v.y, z ? 0u : v.z, z ? 0u : v.w);
}

SS_DEV uint32_t pack_bf16x2_rne(float lo, float hi) { return ss_f32_to_bf16(lo) | (ss_f32_to_bf16(hi) << 16); }

// 32 nibbles (one 16-byte word group of a weight row: elements k .. k+31) -> 16 words of bf16 pairs
// bf16(q * s + b) in element order.
SS_DEV void dequant32(uint4 w, float s, float b, uint32_t out[16]) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float q0 = (float)((ww[d] >> (8 * p)) & 15u);
      const float q1 = (float)((ww[d] >> (8 * p + 4)) & 15u);
      out[4 * d + p] = pack_bf16x2_rne(__builtin_fmaf(q0, s, b), __builtin_fmaf(q1, s, b));
    }
  }
}

// One K step of a 64-row x (NT x 16)-column output tile per wave pair layout: waves (wm, wn) = (w >> 1, w & 1).
// A: As[row][k] bf16 (kLdsRow stride); B: Bs[col][k] bf16 (kLdsRow stride).
SS_DEV ss_u32x4 lds_frag(const uint16_t* base, int row, int k) {
  return *reinterpret_cast<const ss_u32x4*>(base + row * kLdsRow + k);
}

struct GemmArgs {
  const uint16_t* a;          // gate/up: x bf16 [T, H]; down: h bf16 [R, I]
  const int32_t* row_token;   // [R] (gate/up)
  const float* row_weight;    // [R] (down)
  const int32_t* sorted_rows; // [P]
  const int32_t* block_expert;// [P / kBM]
  const int32_t* num_padded;  // [1]
  const int64_t* group_ptr;   // [num_local] record base addresses
  uint16_t* h;                // gate/up output bf16 [R, I]
  float* out_rows;            // down output fp32 [R, H]
  int64_t R;
  int T, H, I;
  int64_t w_off, s_off, b_off;   // gate (or down) pieces
  int64_t w2_off, s2_off, b2_off;  // up pieces (gate/up)
};

// Gate/up: grid (I / kBN, P / kBM). Per block: 64 sorted rows x (64 gate + 64 up) columns, K = H.
__global__ __launch_bounds__(256) void prefill_gate_up_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][2 * kBN * kLdsRow];
  __shared__ int tok_s[kBM];
  __shared__ int row_s[kBM];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int pid_n = blockIdx.x, pid_m = blockIdx.y;
  if ((int64_t)pid_m * kBM >= (int64_t)g.num_padded[0]) return;
  const int e = g.block_expert[pid_m];
  if (e < 0) return;
  const uint8_t* base = reinterpret_cast<const uint8_t*>(g.group_ptr[e]);
  const int H = g.H, I = g.I;
  if (tid < kBM) {
    const int r = g.sorted_rows[(int64_t)pid_m * kBM + tid];
    row_s[tid] = r;
    const int t = r < g.R ? g.row_token[r] : -1;
    tok_s[tid] = (t >= 0 && t < g.T) ? t : -1;
  }
  __syncthreads();
  // Loader roles. x: 64 rows x 8 chunks of 16 B -> two chunks per thread (rows tid / 8 and tid / 8 + 32).
  const int xr0 = tid >> 3, xc = tid & 7;
  const int t0 = tok_s[xr0], t1 = tok_s[xr0 + 32];
  const uint16_t* xp0 = g.a + (int64_t)(t0 < 0 ? 0 : t0) * H + 8 * xc;
  const uint16_t* xp1 = g.a + (int64_t)(t1 < 0 ? 0 : t1) * H + 8 * xc;
  // Weights: 128 rows (64 gate, 64 up) x 2 halves of 32 nibbles -> one 16-byte word per thread.
  const int wcol = tid >> 1, whalf = tid & 1;
  const int nrow = pid_n * kBN + (wcol & 63);
  const bool up = wcol >= 64;
  const uint8_t* wp = base + (up ? g.w2_off : g.w_off) + (int64_t)nrow * (H / 2) + 16 * whalf;
  const uint16_t* sp = reinterpret_cast<const uint16_t*>(base + (up ? g.s2_off : g.s_off)) + (int64_t)nrow * (H / 64);
  const uint16_t* bp = reinterpret_cast<const uint16_t*>(base + (up ? g.b2_off : g.b_off)) + (int64_t)nrow * (H / 64);
  const int nsteps = H / kBK;

  uint4 xv0, xv1, wv;
  uint16_t sv, bv;
  auto fetch = [&](int ks) {
    const int k0 = ks * kBK;
    xv0 = ldg16(xp0 + k0);
    xv1 = ldg16(xp1 + k0);
    wv = ldg16(wp + k0 / 2);
    sv = sp[ks];
    bv = bp[ks];
  };
  auto stage = [&](int buf) {
    *reinterpret_cast<uint4*>(&As[buf][xr0 * kLdsRow + 8 * xc]) = zero_if(t0 < 0, xv0);
    *reinterpret_cast<uint4*>(&As[buf][(xr0 + 32) * kLdsRow + 8 * xc]) = zero_if(t1 < 0, xv1);
    uint32_t d[16];
    dequant32(wv, ss_bf16_to_f32(sv), ss_bf16_to_f32(bv), d);
    uint4* dst = reinterpret_cast<uint4*>(&Bs[buf][wcol * kLdsRow + 32 * whalf]);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = make_uint4(d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]);
  };

  const int wm = w >> 1, wn = w & 1;
  const int fr = lane & 15, fk = 8 * (lane >> 4);
  ss_f32x4 accg[2][2], accu[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      accg[i][j] = ss_f32x4{0.f, 0.f, 0.f, 0.f};
      accu[i][j] = ss_f32x4{0.f, 0.f, 0.f, 0.f};
    }
  fetch(0);
  stage(0);
  __syncthreads();
#pragma unroll 1
  for (int ks = 0; ks < nsteps; ++ks) {
    const int buf = ks & 1;
    if (ks + 1 < nsteps) fetch(ks + 1);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      ss_u32x4 af[2], bg[2], bu[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = lds_frag(As[buf], 32 * wm + 16 * i + fr, kk + fk);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bg[j] = lds_frag(Bs[buf], 32 * wn + 16 * j + fr, kk + fk);
        bu[j] = lds_frag(Bs[buf], kBN + 32 * wn + 16 * j + fr, kk + fk);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          accg[i][j] = ss_mfma(af[i], bg[j], accg[i][j]);
          accu[i][j] = ss_mfma(af[i], bu[j], accu[i][j]);
        }
    }
    if (ks + 1 < nsteps) stage(buf ^ 1);
    __syncthreads();
  }
  // Epilogue: D[m][n] of tile (i, j) sits in lane n + 16 (m / 4), element m % 4.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 32 * wm + 16 * i + 4 * (lane >> 4) + q;
        const int r = row_s[m];
        if (r >= g.R) continue;
        const float gv = accg[i][j][q], uv = accu[i][j][q];
        const float hv = gv / (1.f + ss_expf(-gv)) * uv;
        const int n = pid_n * kBN + 32 * wn + 16 * j + (lane & 15);
        g.h[(int64_t)r * I + n] = (uint16_t)ss_f32_to_bf16(hv);
      }
}

// Down: grid (H / (2 kBN), P / kBM). Per block: 64 sorted rows x 128 output columns, K = I.
__global__ __launch_bounds__(256) void prefill_down_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][2 * kBN * kLdsRow];
  __shared__ int row_s[kBM];
  __shared__ float wt_s[kBM];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int pid_n = blockIdx.x, pid_m = blockIdx.y;
  if ((int64_t)pid_m * kBM >= (int64_t)g.num_padded[0]) return;
  const int e = g.block_expert[pid_m];
  if (e < 0) return;
  const uint8_t* base = reinterpret_cast<const uint8_t*>(g.group_ptr[e]);
  const int H = g.H, I = g.I;
  if (tid < kBM) {
    const int r = g.sorted_rows[(int64_t)pid_m * kBM + tid];
    row_s[tid] = r;
    wt_s[tid] = r < g.R ? g.row_weight[r] : 0.f;
  }
  __syncthreads();
  const int ar0 = tid >> 3, ac = tid & 7;
  const int r0 = row_s[ar0], r1 = row_s[ar0 + 32];
  const uint16_t* ap0 = g.a + (int64_t)(r0 < g.R ? r0 : 0) * I + 8 * ac;
  const uint16_t* ap1 = g.a + (int64_t)(r1 < g.R ? r1 : 0) * I + 8 * ac;
  const int wcol = tid >> 1, whalf = tid & 1;
  const int nrow = pid_n * 2 * kBN + wcol;
  const uint8_t* wp = base + g.w_off + (int64_t)nrow * (I / 2) + 16 * whalf;
  const uint16_t* sp = reinterpret_cast<const uint16_t*>(base + g.s_off) + (int64_t)nrow * (I / 64);
  const uint16_t* bp = reinterpret_cast<const uint16_t*>(base + g.b_off) + (int64_t)nrow * (I / 64);
  const int nsteps = I / kBK;

  uint4 av0, av1, wv;
  uint16_t sv, bv;
  auto fetch = [&](int ks) {
    const int k0 = ks * kBK;
    av0 = ldg16(ap0 + k0);
    av1 = ldg16(ap1 + k0);
    wv = ldg16(wp + k0 / 2);
    sv = sp[ks];
    bv = bp[ks];
  };
  auto stage = [&](int buf) {
    *reinterpret_cast<uint4*>(&As[buf][ar0 * kLdsRow + 8 * ac]) = zero_if(r0 >= g.R, av0);
    *reinterpret_cast<uint4*>(&As[buf][(ar0 + 32) * kLdsRow + 8 * ac]) = zero_if(r1 >= g.R, av1);
    uint32_t d[16];
    dequant32(wv, ss_bf16_to_f32(sv), ss_bf16_to_f32(bv), d);
    uint4* dst = reinterpret_cast<uint4*>(&Bs[buf][wcol * kLdsRow + 32 * whalf]);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = make_uint4(d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]);
  };

  const int wm = w >> 1, wn = w & 1;
  const int fr = lane & 15, fk = 8 * (lane >> 4);
  ss_f32x4 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = ss_f32x4{0.f, 0.f, 0.f, 0.f};
  fetch(0);
  stage(0);
  __syncthreads();
#pragma unroll 1
  for (int ks = 0; ks < nsteps; ++ks) {
    const int buf = ks & 1;
    if (ks + 1 < nsteps) fetch(ks + 1);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      ss_u32x4 af[2], bf[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = lds_frag(As[buf], 32 * wm + 16 * i + fr, kk + fk);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = lds_frag(Bs[buf], 64 * wn + 16 * j + fr, kk + fk);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = ss_mfma(af[i], bf[j], acc[i][j]);
    }
    if (ks + 1 < nsteps) stage(buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 32 * wm + 16 * i + 4 * (lane >> 4) + q;
        const int r = row_s[m];
        if (r >= g.R) continue;
        const int n = pid_n * 2 * kBN + 64 * wn + 16 * j + (lane & 15);
        g.out_rows[(int64_t)r * H + n] = acc[i][j][q] * wt_s[m];
      }
}

hipError_t launch_prefill_gemm(const PrefillArgs& p, hipStream_t st) {
  const SsRecord rec = ss_record_layout(p.H, p.I);
  static_assert(kBM == kPrefillBlockM, "one block size for the plan and the GEMM");
  const int64_t P = padded_rows(p.R, p.num_local, kBM);
  GemmArgs g{};
  g.row_token = p.row_token;
  g.row_weight = p.row_weight;
  g.sorted_rows = p.sorted_rows;
  g.block_expert = p.block_expert;
  g.num_padded = p.num_padded;
  g.group_ptr = p.group_ptr;
  g.h = p.h_buf;
  g.out_rows = p.out_rows;
  g.R = p.R;
  g.T = p.T;
  g.H = p.H;
  g.I = p.I;
  if (P == 0) return hipSuccess;
  g.a = p.x;
  g.w_off = rec.gw;
  g.s_off = rec.gs;
  g.b_off = rec.gb;
  g.w2_off = rec.uw;
  g.s2_off = rec.us;
  g.b2_off = rec.ub;
  hipLaunchKernelGGL(prefill_gate_up_kernel, dim3(p.I / kBN, (unsigned)(P / kBM)), dim3(256), 0, st, g);
  g.a = p.h_buf;
  g.w_off = rec.dw;
  g.s_off = rec.ds;
  g.b_off = rec.db;
  hipLaunchKernelGGL(prefill_down_kernel, dim3(p.H / (2 * kBN), (unsigned)(P / kBM)), dim3(256), 0, st, g);
  return hipGetLastError();
}

// ---------------------------------------------------------------- combine_rank_order (fused_moe_affine.py:164-172)
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ rows,
                                                      const int32_t* __restrict__ row_local, int T, int K, int H,
                                                      float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one float4 of one token
  const int h4 = H >> 2;
  if (idx >= (int64_t)T * h4) return;
  const int64_t t = idx / h4, c = idx - t * h4;
  const float4* p = reinterpret_cast<const float4*>(rows) + (t * K) * h4 + c;
  // Every row is loaded (in bounds) and a skipped row's value replaced by +0 afterwards: a select between a local
  // zero and a loaded value is kept on values, never turned into a load through a selected address.
  float4 acc = p[0];
  if (row_local && row_local[t * K] < 0) acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k = 1; k < K; ++k) {
    const float4 v = p[(int64_t)k * h4];
    const bool skip = row_local && row_local[t * K + k] < 0;
    acc.x = acc.x + (skip ? 0.f : v.x);
    acc.y = acc.y + (skip ? 0.f : v.y);
    acc.z = acc.z + (skip ? 0.f : v.z);
    acc.w = acc.w + (skip ? 0.f : v.w);
  }
  reinterpret_cast<float4*>(out)[idx] = acc;
}

hipError_t launch_combine(const float* rows, const int32_t* row_local, int T, int K, int H, float* out,
                          hipStream_t st) {
  const int64_t n = (int64_t)T * (H / 4);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, rows, row_local, T, K, H,
                     out);
  return hipGetLastError();
}

// group_ptr[e] = slot_ptr[map[map_base + e]] for the resident-pool entry point (0 when absent: such rows are
// skipped by setting their local expert to -1 in the caller's routing).
__global__ void group_ptr_kernel(const int32_t* __restrict__ map, int64_t map_base, int64_t map_len,
                                 const int64_t* __restrict__ slot_ptr, int64_t n_slots, int E, int64_t* gptr,
                                 const int32_t* __restrict__ ids, int64_t R, int32_t* __restrict__ local, int* err) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < E) {
    const int64_t mi = map_base + i;
    const int slot = mi < map_len ? map[mi] : -1;
    gptr[i] = (slot >= 0 && slot < n_slots) ? slot_ptr[slot] : 0;
  }
  if (i < R) {
    const int e = ids[i];
    int le = -1;
    if (e >= 0 && e < E) {
      const int64_t mi = map_base + e;
      const int slot = mi < map_len ? map[mi] : -1;
      if (slot >= 0 && slot < n_slots) le = e;
      else ss_raise(err, SS_ERR_SLOT);
    } else {
      ss_raise(err, SS_ERR_EXPERT_ID);
    }
    local[i] = le;
  }
}

__global__ void row_token_kernel(int64_t R, int K, int32_t* row_token) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < R) row_token[i] = (int32_t)(i / K);
}

hipError_t launch_prefill_tables(const int32_t* map, int64_t map_base, int64_t map_len, const int64_t* slot_ptr,
                                 int64_t n_slots, int E, int64_t* gptr, const int32_t* ids, int64_t R, int K,
                                 int32_t* local, int32_t* row_token, int* err, hipStream_t st) {
  const int64_t n = R > E ? R : E;
  hipLaunchKernelGGL(group_ptr_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, map, map_base, map_len,
                     slot_ptr, n_slots, E, gptr, ids, R, local, err);
  if (R > 0) hipLaunchKernelGGL(row_token_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, st, R, K, row_token);
  return hipGetLastError();
}

}  // namespace ss
