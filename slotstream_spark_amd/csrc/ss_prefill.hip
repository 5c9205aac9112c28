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
    // Sequential per key; the loads of 16 chunks are issued before their stores so the scan is not one memory
    // round trip per chunk.
    int run = 0;
    for (int c0 = 0; c0 < nch; c0 += 16) {
      int v[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = c0 + q < nch ? chunk_cnt[(int64_t)(c0 + q) * nl + e] : 0;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        if (c0 + q < nch) chunk_cnt[(int64_t)(c0 + q) * nl + e] = run;
        run += v[q];
      }
    }
    tot[e] = run;
  }
  __syncthreads();
  // Exclusive scan of the padded expert sizes: each thread sums up to 4 consecutive experts, a Hillis-Steele scan
  // over the 1024 thread totals, then the per-thread prefixes (nl <= 4096).
  __shared__ int part[1024];
  int loc[4], sum = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = 4 * tid + q;
    loc[q] = e < nl ? (tot[e] + bm - 1) / bm * bm : 0;
    sum += loc[q];
  }
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int run = part[tid] - sum;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = 4 * tid + q;
    if (e < nl) ps[e] = run;
    run += loc[q];
  }
  if (tid == 1023) {
    ps[nl] = part[1023];
    *num_padded = part[1023];
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

// ---------------------------------------------------------------- grouped GEMM
// Block: 256 threads, 64 sorted rows x 128 weight rows (gate/up: 64 gate + the same 64 up rows; down: 128 rows),
// K in steps of 64 (one quantisation group). Each step's operands arrive in LDS by direct-to-LDS loads into a ring
// of kStages slots, kStages - 1 steps ahead of the MFMAs:
//   A    64 rows x 128 B of bf16 activations; the 16-byte chunk c of row r sits in slot c ^ (r & 7), so the 16 rows an
//        MFMA operand read touches fall in different banks;
//   W    128 weight rows x 32 B of packed nibbles;
//   S, B the scale and bias dwords (two groups each) of the 128 rows.
// The step's weights are then dequantized once into a bf16 tile (bf16(q*s + b), rows 144 B apart) that the four
// waves read as MFMA B operands; each wave owns 32 rows x 64 columns of the output.
constexpr int kBM = 64;
constexpr int kBK = 64;
constexpr int kNR = 128;               // weight rows per block
constexpr int kStages = 4;
constexpr int kOffA = 0, kOffW = 8192, kOffS = 12288, kOffB = 12800, kStageBytes = 13312;
constexpr int kTileRow = 72;           // bf16 per row of the dequantized tile
constexpr int kTileBytes = kNR * kTileRow * 2;
constexpr size_t kGemmLds = (size_t)kStages * kStageBytes + kTileBytes;

typedef __bf16 ss_bf16x2 __attribute__((ext_vector_type(2)));

// bf16 pair (lo, hi) rounded to nearest even by the hardware conversion.
SS_DEV uint32_t cvt_pk_bf16(float lo, float hi) {
  const ss_bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

struct GemmArgs {
  const uint16_t* a;           // gate/up: x bf16 [T, H]; down: h bf16 [R, I]
  const int32_t* row_token;    // [R] (gate/up)
  const float* row_weight;     // [R] (down)
  const int32_t* sorted_rows;  // [P]
  const int32_t* block_expert; // [P / kBM]
  const int32_t* num_padded;   // [1]
  const int64_t* group_ptr;    // [num_local] record base addresses
  uint16_t* h;                 // gate/up output bf16 [R, I]
  float* out_rows;             // down output fp32 [R, H]
  int64_t R;
  int T, H, I;
  int64_t w_off, s_off, b_off;     // gate (or down) pieces
  int64_t w2_off, s2_off, b2_off;  // up pieces (gate/up)
};

SS_DEV void waitcnt_vm(int n) {
  // s_waitcnt with only vmcnt constrained (expcnt and lgkmcnt at their maxima); n in {0, 4, 8}.
  if (n >= 8) __builtin_amdgcn_s_waitcnt(0xF78);
  else if (n >= 4) __builtin_amdgcn_s_waitcnt(0xF74);
  else __builtin_amdgcn_s_waitcnt(0xF70);
}

// The shared main loop. GATE_UP: rows 0..63 of the weight tile are gate rows n0 + r, rows 64..127 the up rows
// n0 + r; otherwise 128 consecutive down rows n0 + r. kdim = the K extent, wstride = weight row bytes (kdim / 2),
// sstride = scale row bytes (kdim / 32). acc[i][j]: output rows 32 wm + 16 i, tile columns 64 wn + 16 j.
template <bool GATE_UP>
SS_DEV void gemm_main(const GemmArgs& g, uint8_t* lds, const int* src_row, const uint8_t* base, int n0, int kdim,
                      int astride, ss_f32x4 (&acc)[2][4]) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint8_t* tile = lds + kStages * kStageBytes;
  const int nsteps = kdim / kBK;
  const int64_t wstride = kdim / 2, sstride = kdim / 32;
  // DMA sources of this lane (A: two instructions q = 2w, 2w+1 covering rows 8q .. 8q+7).
  const uint16_t* asrc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 8 * (2 * w + i) + (lane >> 3);
    const int chunk = (lane & 7) ^ (row & 7);
    asrc[i] = g.a + (int64_t)src_row[row] * astride + 8 * chunk;
  }
  const int wrow = 32 * w + (lane >> 1);
  const bool up_row = GATE_UP && wrow >= 64;
  const int64_t wrow_g = n0 + (GATE_UP ? (wrow & 63) : wrow);
  const uint8_t* wsrc = base + (up_row ? g.w2_off : g.w_off) + wrow_g * wstride + 16 * (lane & 1);
  // scale / bias dwords: waves 0, 1 scales of rows 64 w + lane; waves 2, 3 biases of rows 64 (w - 2) + lane.
  const int srow = 64 * (w & 1) + lane;
  const bool s_up = GATE_UP && srow >= 64;
  const int64_t srow_g = n0 + (GATE_UP ? (srow & 63) : srow);
  const int64_t soff = (w < 2) ? (s_up ? g.s2_off : g.s_off) : (s_up ? g.b2_off : g.b_off);
  const uint8_t* ssrc = base + soff + srow_g * sstride;
  auto issue = [&](int ks) {
    uint8_t* st = lds + (ks % kStages) * kStageBytes;
    const int k0 = ks * kBK;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds(asrc[i] + k0, (__attribute__((address_space(3))) void*)(st + kOffA + 1024 * (2 * w + i)), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(wsrc + k0 / 2, (__attribute__((address_space(3))) void*)(st + kOffW + 1024 * w), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(ssrc + ((2 * ks) & ~3), (__attribute__((address_space(3))) void*)(st + (w < 2 ? kOffS + 256 * w : kOffB + 256 * (w - 2))), 4, 0, 0);
  };
#pragma unroll
  for (int ks = 0; ks < kStages - 1; ++ks)
    if (ks < nsteps) issue(ks);
  const int wm = w >> 1, wn = w & 1;
  const int fr = lane & 15, fq = lane >> 4;
  const int drow = tid >> 1, dhalf = tid & 1;  // dequant role: one 16-byte word of one weight row
#pragma unroll 1
  for (int ks = 0; ks < nsteps; ++ks) {
    const int ahead = nsteps - 1 - ks;
    waitcnt_vm(4 * (ahead < kStages - 2 ? ahead : kStages - 2));
    __syncthreads();
    if (ks + kStages - 1 < nsteps) issue(ks + kStages - 1);
    const uint8_t* st = lds + (ks % kStages) * kStageBytes;
    {
      const uint4 wv = *reinterpret_cast<const uint4*>(st + kOffW + 32 * drow + 16 * dhalf);
      const uint32_t sw = *reinterpret_cast<const uint32_t*>(st + kOffS + 4 * drow);
      const uint32_t bw = *reinterpret_cast<const uint32_t*>(st + kOffB + 4 * drow);
      const float sc = __uint_as_float((ks & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
      const float bi = __uint_as_float((ks & 1) ? (bw & 0xFFFF0000u) : (bw << 16));
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t o[16];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t lo = ww[d] & 0x0F0F0F0Fu, hi = (ww[d] >> 4) & 0x0F0F0F0Fu;
        const float q0 = (float)((lo >> 0) & 0xFFu), q1 = (float)((hi >> 0) & 0xFFu);
        const float q2 = (float)((lo >> 8) & 0xFFu), q3 = (float)((hi >> 8) & 0xFFu);
        const float q4 = (float)((lo >> 16) & 0xFFu), q5 = (float)((hi >> 16) & 0xFFu);
        const float q6 = (float)((lo >> 24) & 0xFFu), q7 = (float)((hi >> 24) & 0xFFu);
        o[4 * d + 0] = cvt_pk_bf16(__builtin_fmaf(q0, sc, bi), __builtin_fmaf(q1, sc, bi));
        o[4 * d + 1] = cvt_pk_bf16(__builtin_fmaf(q2, sc, bi), __builtin_fmaf(q3, sc, bi));
        o[4 * d + 2] = cvt_pk_bf16(__builtin_fmaf(q4, sc, bi), __builtin_fmaf(q5, sc, bi));
        o[4 * d + 3] = cvt_pk_bf16(__builtin_fmaf(q6, sc, bi), __builtin_fmaf(q7, sc, bi));
      }
      uint4* dst = reinterpret_cast<uint4*>(tile + (drow * kTileRow + 32 * dhalf) * 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      ss_u32x4 af[2], bf[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int m = 32 * wm + 16 * i + fr;
        const int chunk = (kk >> 3) + fq;
        af[i] = *reinterpret_cast<const ss_u32x4*>(st + kOffA + 128 * m + 16 * (chunk ^ (m & 7)));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = GATE_UP ? (j < 2 ? 32 * wn + 16 * j + fr : 64 + 32 * wn + 16 * (j - 2) + fr)
                                : 64 * wn + 16 * j + fr;
        bf[j] = *reinterpret_cast<const ss_u32x4*>(tile + (col * kTileRow + kk + 8 * fq) * 2);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = ss_mfma(af[i], bf[j], acc[i][j]);
    }
  }
}

// Gate/up: one block per (M block, 64-column N tile), mapped by xcd_tile. Output h[r, n0 .. n0 + 63] = bf16(silu(g) * u).
// Workgroups are dealt to the 8 XCDs round-robin (b % 8). Block b is mapped to M block m and N tile n so that
// the N tiles of one M block run on one XCD, one after another: the gathered activation rows of the M block are
// read once into that XCD's L2 instead of once per XCD.
SS_DEV bool xcd_tile(int nt, int mb, int& pid_n, int& pid_m) {
  const int b = blockIdx.x;
  const int xcd = b & 7, j = b >> 3;
  pid_m = (j / nt) * 8 + xcd;
  pid_n = j % nt;
  return pid_m < mb;
}

__global__ __launch_bounds__(256) void prefill_gate_up_kernel(GemmArgs g, int nt, int mb) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_g[];
  __shared__ int src_row[kBM];
  __shared__ int out_row[kBM];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int pid_n, pid_m;
  if (!xcd_tile(nt, mb, pid_n, pid_m)) return;
  if ((int64_t)pid_m * kBM >= (int64_t)g.num_padded[0]) return;
  const int e = g.block_expert[pid_m];
  if (e < 0) return;
  const uint8_t* base = reinterpret_cast<const uint8_t*>(g.group_ptr[e]);
  if (tid < kBM) {
    const int r = g.sorted_rows[(int64_t)pid_m * kBM + tid];
    const int t = r < g.R ? g.row_token[r] : -1;
    const bool ok = t >= 0 && t < g.T;
    out_row[tid] = ok ? r : -1;
    src_row[tid] = ok ? t : 0;  // padding rows read token 0; their outputs are never stored
  }
  __syncthreads();
  ss_f32x4 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = ss_f32x4{0.f, 0.f, 0.f, 0.f};
  const int n0 = pid_n * 64;
  gemm_main<true>(g, lds_g, src_row, base, n0, g.H, g.H, acc);
  const int wm = w >> 1, wn = w & 1;
  // acc[i][0..1]: gate columns 32 wn + 16 j, acc[i][2..3]: the matching up columns.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 32 * wm + 16 * i + 4 * (lane >> 4) + q;
        const int r = out_row[m];
        if (r < 0) continue;
        const float gv = acc[i][j][q], uv = acc[i][j + 2][q];
        const float hv = gv / (1.f + ss_expf(-gv)) * uv;
        const int n = n0 + 32 * wn + 16 * j + (lane & 15);
        g.h[(int64_t)r * g.I + n] = (uint16_t)ss_f32_to_bf16(hv);
      }
}

// Down: one block per (M block, 128-row N tile), mapped by xcd_tile. Output out_rows[r, n0 .. n0 + 127] = (h Wd^T) * row_weight.
__global__ __launch_bounds__(256) void prefill_down_kernel(GemmArgs g, int nt, int mb) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_d[];
  __shared__ int src_row[kBM];
  __shared__ int out_row[kBM];
  __shared__ float wt_s[kBM];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int pid_n, pid_m;
  if (!xcd_tile(nt, mb, pid_n, pid_m)) return;
  if ((int64_t)pid_m * kBM >= (int64_t)g.num_padded[0]) return;
  const int e = g.block_expert[pid_m];
  if (e < 0) return;
  const uint8_t* base = reinterpret_cast<const uint8_t*>(g.group_ptr[e]);
  if (tid < kBM) {
    const int r = g.sorted_rows[(int64_t)pid_m * kBM + tid];
    const bool ok = r < g.R;
    out_row[tid] = ok ? r : -1;
    src_row[tid] = ok ? r : 0;
    wt_s[tid] = ok ? g.row_weight[r] : 0.f;
  }
  __syncthreads();
  ss_f32x4 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = ss_f32x4{0.f, 0.f, 0.f, 0.f};
  const int n0 = pid_n * kNR;
  gemm_main<false>(g, lds_d, src_row, base, n0, g.I, g.I, acc);
  const int wm = w >> 1, wn = w & 1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 32 * wm + 16 * i + 4 * (lane >> 4) + q;
        const int r = out_row[m];
        if (r < 0) continue;
        const int n = n0 + 64 * wn + 16 * j + (lane & 15);
        g.out_rows[(int64_t)r * g.H + n] = acc[i][j][q] * wt_s[m];
      }
}

hipError_t launch_prefill_gemm(const PrefillArgs& p, hipStream_t st) {
  static_assert(kBM == kPrefillBlockM, "one block size for the plan and the GEMM");
  static bool attr = false;
  if (!attr) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(prefill_gate_up_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLds);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(prefill_down_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLds);
    if (e != hipSuccess) return e;
    attr = true;
  }
  const SsRecord rec = ss_record_layout(p.H, p.I);
  const int64_t P = padded_rows(p.R, p.num_local, kBM);
  if (P == 0 || p.R == 0) return hipSuccess;
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
  g.a = p.x;
  g.w_off = rec.gw;
  g.s_off = rec.gs;
  g.b_off = rec.gb;
  g.w2_off = rec.uw;
  g.s2_off = rec.us;
  g.b2_off = rec.ub;
  const int mb = (int)(P / kBM), mb8 = (mb + 7) / 8 * 8;
  hipLaunchKernelGGL(prefill_gate_up_kernel, dim3((unsigned)(mb8 * (p.I / 64))), dim3(256), kGemmLds, st, g, p.I / 64,
                     mb);
  g.a = p.h_buf;
  g.w_off = rec.dw;
  g.s_off = rec.ds;
  g.b_off = rec.db;
  hipLaunchKernelGGL(prefill_down_kernel, dim3((unsigned)(mb8 * (p.H / kNR))), dim3(256), kGemmLds, st, g, p.H / kNR,
                     mb);
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
