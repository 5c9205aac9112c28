// Prefill MoE: rows sorted into expert-contiguous blocks, a grouped bf16 MFMA GEMM over affine-4bit records
// dequantized into MFMA registers, and the rank-order combine.
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
// Tiles are constants of the kernel (128 rows x 256 weight rows x 64 K), never functions of R.
#include <type_traits>
#include <utility>

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
// Inside a wave the rank is the number of lower lanes holding the same key (one ballot per distinct key of the
// wave, taken in lane order); the earlier waves of the chunk add their counts of that key from LDS.
__global__ __launch_bounds__(kAlignChunk) void align_count_kernel(const int32_t* __restrict__ le, int64_t R, int nl,
                                                                  int32_t* __restrict__ rank,
                                                                  int32_t* __restrict__ chunk_cnt) {
  extern __shared__ uint8_t sm_cnt[];  // [kAlignChunk / 64 waves][nl + 2]: per-wave counts (<= 64) of every key
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  constexpr int NW = kAlignChunk / 64;
  const int nk = nl + 2;  // keys 0 .. nl + 1 (nl: outside [0, nl), nl + 1: past R)
  const int64_t i = (int64_t)blockIdx.x * kAlignChunk + tid;
  const int key = align_key(le, i, R, nl);
  for (int e = tid; e < NW * nk; e += kAlignChunk) sm_cnt[e] = 0;
  __syncthreads();
  // rank inside the wave: walk the wave's distinct keys in the order of their lowest lane
  int r_in = 0;
  uint64_t todo = ~0ull;
  while (todo) {
    const int l0 = (int)__builtin_ctzll(todo);
    const int k0 = __builtin_amdgcn_readlane(key, l0);
    const uint64_t same = __ballot(key == k0);
    if (key == k0) r_in = __popcll(same & ((1ull << lane) - 1ull));
    if (lane == l0) sm_cnt[w * nk + k0] = (uint8_t)__popcll(same);
    todo &= ~same;
  }
  __syncthreads();
  int r = r_in;
  for (int v = 0; v < w; ++v) r += sm_cnt[v * nk + key];
  if (i < R) rank[i] = r;
  for (int e = tid; e < nl; e += kAlignChunk) {
    int c = 0;
#pragma unroll
    for (int v = 0; v < NW; ++v) c += sm_cnt[v * nk + e];
    chunk_cnt[(int64_t)blockIdx.x * nl + e] = c;
  }
}

__global__ void align_zero_kernel(int nl, int32_t* __restrict__ tot) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e < nl) tot[e] = 0;
}

// Per key: exclusive offsets of the key's rows in each chunk (chunk order) and the key's total. One thread per key;
// its nch loads are independent, so they are all in flight at once.
__global__ __launch_bounds__(256) void align_keyscan_kernel(int nl, int nch, int32_t* __restrict__ chunk_cnt,
                                                            int32_t* __restrict__ tot) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= nl) return;
  int run = 0;
  for (int c0 = 0; c0 < nch; c0 += 32) {
    int v[32];
#pragma unroll
    for (int q = 0; q < 32; ++q) v[q] = c0 + q < nch ? chunk_cnt[(int64_t)(c0 + q) * nl + e] : 0;
#pragma unroll
    for (int q = 0; q < 32; ++q) {
      if (c0 + q < nch) chunk_cnt[(int64_t)(c0 + q) * nl + e] = run;
      run += v[q];
    }
  }
  tot[e] = run;
}

// One workgroup: exclusive scan of the padded key sizes -> pad[0 .. nl] (pad[nl] = num_padded), and the expert of
// every block of bm positions (-1 past num_padded).
__global__ __launch_bounds__(1024) void align_padscan_kernel(int nl, int bm, int64_t nb, const int32_t* __restrict__ tot,
                                                             int32_t* __restrict__ pad, int32_t* __restrict__ block_expert,
                                                             int32_t* __restrict__ num_padded) {
  extern __shared__ int ps[];  // [nl + 1]
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  // Each thread sums up to 4 consecutive keys, a Hillis-Steele scan over the 1024 thread totals, then the per-thread
  // prefixes (nl <= 4096).
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
  for (int64_t q = tid; q < nb; q += 1024) {
    const int64_t pos = q * bm;
    // the last key e with ps[e] <= pos (binary search), -1 past the end
    int lo = 0, hi = nl;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (ps[mid] <= pos) lo = mid;
      else hi = mid - 1;
    }
    block_expert[q] = pos < ps[nl] ? lo : -1;
  }
}

// Sentinel R at every position that holds no row: past a key's rows inside its padded range, and past num_padded.
__global__ __launch_bounds__(256) void align_fill_kernel(int64_t R, int nl, int bm, int64_t P,
                                                         const int32_t* __restrict__ pad, const int32_t* __restrict__ tot,
                                                         const int32_t* __restrict__ block_expert,
                                                         int32_t* __restrict__ sorted_rows) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= P) return;
  const int e = block_expert[p / bm];
  if (e < 0 || p - pad[e] >= tot[e]) sorted_rows[p] = (int32_t)R;
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
  int32_t* tot = pad + a.num_local + 1;
  const int64_t P = padded_rows(a.R, a.num_local, a.block_m);
  if (nch > 0) {
    hipLaunchKernelGGL(align_count_kernel, dim3(nch), dim3(kAlignChunk), (size_t)(kAlignChunk / 64) * (a.num_local + 2),
                       st, a.local_expert,
                       a.R, a.num_local, rank, chunk);
    hipLaunchKernelGGL(align_keyscan_kernel, dim3((a.num_local + 255) / 256), dim3(256), 0, st, a.num_local, nch,
                       chunk, tot);
  } else {
    hipLaunchKernelGGL(align_zero_kernel, dim3((a.num_local + 255) / 256), dim3(256), 0, st, a.num_local, tot);
  }
  hipLaunchKernelGGL(align_padscan_kernel, dim3(1), dim3(1024), (size_t)(a.num_local + 1) * 4, st, a.num_local,
                     a.block_m, P / a.block_m, tot, pad, a.block_expert, a.num_padded);
  if (P > 0)
    hipLaunchKernelGGL(align_fill_kernel, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, st, a.R, a.num_local,
                       a.block_m, P, pad, tot, a.block_expert, a.sorted_rows);
  if (nch > 0)
    hipLaunchKernelGGL(align_scatter_kernel, dim3(nch), dim3(kAlignChunk), 0, st, a.local_expert, a.R, a.num_local,
                       rank, chunk, pad, a.sorted_rows);
  return hipGetLastError();
}

// ---------------------------------------------------------------- grouped GEMM
// Block: 256 threads (4 waves) x 128 sorted rows (one expert) x 256 weight rows, K in steps of 64 (one
// quantisation group). Each wave owns 64 weight rows (four 16-column MFMA B fragments) for all 128 rows of the
// block, so every weight of the block is dequantized exactly once, by the wave that multiplies it, straight into
// MFMA B registers. Gate/up: wave w owns gate rows n0 + 32 w .. + 31 (fragments 0, 1) and the same up rows
// (fragments 2, 3), so silu(g) * u is formed in registers. Down: wave w owns rows n0 + 64 w .. + 63. Column n of
// fragment j is the wave's weight row 4 n + j (gate/up: h column 2 n + (j & 1)), so a lane's fragments hold adjacent
// outputs and the epilogues store 16-byte pieces.
// K order inside a group: lane quad q (lane >> 4) holds packed words 2q, 2q + 1 of its weight row's group
// (elements 16 q .. 16 q + 15); MFMA slice s (0, 1) uses word 2q + s, i.e. elements 16 q + 8 s .. + 7, and the A
// fragment of slice s holds the same elements of each row. A dot product does not depend on which MFMA lanes its
// K terms go to, only on the accumulation, which the MFMA unit fixes.
// Memory paths:
//  * A (activations for gate/up, h for down): global -> registers -> LDS (two LDS stages); each load instruction
//    covers 8 whole 128-byte rows (8 lanes per row), and only the live rows are loaded. The register-staged path
//    keeps every wait precise (a direct-to-LDS load in flight makes the compiler wait for it before any LDS read).
//  * Scales and biases of the block's 256 weight rows for the whole K range: read once, coalesced, into LDS as
//    (s, b) dword pairs.
//  * Packed weights: 8 bytes per lane per K step straight into registers.
//  * The loads of a step are issued PD steps ahead of its MFMAs (register slots; see gemm_loop).
// 16-byte chunk c of A row m sits at chunk position a_pos(m, c) of the row's 128 bytes, so the 16 rows one MFMA
// operand read touches (and each group of 8 of them) fall on distinct banks. Rows past the block's valid count
// get no MFMAs beyond the last 32-row pair of fragments that holds a valid row.
constexpr int kBM = 128;
constexpr int kBK = 64;
constexpr int kAStage = kBM * kBK * 2;  // 16 KB
constexpr int kGateUpTileN = 128;       // gate (and up) rows per block
constexpr int kDownTileN = 256;         // down rows per block
constexpr int kBN = 256;                // weight rows per block (both kernels)
constexpr int kMaxGroups = 64;          // K / 64 <= 64 (H, I <= 4096)
// Dynamic LDS of one block: the two A stages, then the (s, b) table of kBN rows x (G + 1) dwords (G = K / 64; the
// extra dword per row staggers the banks). Two blocks per CU fit for G <= 60.
static size_t gemm_lds_bytes(int G) { return 2 * (size_t)kAStage + (size_t)kBN * (G + 1) * 4; }
constexpr size_t kGemmLdsMax = 2 * kAStage + (size_t)kBN * (kMaxGroups + 1) * 4;

typedef __bf16 ss_bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t ss_u32x2 __attribute__((ext_vector_type(2)));

// bf16 pair (lo, hi) rounded to nearest even by the hardware conversion.
SS_DEV uint32_t cvt_pk_bf16(float lo, float hi) {
  const ss_bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// 8 nibbles (element e at bits 4e) -> bf16(q * s + b) x 8 as an MFMA operand (pairs low element first).
// A nibble q in a byte of its own is the OCP fp8 e4m3 value q * 2^-9 exactly (q < 8 subnormal, q >= 8 with
// exponent field 1), so one v_cvt_pk_f32_fp8 turns two nibbles into fp32. s9 = s * 2^9 (exact), hence
// (q * 2^-9) * s9 = q * s exactly and the fused multiply-add rounds q * s + b once, as the reference's fp32
// q * s + b does (q * s is exact in fp32: 4-bit by 8-bit mantissas); then one rounding to bf16. (A scale of 2^119
// or more would overflow s9; bf16 weight scales are far below that.) The masks are opaque to the compiler, so it
// keeps them as two v_and_b32 instead of folding them into per-nibble bit-field extracts.
SS_DEV uint32_t and_opaque(uint32_t x, uint32_t m) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "s"(m), "v"(x));
  return r;
}
SS_DEV ss_u32x4 dequant8(uint32_t w, float s9, float bi) {
  const int lo = (int)and_opaque(w, 0x0F0F0F0Fu), hi = (int)and_opaque(w >> 4, 0x0F0F0F0Fu);  // n0 n2 n4 n6 / n1 n3 n5 n7
  const auto e02 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false), e46 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
  const auto e13 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false), e57 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
  ss_u32x4 r;
  r.x = cvt_pk_bf16(__builtin_fmaf(e02[0], s9, bi), __builtin_fmaf(e13[0], s9, bi));
  r.y = cvt_pk_bf16(__builtin_fmaf(e02[1], s9, bi), __builtin_fmaf(e13[1], s9, bi));
  r.z = cvt_pk_bf16(__builtin_fmaf(e46[0], s9, bi), __builtin_fmaf(e57[0], s9, bi));
  r.w = cvt_pk_bf16(__builtin_fmaf(e46[1], s9, bi), __builtin_fmaf(e57[1], s9, bi));
  return r;
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
  uint64_t* trace;                 // per-block stamps (start, end, expert << 32 | valid rows, XCC << 32 | HW_ID) or null
};

// LDS barrier for data exchanged through LDS only: waits for this wave's LDS operations, not for its global loads
// in flight (which a workgroup-scope fence would also wait for).
SS_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block index -> (M block, N tile). The plan's M blocks are dealt round-robin to the XCDs (workgroup b runs on XCD
// b % 8), in plan order, so every XCD gets an even share of the heavy and the light experts' blocks (the mix also
// pairs MFMA-bound full blocks with VALU-bound partial ones on a CU); each XCD takes all N tiles of one M block in a
// row (they share its activation rows in the XCD's L2). Measured on MI355X at BASELINE config 3, this beats both
// contiguous per-XCD ranges of the plan (XCDs ending 140-180 us apart) and a full-blocks-first order (full blocks
// sharing a CU slow each other down).
SS_DEV bool xcd_tile(int mb, int nt, int& pid_m, int& pid_n) {
  const int b = blockIdx.x, x = b & 7, s = b >> 3;
  const int sm = s / nt;
  pid_m = sm * 8 + x;
  pid_n = s - sm * nt;
  return pid_m < mb;
}

// 16-byte chunk c of A row m sits at chunk position a_pos(m, c) of the row's 128 bytes.
SS_DEV int a_pos(int m, int c) { return c ^ (m & 7) ^ ((m >> 3) & 1); }

// Local index of weight row (fragment j, lane row n) of wave w: 64 w + 16 j + n; the (s, b) table row stride is
// G + 1 dwords, so 16 consecutive rows at one group fall on distinct banks.

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>), in order.
template <typename F, int... I>
SS_DEV void ss_static_for_seq(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
SS_DEV void ss_static_for(F&& f) {
  ss_static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// The K loop for NF live 16-row fragments (fragments NF .. 7 are all padding and get no loads or MFMAs), with the
// global loads of step k + PD issued at the end of step k into register slot k % PD: the packed weights are PD steps
// ahead of their use, the A rows PD - 1 steps ahead of their LDS store (two LDS stages). Blocks with fewer live rows
// hold fewer accumulators, so they afford a deeper register ring (their steps are shorter, so they need it more).
// Thread t stages A rows t / 8 + 32 c (c < NF / 2), 16-byte chunk t % 8.
template <int NF, int PD>
SS_DEV void gemm_loop(uint8_t* lds, const uint32_t* sbt, int nsteps, int aoff0, int aoff1, ss_f32x4 (&acc)[8][4],
                      const uint16_t* const (&asrc)[4], int arow0, int achunk, const uint8_t* wbase,
                      const int64_t (&wc)[4], uint32_t lw, int sb_lane, int sb_stride) {
  static_assert(PD % 2 == 0, "the LDS stage of step k is k & 1 = (k % PD) & 1");
  constexpr int NA = NF / 2;
  uint4 areg[PD][NA];
  ss_u32x2 bw[PD][4];
  // Loads of step k (the last step again past the end: never used) into register slot S.
  auto load = [&](int k, auto slot_c) {
    constexpr int S = decltype(slot_c)::value;
    const int kk = k < nsteps ? k : nsteps - 1;
#pragma unroll
    for (int c = 0; c < NA; ++c) areg[S][c] = ldg16(asrc[c] + (size_t)kk * kBK);
#pragma unroll
    for (int j = 0; j < 4; ++j) bw[S][j] = *(const SS_G ss_u32x2*)(wbase + wc[j] + lw + 32 * kk);
  };
  auto store_a = [&](auto slot_c, int stage) {
    constexpr int S = decltype(slot_c)::value;
#pragma unroll
    for (int c = 0; c < NA; ++c) {
      const int m = arow0 + 32 * c;
      *reinterpret_cast<uint4*>(lds + stage * kAStage + m * (kBK * 2) + 16 * a_pos(m, achunk)) = areg[S][c];
    }
  };
  ss_static_for<PD>([&](auto p) { load(decltype(p)::value, p); });
  store_a(std::integral_constant<int, 0>{}, 0);
  lds_barrier();
  // One K step from register slot S (= k % PD) and LDS stage S & 1; then A of step k + 1 into the other stage, the
  // loads of step k + PD into slot S, and the barrier.
  auto step = [&](int k, auto slot_c) {
    constexpr int S = decltype(slot_c)::value;
    const uint8_t* st = lds + (S & 1) * kAStage;
    float sc[4], bi[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t sb = sbt[sb_lane + j * sb_stride + k];
      sc[j] = __uint_as_float(sb << 16) * 512.f;  // s * 2^9, exact
      bi[j] = __uint_as_float(sb & 0xFFFF0000u);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      ss_u32x4 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = dequant8(s ? bw[S][j].y : bw[S][j].x, sc[j], bi[j]);
      const uint8_t* ap = st + (s ? aoff1 : aoff0);
      // A fragments in batches of up to four: one LDS wait per batch. The scheduling barriers keep one slice's
      // operands live at a time (the register budget of two waves per SIMD); the two waves of a SIMD overlap one
      // wave's dequantization with the other's MFMAs.
#pragma unroll
      for (int i0 = 0; i0 < NF; i0 += 4) {
        constexpr int NB = NF < 4 ? NF : 4;
        ss_u32x4 av[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i)
          if (i0 + i < NF) av[i] = *reinterpret_cast<const ss_u32x4*>(ap + (i0 + i) * 16 * (kBK * 2));
#pragma unroll
        for (int i = 0; i < NB; ++i)
          if (i0 + i < NF)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i0 + i][j] = ss_mfma(av[i], bf[j], acc[i0 + i][j]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    store_a(std::integral_constant<int, (S + 1) % PD>{}, (S & 1) ^ 1);
    load(k + PD, slot_c);
    lds_barrier();
  };
  // Whole groups of PD steps with no guard inside, so that every path into the loop head has the same loads in
  // flight (a guarded step gave the head a second path without the last slot's loads, and the compiler then waited
  // for every load at the head: the next steps' prefetches included); the nsteps % PD last steps after it.
  const int nfull = nsteps - nsteps % PD;
#pragma unroll 1
  for (int k = 0; k < nfull; k += PD) ss_static_for<PD>([&](auto u) { step(k + decltype(u)::value, u); });
  if (nfull < nsteps)
    ss_static_for<PD>([&](auto u) {
      if (nfull + decltype(u)::value < nsteps) step(nfull + decltype(u)::value, u);
    });
}

template <bool GATE_UP>
__global__ __launch_bounds__(256, 2) void prefill_gemm_kernel(GemmArgs g, int nt) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ int64_t a_off[kBM];  // element offset of each row's A operand, -1 for a zero row
  __shared__ int out_row[kBM];
  __shared__ float wt_s[kBM];
  uint32_t* sbt = reinterpret_cast<uint32_t*>(lds + 2 * kAStage);  // [kBN][G + 1] (s | b << 16)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int mb = g.num_padded[0] / kBM;
  int pid_m, pid_n;
  if (!xcd_tile(mb, nt, pid_m, pid_n)) return;
  const int e = g.block_expert[pid_m];
  if (e < 0) return;
  const uint64_t t_start = g.trace ? __builtin_amdgcn_s_memrealtime() : 0;
  const uint8_t* base = reinterpret_cast<const uint8_t*>(g.group_ptr[e]);
  const int kdim = GATE_UP ? g.H : g.I;
  const int G = kdim / 64, sb_stride = G + 1;
  bool valid = false;
  if (tid < kBM) {
    const int r = g.sorted_rows[(int64_t)pid_m * kBM + tid];
    valid = r < g.R;
    int64_t off = -1;  // -1: a zero row (a token outside [0, T))
    if (valid) {
      if (GATE_UP) {
        const int t = g.row_token[r];
        if (t >= 0 && t < g.T) off = (int64_t)t * g.H;
      } else {
        off = (int64_t)r * g.I;
      }
    }
    a_off[tid] = off;
    out_row[tid] = valid ? r : -1;
    if (!GATE_UP) wt_s[tid] = valid ? g.row_weight[r] : 0.f;
  }
  // Column n of B fragment j of wave w is local weight row lr = 64 w + 4 n + j, so a lane's four fragments hold four
  // adjacent outputs. Global weight row of local row lr and its piece: gate/up local rows map to gate rows (j < 2)
  // or up rows (j >= 2) n0 + 32 w + 2 n + (j & 1), so g and u of one h column sit in one lane (fragments j and
  // j + 2) and its two h columns are adjacent; down local rows are rows n0 + lr.
  auto grow = [&](int lr, bool& up) -> int64_t {
    if (GATE_UP) {
      const int ww = lr >> 6, nn = (lr >> 2) & 15, j = lr & 3;
      up = j >= 2;
      return (int64_t)pid_n * kGateUpTileN + 32 * ww + 2 * nn + (j & 1);
    }
    up = false;
    return (int64_t)pid_n * kDownTileN + lr;
  };
  // (s, b) table: thread t fills local rows t (one row, all G groups; 16-byte loads of 8 groups).
  {
    bool up;
    const int64_t row = grow(tid, up);
    const uint8_t* srow = base + (up ? g.s2_off : g.s_off) + row * G * 2;
    const uint8_t* brow = base + (up ? g.b2_off : g.b_off) + row * G * 2;
    uint32_t* dst = sbt + tid * sb_stride;
    if (G % 8 == 0) {
      for (int c = 0; c < G; c += 8) {
        const uint4 sv = ldg16(srow + 2 * c), bv = ldg16(brow + 2 * c);
        const uint32_t s4[4] = {sv.x, sv.y, sv.z, sv.w}, b4[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          dst[c + 2 * d] = (s4[d] & 0xFFFFu) | (b4[d] << 16);
          dst[c + 2 * d + 1] = (s4[d] >> 16) | (b4[d] & 0xFFFF0000u);
        }
      }
    } else {  // G is even (K is a multiple of 128): two groups per dword
      for (int c = 0; c < G; c += 2) {
        const uint32_t sv = *(const SS_G uint32_t*)(srow + 2 * c), bv = *(const SS_G uint32_t*)(brow + 2 * c);
        dst[c] = (sv & 0xFFFFu) | (bv << 16);
        dst[c + 1] = (sv >> 16) | (bv & 0xFFFF0000u);
      }
    }
  }
  // Valid rows are a prefix of the block (each expert's rows come first in its padded range).
  const int nvalid = __syncthreads_count(valid);

  // A staging: load instruction c of thread t covers row arow0 + 32 c (arow0 = t / 8), 16-byte chunk t % 8 (each
  // instruction of a wave covers 8 whole 128-byte rows). A padding row or a zero row reads the first kdim elements
  // of the expert record (always present): a padding row's MFMA output row is never stored, and a zero row's h is
  // stored as 0 (silu(0) * 0).
  const int arow0 = tid >> 3, achunk = tid & 7;
  const uint16_t* asrc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int m = arow0 + 32 * c;
    const int64_t off = a_off[m];
    asrc[c] = (m < nvalid && off >= 0 ? g.a + off : reinterpret_cast<const uint16_t*>(base)) + 8 * achunk;
  }
  // B: lane (n = lane & 15, q = lane >> 4) of fragment j reads words 2q, 2q + 1 of its row's group.
  const int n = lane & 15, q = lane >> 4;
  const int64_t wrow_b = kdim / 2;
  int64_t wc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bool up;
    const int64_t row0 = grow(64 * w + j, up);
    wc[j] = (up ? g.w2_off : g.w_off) + row0 * wrow_b;
  }
  // lane row n is weight row row0 + 2 n (gate/up) or row0 + 4 n (down) of its fragment
  const uint32_t lw = (uint32_t)((GATE_UP ? 2 : 4) * n * wrow_b + 8 * q);
  const int sb_lane = (64 * w + 4 * n) * sb_stride;

  ss_f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = ss_f32x4{0.f, 0.f, 0.f, 0.f};

  // Lane offsets of the A fragments (slice s): row 16 i + n, chunk 2q + s (a_pos depends on n only).
  const int aoff0 = n * (kBK * 2) + 16 * a_pos(n, 2 * q);
  const int aoff1 = n * (kBK * 2) + 16 * a_pos(n, 2 * q + 1);
  const int nsteps = kdim / kBK;  // even: kdim is a multiple of 128
  const int nf2 = (nvalid + 31) >> 5;  // live fragment pairs (1..4)
  if (nf2 >= 4)
    gemm_loop<8, 2>(lds, sbt, nsteps, aoff0, aoff1, acc, asrc, arow0, achunk, base, wc, lw, sb_lane, sb_stride);
  else if (nf2 == 3)
    gemm_loop<6, 2>(lds, sbt, nsteps, aoff0, aoff1, acc, asrc, arow0, achunk, base, wc, lw, sb_lane, sb_stride);
  else if (nf2 == 2)
    gemm_loop<4, 4>(lds, sbt, nsteps, aoff0, aoff1, acc, asrc, arow0, achunk, base, wc, lw, sb_lane, sb_stride);
  else
    gemm_loop<2, 4>(lds, sbt, nsteps, aoff0, aoff1, acc, asrc, arow0, achunk, base, wc, lw, sb_lane, sb_stride);

  if (GATE_UP) {
    // h = bf16(silu(g) * u) of the live fragments into an LDS tile [128 rows][128 columns] (a lane's two adjacent
    // columns as one dword), then 16-byte row-contiguous stores of the valid rows.
    uint32_t* ht = reinterpret_cast<uint32_t*>(lds);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i >= 2 * nf2) break;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * i + 4 * q + r;
        const bool live = a_off[m] >= 0;
        uint32_t hp = 0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float gv = acc[i][j][r], uv = acc[i][j + 2][r];
          // silu with the hardware exp2 and reciprocal (about 1 ulp each): h is rounded to bf16 next, which
          // hides fp32 differences of a few ulp except at a rounding tie.
          const float sig = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(gv * -1.4426950408889634f));
          const float hv = live ? gv * sig * uv : 0.f;
          hp |= (uint32_t)ss_f32_to_bf16(hv) << (16 * j);
        }
        ht[m * (kGateUpTileN / 2) + 16 * w + n] = hp;
      }
    }
    lds_barrier();
    const int n0 = pid_n * kGateUpTileN;
#pragma unroll
    for (int u = 0; u < (kBM * kGateUpTileN * 2) / (16 * 256); ++u) {
      const int id = u * 256 + tid;
      const int m = id >> 4, cc = id & 15;
      if (m >= nvalid) break;
      const int r = out_row[m];
      if (r >= 0) {
        const uint4 v = *reinterpret_cast<const uint4*>(ht + m * (kGateUpTileN / 2) + 4 * cc);
        stg16(g.h + (int64_t)r * g.I + n0 + 8 * cc, v);
      }
    }
  } else {
    // A lane's four fragments are four adjacent outputs: one 16-byte store per row.
    const int n0 = pid_n * kDownTileN + 64 * w + 4 * n;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i >= 2 * nf2) break;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * i + 4 * q + r;
        const int orow = out_row[m];
        if (orow >= 0) {
          const float wt = wt_s[m];
          const uint4 v = make_uint4(__float_as_uint(acc[i][0][r] * wt), __float_as_uint(acc[i][1][r] * wt),
                                     __float_as_uint(acc[i][2][r] * wt), __float_as_uint(acc[i][3][r] * wt));
          stg16(g.out_rows + (int64_t)orow * g.H + n0, v);
        }
      }
    }
  }
  // Diagnostics: gate/up blocks at entries [0, 8192), down blocks at [8192, 16384), four per block.
  if (g.trace && tid == 0) {
    const size_t at = (GATE_UP ? 0 : 8192) + 4 * (size_t)blockIdx.x;
    if (at + 4 <= (GATE_UP ? 8192u : 16384u)) {
      const uint32_t hw = __builtin_amdgcn_s_getreg(4 | (31 << 11));   // HW_ID
      const uint32_t xcc = __builtin_amdgcn_s_getreg(20 | (31 << 11)); // XCC_ID
      g.trace[at] = t_start;
      g.trace[at + 1] = __builtin_amdgcn_s_memrealtime();
      g.trace[at + 2] = ((uint64_t)(uint32_t)e << 32) | (uint32_t)nvalid;
      g.trace[at + 3] = ((uint64_t)xcc << 32) | hw;
    }
  }
}

hipError_t launch_prefill_gemm(const PrefillArgs& p, hipStream_t st) {
  static_assert(kBM == kPrefillBlockM, "one block size for the plan and the GEMM");
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
  g.trace = p.trace;
  g.a = p.x;
  g.w_off = rec.gw;
  g.s_off = rec.gs;
  g.b_off = rec.gb;
  g.w2_off = rec.uw;
  g.s2_off = rec.us;
  g.b2_off = rec.ub;
  // Grids cover the plan's upper bound of M blocks (rounded up to a multiple of 8) times the N tiles; blocks past
  // the device-side count exit at once.
  KernelCfg cfg;
  hipError_t e = kernel_cfg(reinterpret_cast<const void*>(prefill_gemm_kernel<true>), 256, kGemmLdsMax, &cfg);
  if (e == hipSuccess)
    e = kernel_cfg(reinterpret_cast<const void*>(prefill_gemm_kernel<false>), 256, kGemmLdsMax, &cfg);
  if (e != hipSuccess) return e;
  const int64_t mb = P / kBM;
  const int nt_gu = p.I / kGateUpTileN, nt_d = p.H / kDownTileN;
  auto grid_of = [&](int nt) { return (unsigned)(8 * nt * ((mb + 7) / 8)); };
  hipLaunchKernelGGL(prefill_gemm_kernel<true>, dim3(grid_of(nt_gu)), dim3(256), gemm_lds_bytes(p.H / 64), st, g,
                     nt_gu);
  g.a = p.h_buf;
  g.w_off = rec.dw;
  g.s_off = rec.ds;
  g.b_off = rec.db;
  hipLaunchKernelGGL(prefill_gemm_kernel<false>, dim3(grid_of(nt_d)), dim3(256), gemm_lds_bytes(p.I / 64), st, g,
                     nt_d);
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
