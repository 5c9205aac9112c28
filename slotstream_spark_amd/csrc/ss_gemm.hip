// Dense bf16 GEMM C = bf16(A B^T) for the prefill's plain projections (lin on bf16 weights over a prompt chunk,
// model/layers.py:62-76): the router logits (x W_gate^T), the shared expert's gate/up/gate-logit rows
// (x [W_g; W_u; w_sg]^T) and its down projection (hs W_d^T). A [M][K] and B [N][K] are row-major with K contiguous
// (the torch layout of activations and nn.Linear weights), the dot is accumulated in fp32 by the MFMA unit and
// rounded once to bf16.
//
// Block tile (2 WM 16) x (2 WN 16): four waves in a 2 x 2 arrangement, each owning WM x WN 16 x 16 output fragments
// (v_mfma_f32_16x16x32_bf16). K advances in steps of 64: the A and B tiles of a step go global -> registers -> LDS,
// the global loads four steps ahead of their LDS stores (four register slots) and the LDS double-buffered, each load
// instruction covering whole 128-byte row pieces. In LDS the 16-byte chunk c of tile row m sits at position
// c ^ (m & 7) ^ ((m >> 3) & 1) of the row's 128 bytes, so the 16 rows one MFMA operand read touches fall on distinct
// banks. K order inside a step: lane quad q (lane >> 4) of a fragment
// holds elements 16 q + 8 s .. + 7 of its row for MFMA slice s (0, 1), for A and B alike.
// Rows of A past M and of B past N read row 0 (a valid address) and their results are not stored.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

namespace {

constexpr int kGK = 64;    // K per step
constexpr int kSlots = 4;  // register slots of global loads in flight (K is a multiple of kGK * kSlots)

SS_DEV int chunk_pos(int m, int c) { return c ^ (m & 7) ^ ((m >> 3) & 1); }

SS_DEV void gemm_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

struct DenseGemmArgs {
  const uint16_t* a;  // [M][lda]
  const uint16_t* b;  // [N][ldb]
  uint16_t* c;        // [M][ldc]
  int M, N, K;
  int64_t lda, ldb, ldc;
  int tiles_n, nsteps, tiles, tiles_per_xcd;
};

template <int WM, int WN>
__global__ __launch_bounds__(256) void dense_gemm_kernel(DenseGemmArgs g) {
  constexpr int BM = 2 * WM * 16, BN = 2 * WN * 16;
  constexpr int CA = BM * 8 / 256, CB = BN * 8 / 256;  // 16-byte chunks per thread per step
  static_assert(CA >= 1 && CB >= 1, "whole chunks per thread");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][(BM + BN) * 128];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  // Workgroups are dealt to the 8 XCDs round-robin; XCD x takes the contiguous tile range [x per, (x + 1) per), so
  // the N tiles of one M tile share an XCD and its L2 holds that A tile for all of them.
  const int per = g.tiles_per_xcd, L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (L >= g.tiles) return;  // whole workgroup, before any barrier
  const int tm = L / g.tiles_n, tn = L - tm * g.tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;

  // This thread's chunks: tile row r = (tid >> 3) + 32 i, chunk c = tid & 7.
  const int cr = tid >> 3, cc = tid & 7;
  const uint16_t* asrc[CA];
  const uint16_t* bsrc[CB];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int m = m0 + cr + 32 * i;
    asrc[i] = g.a + (size_t)(m < g.M ? m : 0) * g.lda + 8 * cc;
  }
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    const int n = n0 + cr + 32 * i;
    bsrc[i] = g.b + (size_t)(n < g.N ? n : 0) * g.ldb + 8 * cc;
  }
  // kSlots register slots: the global loads of step k are issued kSlots steps before its LDS store, which precedes
  // its MFMAs by one step. The loop body is straight-line over kSlots steps (nsteps is a multiple of kSlots), so the
  // wait before each store covers exactly the loads of that step.
  uint4 ar[kSlots][CA], br[kSlots][CB];
  auto load = [&](int k, auto slot_c) {
    constexpr int S = decltype(slot_c)::value;
    const int kk = k < g.nsteps ? k : g.nsteps - 1;  // past the end: reload the last step (stored, never read)
#pragma unroll
    for (int i = 0; i < CA; ++i) ar[S][i] = ldg16(asrc[i] + (size_t)kk * kGK);
#pragma unroll
    for (int i = 0; i < CB; ++i) br[S][i] = ldg16(bsrc[i] + (size_t)kk * kGK);
  };
  auto store = [&](int st, auto slot_c) {
    constexpr int S = decltype(slot_c)::value;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int r = cr + 32 * i;
      *reinterpret_cast<uint4*>(&lds[st][r * 128 + 16 * chunk_pos(r, cc)]) = ar[S][i];
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int r = BM + cr + 32 * i;
      *reinterpret_cast<uint4*>(&lds[st][r * 128 + 16 * chunk_pos(r, cc)]) = br[S][i];
    }
  };

  const int n = lane & 15, q = lane >> 4;
  ss_f32x4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = ss_f32x4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = g.nsteps;
  // Step 0 into LDS buffer 0; steps 1 .. kSlots into the slots (step s in slot s % kSlots).
  load(0, std::integral_constant<int, 0>{});
  store(0, std::integral_constant<int, 0>{});
  load(1, std::integral_constant<int, 1 % kSlots>{});
  load(2, std::integral_constant<int, 2 % kSlots>{});
  load(3, std::integral_constant<int, 3 % kSlots>{});
  load(4, std::integral_constant<int, 4 % kSlots>{});
  gemm_barrier();
  // Step k: MFMAs on LDS buffer k & 1, then step k + 1 (slot (k + 1) % kSlots) into the other buffer and step
  // k + 1 + kSlots into that slot.
  auto step = [&](int k, auto next_c) {
    const uint8_t* st = lds[k & 1];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      ss_u32x4 av[WM], bv[WN];
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        const int r = wm * WM * 16 + 16 * i + n;
        av[i] = *reinterpret_cast<const ss_u32x4*>(st + r * 128 + 16 * chunk_pos(r, 2 * q + s));
      }
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int r = BM + wn * WN * 16 + 16 * j + n;
        bv[j] = *reinterpret_cast<const ss_u32x4*>(st + r * 128 + 16 * chunk_pos(r, 2 * q + s));
      }
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = ss_mfma(av[i], bv[j], acc[i][j]);
    }
    store((k + 1) & 1, next_c);
    load(k + 1 + kSlots, next_c);
    gemm_barrier();
  };
#pragma unroll 1
  for (int k = 0; k < nsteps; k += kSlots) {
    step(k, std::integral_constant<int, 1 % kSlots>{});
    step(k + 1, std::integral_constant<int, 2 % kSlots>{});
    step(k + 2, std::integral_constant<int, 3 % kSlots>{});
    step(k + 3, std::integral_constant<int, 4 % kSlots>{});
  }
  // acc[i][j][r]: row 16 i + 4 q + r, column 16 j + n of the wave's fragment grid. The block's C tile goes through
  // LDS (the operand buffers are dead after the last barrier) so that it leaves in 16-byte row pieces.
  uint16_t* ct = reinterpret_cast<uint16_t*>(&lds[0][0]);
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int col = wn * WN * 16 + 16 * j + n;
#pragma unroll
      for (int r = 0; r < 4; ++r) ct[(wm * WM * 16 + 16 * i + 4 * q + r) * BN + col] = (uint16_t)ss_f32_to_bf16(acc[i][j][r]);
    }
  gemm_barrier();
  constexpr int CPR = BN / 8;  // 16-byte pieces per tile row
#pragma unroll
  for (int idx = tid; idx < BM * CPR; idx += 256) {
    const int r = idx / CPR, c8 = idx - r * CPR;
    const int row = m0 + r, col = n0 + 8 * c8;
    if (row < g.M && col < g.N)
      *reinterpret_cast<uint4*>(g.c + (size_t)row * g.ldc + col) = *reinterpret_cast<const uint4*>(ct + r * BN + 8 * c8);
  }
}

template <int WM, int WN>
hipError_t launch_tiles(const DenseGemmArgs& g0, hipStream_t st) {
  DenseGemmArgs g = g0;
  constexpr int BM = 2 * WM * 16, BN = 2 * WN * 16;
  g.tiles_n = (g.N + BN - 1) / BN;
  g.tiles = ((g.M + BM - 1) / BM) * g.tiles_n;
  g.tiles_per_xcd = (g.tiles + 7) / 8;
  hipLaunchKernelGGL((dense_gemm_kernel<WM, WN>), dim3((unsigned)(8 * g.tiles_per_xcd)), dim3(256), 0, st, g);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_dense_gemm(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c, int64_t ldc,
                             int M, int N, int K, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  DenseGemmArgs g{a, b, c, M, N, K, lda, ldb, ldc, 0, K / kGK, 0, 0};
  // 64 x 64 tiles: measured on MI355X at the prefill's three shapes, they beat 64 x 128, 128 x 64 and 128 x 128 tiles
  // or tie with them (the steps are bound by load latency, and the smaller tile gives more workgroups).
  return launch_tiles<2, 2>(g, st);
}

}  // namespace ss
