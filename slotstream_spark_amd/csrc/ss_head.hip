// Dense operations of the MTP draft head without its attention (engine/mtp.py:194-227, model/layers.py:190-198):
// RMSNorm over groups, bf16 GEMV with the elementwise op that follows each `lin` of the head fused into its store,
// the hyper-connection mean and residual, and a row gather by device index (the embedding lookup of a drafted token,
// the kept row of a verify round). Every op is row-independent and has one fixed reduction order, so an S-row call
// equals S one-row calls bit for bit, and the CPU restatement reproduces it exactly.
#include <hip/hip_runtime.h>

#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

namespace {

SS_DEV float lo16(uint32_t v) { return ss_bf16_to_f32(v & 0xFFFFu); }
SS_DEV float hi16(uint32_t v) { return ss_bf16_to_f32(v >> 16); }

// One wave per (row, group): lane l sums x^2 over the 8-element chunks l, l + 64, ... of the group with fmaf from 0,
// then the xor butterfly; r = 1 / sqrt(sum / G + eps); out = bf16((x * r) * w).
__global__ __launch_bounds__(256) void rmsnorm_groups_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ w, float eps, int64_t nseg,
                                                             int n, int G, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t seg = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (seg >= nseg) return;  // whole waves; no workgroup barrier follows
  const int per_row = n / G;
  const int64_t row = seg / per_row;
  const int g = (int)(seg - row * per_row);
  const int64_t base = row * n + (int64_t)g * G;
  const uint4* xs = reinterpret_cast<const uint4*>(x + base);
  const uint4* ws = w ? reinterpret_cast<const uint4*>(w + (int64_t)g * G) : nullptr;
  uint4* os = reinterpret_cast<uint4*>(out + base);
  const int g8 = G >> 3;
  // Chunks in batches of kUB whose loads are all issued before their arithmetic (one round trip per batch); the
  // arithmetic keeps the lane's chunk order.
  constexpr int kUB = 8;
  float acc = 0.f;
  auto square = [&](const uint4& a) {
    const uint32_t v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float e0 = lo16(v[c]), e1 = hi16(v[c]);
      acc = fmaf(e0, e0, acc);
      acc = fmaf(e1, e1, acc);
    }
  };
  int k8 = lane;
  for (; k8 + 64 * (kUB - 1) < g8; k8 += 64 * kUB) {
    uint4 a[kUB];
#pragma unroll
    for (int u = 0; u < kUB; ++u) a[u] = xs[k8 + 64 * u];
#pragma unroll
    for (int u = 0; u < kUB; ++u) square(a[u]);
  }
  for (; k8 < g8; k8 += 64) square(xs[k8]);
  const float r = 1.f / sqrtf(ss_wave_sum(acc) / (float)G + eps);
  auto scale = [&](int k, const uint4& a, const uint4& b) {
    const uint32_t v[4] = {a.x, a.y, a.z, a.w};
    const uint32_t wv[4] = {b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      o[c] = ss_f32_to_bf16((lo16(v[c]) * r) * lo16(wv[c])) | (ss_f32_to_bf16((hi16(v[c]) * r) * hi16(wv[c])) << 16);
    os[k] = make_uint4(o[0], o[1], o[2], o[3]);
  };
  const uint4 one = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);  // bf16 1.0 pairs
  k8 = lane;
  for (; k8 + 64 * (kUB - 1) < g8; k8 += 64 * kUB) {
    uint4 a[kUB], b[kUB];
#pragma unroll
    for (int u = 0; u < kUB; ++u) {
      a[u] = xs[k8 + 64 * u];
      b[u] = ws ? ws[k8 + 64 * u] : one;
    }
#pragma unroll
    for (int u = 0; u < kUB; ++u) scale(k8 + 64 * u, a[u], b[u]);
  }
  for (; k8 < g8; k8 += 64) scale(k8, xs[k8], ws ? ws[k8] : one);
}

constexpr int kDR = 4;  // x rows per GEMV launch

struct DenseEpiArgs {
  const uint16_t* x;    // [R][K] (this launch's rows)
  const uint16_t* w;    // [N][K]
  uint16_t* out;        // [R][N]
  const uint16_t* add;  // SSMOE_EPI_ADD: bf16 rows added after the rounding, row (row0 + r) / add_div
  int R, K, N, epi, row0, add_div;
  float hc;
};

SS_DEV float sigmoid_f(float v) { return 1.0f / (1.0f + ss_expf(-v)); }

// The op after the GEMV, on the fp32 dot d, with torch's bf16 rounding after every step (the head's tensors are bf16).
SS_DEV uint32_t epilogue(float d, const DenseEpiArgs& a, int r, int n) {
  const float v = ss_round_bf16(d);
  switch (a.epi) {
    case SSMOE_EPI_ADD: {
      const float e = ss_bf16_to_f32(a.add[(size_t)((a.row0 + r) / a.add_div) * a.N + n]);
      return ss_f32_to_bf16(e + v);
    }
    case SSMOE_EPI_SILU_DIV: {
      const float u = ss_round_bf16(v / a.hc);
      return ss_f32_to_bf16(u / (1.0f + ss_expf(-u)));
    }
    case SSMOE_EPI_SIGMOID:
      return ss_f32_to_bf16(sigmoid_f(v));
    case SSMOE_EPI_INJECT:
      return ss_f32_to_bf16(2.0f * ss_round_bf16(sigmoid_f(ss_round_bf16(v / a.hc))));
    default:
      return ss_f32_to_bf16(v);
  }
}

// One wave per weight row n, up to 4 x rows: lane l accumulates the 8-element chunks l, l + 64, ... of row n against
// each x row with fmaf from 0, then the xor butterfly (the order of the dense router rows). Lane r stores x row r.
__global__ __launch_bounds__(256) void dense_epi_kernel(DenseEpiArgs a) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= a.N) return;  // whole waves; no workgroup barrier follows
  const int k8n = a.K >> 3;
  const uint4* wr = reinterpret_cast<const uint4*>(a.w + (size_t)n * a.K);
  float acc[kDR] = {0.f, 0.f, 0.f, 0.f};
  // One chunk of every row into acc, in the lane's chunk order.
  auto fma_chunk = [&](const uint4& wq, const uint4 (&xq)[kDR]) {
    const uint32_t wv[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
    for (int r = 0; r < kDR; ++r) {
      if (r < a.R) {
        const uint32_t xv[4] = {xq[r].x, xq[r].y, xq[r].z, xq[r].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          acc[r] = fmaf(lo16(xv[c]), lo16(wv[c]), acc[r]);
          acc[r] = fmaf(hi16(xv[c]), hi16(wv[c]), acc[r]);
        }
      }
    }
  };
  // Batches of kUB chunks: every load of a batch is issued before its FMAs (one round trip per batch rather than
  // one per load); the FMAs keep the chunk order.
  constexpr int kUB = 8;
  int k8 = lane;
  for (; k8 + 64 * (kUB - 1) < k8n; k8 += 64 * kUB) {
    uint4 wq[kUB], xq[kUB][kDR];
#pragma unroll
    for (int u = 0; u < kUB; ++u) {
      wq[u] = wr[k8 + 64 * u];
#pragma unroll
      for (int r = 0; r < kDR; ++r)
        xq[u][r] = reinterpret_cast<const uint4*>(a.x + (size_t)(r < a.R ? r : 0) * a.K)[k8 + 64 * u];
    }
#pragma unroll
    for (int u = 0; u < kUB; ++u) fma_chunk(wq[u], xq[u]);
  }
  for (; k8 < k8n; k8 += 64) {
    uint4 xq[kDR];
#pragma unroll
    for (int r = 0; r < kDR; ++r) xq[r] = reinterpret_cast<const uint4*>(a.x + (size_t)(r < a.R ? r : 0) * a.K)[k8];
    fma_chunk(wr[k8], xq);
  }
  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < kDR; ++r) {
    const float s = ss_wave_sum(acc[r]);
    mine = lane == r ? s : mine;
  }
  if (lane < a.R) a.out[(size_t)lane * a.N + n] = (uint16_t)epilogue(mine, a, lane, n);
}

// ---------------------------------------------------------------- the fused head GEMV
// One launch for what the head otherwise runs as a row gather, hc_inject, an RMSNorm and one or two GEMVs, or a GEMV
// and the branch mean, with the same bits as those kernels (the same operations in the same order):
//   pre-step, in every workgroup: the launch's source rows (src rows, or table rows src_idx[s]); optionally
//   h = bf16(src + bf16(y[s][j % Hy] * inj[s][j / Hy])) (hc_inject); optionally x = bf16((h * r_g) * norm_w) with
//   r_g = 1 / sqrt(sum over group g of h^2 / G + eps), the sum in rmsnorm_groups_kernel's order (one wave per group:
//   lane l over the 8-element chunks l, l + 64, .. with fmaf from 0, then the xor butterfly); x into LDS, and
//   workgroup 0 writes h and x out when asked. Staged form (CPG = 0): all threads copy the rows (and inject) into
//   LDS, the group sums read LDS, all threads normalize in place. Grouped form (CPG > 0, groups of CPG 512-element
//   pieces, at most four): wave w loads, injects, sums and normalizes group w in registers and stores x once;
//
//   then the GEMV of dense_epi_kernel over x viewed as R = Sl n / K rows of K (x from LDS): weight rows [0, N) of w
//   with epilogue epi into out, rows [N, N + N2) of w2 with epi2 into out2;
//   or, with mean_out, the branch mean of hc_mean_kernel fused behind the GEMV (hc == 4, K <= 512): one wave takes
//   the four weight rows c H + j of output j (each the dense order: one chunk per lane, then the butterfly), and
//   mean_out[r][j] = bf16((sum over c of bf16(v_c * mean_hn[r][c H + j])) / hc), with no barrier.
struct HeadGemvArgs {
  const uint16_t* src;
  const int32_t* src_idx;
  int64_t n_src;
  const uint16_t* inj_y;
  const uint16_t* inj;
  int inj_hc;
  const uint16_t* norm_w;
  float eps;
  int G;
  int Sl, n, K;  // this launch's source rows, their width, the GEMV's K
  DenseEpiArgs g;  // w, out, add, N, epi, hc, row0, add_div (x and R are set by the kernel)
  const uint16_t* w2;
  int N2, epi2;
  uint16_t* out2;
  uint16_t* h_out;
  uint16_t* x_out;
  const uint16_t* mean_hn;
  uint16_t* mean_out;
  int mean_H;
  int* err;
  uint64_t* trace;  // diagnostics: per-workgroup phase stamps (thread 0), or null
};

constexpr int kHeadLds = 4 * 8192;  // bf16 elements of the staged source rows (Sl n <= 32768)

template <int CPG, bool INJ, int KU>
__global__ __launch_bounds__(256) void head_gemv_kernel(HeadGemvArgs a) {
  extern __shared__ uint4 xs[];  // the staged source rows: Sl n bf16 (sized per launch)
  __shared__ float rs[64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // stamps 0 start, 1 staged, 2 norm factors, 3 normalized, 4 dot products, 5 stored (wave 0 of the workgroup)
#define HG_TRACE(k)                                                                                    \
  do {                                                                                                 \
    if (a.trace && tid == 0) a.trace[(size_t)blockIdx.x * 8 + (k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
  HG_TRACE(0);
  const int n = a.n, E = a.Sl * n, E8 = E >> 3;
  // This wave's weight row, its first kUB chunks requested before the pre-step's arithmetic (they do not depend on
  // x). In mean mode the wave takes the four branch rows c H + j of one output j instead (K <= 512: one chunk per
  // lane).
  const int R = E / a.K, k8n = a.K >> 3;
  const int nrow = blockIdx.x * 4 + w;
  const bool second = !a.mean_out && nrow >= a.g.N;
  const bool has_row = a.mean_out ? nrow < a.mean_H : nrow < a.g.N + a.N2;
  const int wn = second ? nrow - a.g.N : nrow;
  // a wave without a row points at row 0 of w (w2 may be absent)
  const uint4* wr = reinterpret_cast<const uint4*>((second && has_row ? a.w2 : a.g.w) + (size_t)(has_row ? wn : 0) * a.K);
  constexpr int kUB = 16;  // a lane's 16 weight chunks of a K = 8192 row in flight at once
  // CPG > 0: the grouped pre-step (n and G multiples of 512, at most four norm groups of CPG chunks per lane, norm
  // weights given): wave w takes norm group w, whose chunks in lane l are i = l + 64 u, u = w CPG .. w CPG + CPG - 1
  // (the rmsnorm_groups order), all requested before the weight rows and without branches, so that the group's
  // arithmetic waits for its own loads only. Waves past the last group repeat its loads and drop them.
  constexpr int CQ = CPG > 0 ? CPG : 1;
  uint4 xg[CQ], nwg[CQ], yg[INJ ? CQ : 1];
  float gg[INJ ? CQ : 1];
  bool bad_row = false;
  if constexpr (CPG > 0) {
    const int ng = E / a.G, gw = w < ng ? w : ng - 1;
    const int s2 = (512 * gw * CPG) / n;  // a group lies in one source row
    int64_t row = s2;
    if (a.src_idx) {
      row = a.src_idx[s2];
      bad_row = row < 0 || row >= a.n_src;
      if (bad_row) {
        if (lane == 0 && blockIdx.x == 0 && w < ng) ss_raise(a.err, SS_ERR_TOKEN);
        row = 0;
      }
    }
    const int Hy = INJ ? n / a.inj_hc : n;
#pragma unroll
    for (int m = 0; m < CPG; ++m) {
      const int u = gw * CPG + m, j8 = 512 * u + 8 * lane - s2 * n;
      xg[m] = reinterpret_cast<const uint4*>(a.src + row * n)[j8 >> 3];
      nwg[m] = reinterpret_cast<const uint4*>(a.norm_w)[j8 >> 3];
      if constexpr (INJ) {
        const int c = (512 * u - s2 * n) / Hy;
        yg[m] = reinterpret_cast<const uint4*>(a.inj_y + (size_t)s2 * Hy)[(j8 - c * Hy) >> 3];
        gg[m] = ss_bf16_to_f32(a.inj[s2 * a.inj_hc + c]);
      }
    }
  }
  uint4 wq0[kUB];
  if (a.mean_out) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      wq0[c] = has_row && lane < k8n
                   ? reinterpret_cast<const uint4*>(a.g.w + ((size_t)c * a.mean_H + nrow) * a.K)[lane]
                   : make_uint4(0u, 0u, 0u, 0u);
  } else if constexpr (CPG > 0) {
    // K = 512 KU: every chunk in range, so the loads need no branch (chunks KU .. kUB - 1 are never used)
#pragma unroll
    for (int u = 0; u < KU; ++u) wq0[u] = wr[lane + 64 * u];
  } else {
#pragma unroll
    for (int u = 0; u < kUB; ++u)
      wq0[u] = has_row && lane + 64 * u < k8n ? wr[lane + 64 * u] : make_uint4(0u, 0u, 0u, 0u);
  }
  if constexpr (CPG > 0) {
    if (w < E / a.G) {
#pragma unroll
      for (int m = 0; m < CPG; ++m) {
        if (bad_row) xg[m] = make_uint4(0u, 0u, 0u, 0u);
        if constexpr (INJ) {
          const uint32_t hv[4] = {xg[m].x, xg[m].y, xg[m].z, xg[m].w}, yy[4] = {yg[m].x, yg[m].y, yg[m].z, yg[m].w};
          uint32_t o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float t0 = ss_round_bf16(lo16(yy[q]) * gg[m]), t1 = ss_round_bf16(hi16(yy[q]) * gg[m]);
            o[q] = ss_f32_to_bf16(lo16(hv[q]) + t0) | (ss_f32_to_bf16(hi16(hv[q]) + t1) << 16);
          }
          xg[m] = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < CPG; ++m) {
        if (a.h_out && blockIdx.x == 0) reinterpret_cast<uint4*>(a.h_out)[64 * (w * CPG + m) + lane] = xg[m];
        const uint32_t v[4] = {xg[m].x, xg[m].y, xg[m].z, xg[m].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float e0 = lo16(v[c]), e1 = hi16(v[c]);
          acc = fmaf(e0, e0, acc);
          acc = fmaf(e1, e1, acc);
        }
      }
      const float r = 1.f / sqrtf(ss_wave_sum(acc) / (float)a.G + a.eps);
#pragma unroll
      for (int m = 0; m < CPG; ++m) {
        const uint32_t v[4] = {xg[m].x, xg[m].y, xg[m].z, xg[m].w};
        const uint32_t wv[4] = {nwg[m].x, nwg[m].y, nwg[m].z, nwg[m].w};
        uint32_t o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          o[c] = ss_f32_to_bf16((lo16(v[c]) * r) * lo16(wv[c])) | (ss_f32_to_bf16((hi16(v[c]) * r) * hi16(wv[c])) << 16);
        const uint4 x = make_uint4(o[0], o[1], o[2], o[3]);
        const int i = 64 * (w * CPG + m) + lane;
        xs[i] = x;
        if (a.x_out && blockIdx.x == 0) reinterpret_cast<uint4*>(a.x_out)[i] = x;
      }
    }
    __syncthreads();
    HG_TRACE(3);
  } else {
    (void)bad_row;
    // the norm weights of this thread's chunks, with the source loads
    uint4 nwq[kHeadLds / 8 / 256];
    // pre-step 1: the source rows (and the injection) into LDS, h out from workgroup 0 (chunk i = tid + 256 k:
    // unrolled, so that the norm weights stay in registers)
#pragma unroll
    for (int kq = 0; kq < kHeadLds / 8 / 256; ++kq) {
      const int i = tid + 256 * kq;
      if (i >= E8) break;
      if (a.G > 0) {
        const int j = (i << 3) - ((i << 3) / n) * n;
        nwq[kq] = a.norm_w ? reinterpret_cast<const uint4*>(a.norm_w)[j >> 3]
                           : make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
      }
      const int s = (i << 3) / n, j8 = (i << 3) - s * n;
      int64_t row = s;
      if (a.src_idx) {
        row = a.src_idx[s];
        if (row < 0 || row >= a.n_src) {
          if (j8 == 0) ss_raise(a.err, SS_ERR_TOKEN);
          row = -1;
        }
      }
      uint4 v = row >= 0 ? reinterpret_cast<const uint4*>(a.src + row * n)[j8 >> 3] : make_uint4(0u, 0u, 0u, 0u);
      if (a.inj) {
        const int Hy = n / a.inj_hc, c = j8 / Hy;
        const uint4 yv = reinterpret_cast<const uint4*>(a.inj_y + (size_t)s * Hy)[(j8 - c * Hy) >> 3];
        const float g = ss_bf16_to_f32(a.inj[s * a.inj_hc + c]);
        const uint32_t hv[4] = {v.x, v.y, v.z, v.w}, yy[4] = {yv.x, yv.y, yv.z, yv.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float t0 = ss_round_bf16(lo16(yy[q]) * g), t1 = ss_round_bf16(hi16(yy[q]) * g);
          o[q] = ss_f32_to_bf16(lo16(hv[q]) + t0) | (ss_f32_to_bf16(hi16(hv[q]) + t1) << 16);
        }
        v = make_uint4(o[0], o[1], o[2], o[3]);
      }
      xs[i] = v;
      if (a.h_out && blockIdx.x == 0) reinterpret_cast<uint4*>(a.h_out)[i] = v;
    }
    __syncthreads();
    HG_TRACE(1);
    if (a.G > 0) {
      // pre-step 2: r of every group (one wave per group, rmsnorm_groups_kernel's order)
      const int ng = E / a.G, g8 = a.G >> 3;
      for (int g = w; g < ng; g += 4) {
        float acc = 0.f;
        // the LDS reads of 16 chunks issued before their FMAs (which keep the lane's chunk order)
        for (int k0 = lane; k0 < g8; k0 += 64 * 16) {
          uint4 q[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) q[u] = k0 + 64 * u < g8 ? xs[g * g8 + k0 + 64 * u] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
          for (int u = 0; u < 16; ++u) {
            if (k0 + 64 * u < g8) {
              const uint32_t v[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                const float e0 = lo16(v[c]), e1 = hi16(v[c]);
                acc = fmaf(e0, e0, acc);
                acc = fmaf(e1, e1, acc);
              }
            }
          }
        }
        const float r = 1.f / sqrtf(ss_wave_sum(acc) / (float)a.G + a.eps);
        if (lane == 0) rs[g] = r;
      }
      __syncthreads();
      HG_TRACE(2);
      // pre-step 3: x = bf16((h * r) * norm_w) in place, x out from workgroup 0
#pragma unroll
      for (int kq = 0; kq < kHeadLds / 8 / 256; ++kq) {
        const int i = tid + 256 * kq;
        if (i >= E8) break;
        const int e = i << 3, g = e / a.G;
        const float r = rs[g];
        const uint4 q = xs[i];
        const uint4 b = nwq[kq];
        const uint32_t v[4] = {q.x, q.y, q.z, q.w}, wv[4] = {b.x, b.y, b.z, b.w};
        uint32_t o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          o[c] = ss_f32_to_bf16((lo16(v[c]) * r) * lo16(wv[c])) | (ss_f32_to_bf16((hi16(v[c]) * r) * hi16(wv[c])) << 16);
        const uint4 x = make_uint4(o[0], o[1], o[2], o[3]);
        xs[i] = x;
        if (a.x_out && blockIdx.x == 0) reinterpret_cast<uint4*>(a.x_out)[i] = x;
      }
      __syncthreads();
      HG_TRACE(3);
    }
  }
  // the GEMV: one wave per weight row, the launch's x rows from LDS
  if (!has_row) return;  // whole waves; no workgroup barrier follows
  if (a.mean_out) {
    // the four branch rows of output j = nrow (one chunk per lane each), their epilogues, then the mean
    const int j = nrow, H = a.mean_H;
    float v[4][kDR];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float ac[kDR] = {0.f, 0.f, 0.f, 0.f};
      if (lane < k8n) {
        const uint32_t wv[4] = {wq0[c].x, wq0[c].y, wq0[c].z, wq0[c].w};
#pragma unroll
        for (int r = 0; r < kDR; ++r) {
          if (r < R) {
            const uint4 xq = xs[r * k8n + lane];
            const uint32_t xv[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              ac[r] = fmaf(lo16(xv[q]), lo16(wv[q]), ac[r]);
              ac[r] = fmaf(hi16(xv[q]), hi16(wv[q]), ac[r]);
            }
          }
        }
      }
#pragma unroll
      for (int r = 0; r < kDR; ++r) v[c][r] = ss_wave_sum(ac[r]);
    }
    if (lane < R) {
      DenseEpiArgs ea = a.g;
      ea.R = R;
      float m = 0.f;
      const uint16_t* hn = a.mean_hn + (size_t)lane * 4 * H;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float d = v[c][0];
#pragma unroll
        for (int r = 1; r < kDR; ++r) d = lane == r ? v[c][r] : d;
        const uint32_t e = epilogue(d, ea, lane, c * H + j);
        ea.out[(size_t)lane * ea.N + c * H + j] = (uint16_t)e;
        m += ss_round_bf16(ss_bf16_to_f32(e) * ss_bf16_to_f32(hn[(size_t)c * H + j]));
      }
      a.mean_out[(size_t)lane * H + j] = (uint16_t)ss_f32_to_bf16(m / 4.0f);
    }
    return;
  }
  float acc[kDR] = {0.f, 0.f, 0.f, 0.f};
  auto fma_chunk = [&](const uint4& wq, int kk) {
    const uint32_t wv[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
    for (int r = 0; r < kDR; ++r) {
      if (r < R) {
        const uint4 xq = xs[r * k8n + kk];
        const uint32_t xv[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          acc[r] = fmaf(lo16(xv[c]), lo16(wv[c]), acc[r]);
          acc[r] = fmaf(hi16(xv[c]), hi16(wv[c]), acc[r]);
        }
      }
    }
  };
#pragma unroll
  for (int u = 0; u < kUB; ++u)
    if (lane + 64 * u < k8n) fma_chunk(wq0[u], lane + 64 * u);
  int k8 = lane + 64 * kUB;
  for (; k8 + 64 * (kUB - 1) < k8n; k8 += 64 * kUB) {
    uint4 wq[kUB];
#pragma unroll
    for (int u = 0; u < kUB; ++u) wq[u] = wr[k8 + 64 * u];
#pragma unroll
    for (int u = 0; u < kUB; ++u) fma_chunk(wq[u], k8 + 64 * u);
  }
  for (; k8 < k8n; k8 += 64) fma_chunk(wr[k8], k8);
  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < kDR; ++r) {
    const float s = ss_wave_sum(acc[r]);
    mine = lane == r ? s : mine;
  }
  HG_TRACE(4);
  DenseEpiArgs ea = a.g;
  ea.R = R;
  if (second) {
    ea.epi = a.epi2;
    ea.N = a.N2;
    ea.out = a.out2;
  }
  if (lane < R) ea.out[(size_t)lane * ea.N + wn] = (uint16_t)epilogue(mine, ea, lane, wn);
  HG_TRACE(5);
#undef HG_TRACE
}

// mixed[s][j] = bf16((sum over c = 0 .. hc-1 of bf16(m[s][c H + j] * hn[s][c H + j])) / hc), the sum sequential.
__global__ __launch_bounds__(256) void hc_mean_kernel(const uint16_t* __restrict__ m, const uint16_t* __restrict__ hn,
                                                      int S, int hc, int H, uint16_t* __restrict__ mixed) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)S * H) return;
  const int64_t s = i / H;
  const int j = (int)(i - s * H);
  const size_t b = (size_t)s * hc * H + j;
  float acc = 0.f;
  for (int c = 0; c < hc; ++c)
    acc += ss_round_bf16(ss_bf16_to_f32(m[b + (size_t)c * H]) * ss_bf16_to_f32(hn[b + (size_t)c * H]));
  mixed[i] = (uint16_t)ss_f32_to_bf16(acc / (float)hc);
}

// out[s][c H + j] = bf16(hyp[s][c H + j] + bf16(y[s][j] * inj[s][c])); out may be hyp (each thread reads its element
// before writing it).
__global__ __launch_bounds__(256) void hc_inject_kernel(const uint16_t* hyp, const uint16_t* __restrict__ y,
                                                        const uint16_t* __restrict__ inj, int S, int hc, int H,
                                                        uint16_t* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = (int64_t)hc * H;
  if (i >= (int64_t)S * row) return;
  const int64_t s = i / row;
  const int c = (int)((i - s * row) / H);
  const int j = (int)(i - s * row - (int64_t)c * H);
  const float t = ss_round_bf16(ss_bf16_to_f32(y[s * H + j]) * ss_bf16_to_f32(inj[s * hc + c]));
  out[i] = (uint16_t)ss_f32_to_bf16(ss_bf16_to_f32(hyp[i]) + t);
}

// dst row i = src row (idx[i] + idx_add) in pieces of U (uint4, or uint32 for rows of 4-byte multiples); an index
// outside [0, n_src) writes zeros and raises SS_ERR_TOKEN.
template <typename U>
__global__ __launch_bounds__(256) void gather_rows_kernel(const U* __restrict__ src, int64_t n_src, int64_t row_u,
                                                          const int32_t* __restrict__ idx, int n, int idx_add,
                                                          U* __restrict__ dst, int* err) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)n * row_u) return;
  const int64_t r = i / row_u;
  const int64_t c = i - r * row_u;
  const int64_t k = (int64_t)idx[r] + idx_add;
  U v{};
  if (k >= 0 && k < n_src)
    v = src[k * row_u + c];
  else if (c == 0)
    ss_raise(err, SS_ERR_TOKEN);
  dst[i] = v;
}

}  // namespace

hipError_t launch_rmsnorm_groups(const uint16_t* x, const uint16_t* w, float eps, int R, int n, int G, uint16_t* out,
                                 hipStream_t st) {
  const int64_t nseg = (int64_t)R * (n / G);
  if (nseg == 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_groups_kernel, dim3((unsigned)((nseg + 3) / 4)), dim3(256), 0, st, x, w, eps, nseg, n, G,
                     out);
  return hipGetLastError();
}

hipError_t launch_dense_epi(const uint16_t* x, int R, int K, const uint16_t* w, int N, int epi, int hc,
                            const uint16_t* add, int add_div, uint16_t* out, hipStream_t st) {
  DenseEpiArgs a{};
  a.w = w;
  a.K = K;
  a.N = N;
  a.epi = epi;
  a.hc = (float)hc;
  a.add = add;
  a.add_div = add_div > 0 ? add_div : 1;
  for (int r0 = 0; r0 < R; r0 += kDR) {
    a.x = x + (size_t)r0 * K;
    a.out = out + (size_t)r0 * N;
    a.R = R - r0 < kDR ? R - r0 : kDR;
    a.row0 = r0;
    hipLaunchKernelGGL(dense_epi_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_head_gemv(const HeadGemvIn& in, hipStream_t st) {
  // source rows per launch: the staged rows fit the LDS, their x rows one GEMV pass (<= kDR) and their norm groups
  // the table of 64
  int per = kDR * in.K / in.n < kHeadLds / in.n ? kDR * in.K / in.n : kHeadLds / in.n;
  if (in.G > 0 && 64 * in.G / in.n < per) per = 64 * in.G / in.n;
  if (per < 1) return hipErrorInvalidValue;
  HeadGemvArgs a{};
  a.src_idx = nullptr;
  a.n_src = in.n_src;
  a.inj_hc = in.inj_hc;
  a.norm_w = in.norm_w;
  a.eps = in.eps;
  a.G = in.G;
  a.n = in.n;
  a.K = in.K;
  a.g.K = in.K;
  a.g.epi = in.epi;
  a.g.hc = (float)in.hc;
  a.g.add_div = in.add_div > 0 ? in.add_div : 1;
  a.g.N = in.N;
  a.N2 = in.N2;
  a.epi2 = in.epi2;
  a.mean_H = in.mean_H;
  a.err = in.err;
  a.trace = in.trace;
  const int xr = in.n / in.K;  // x rows per source row
  for (int s0 = 0; s0 < in.S; s0 += per) {
    a.Sl = in.S - s0 < per ? in.S - s0 : per;
    a.src = in.src_idx ? in.src : in.src + (size_t)s0 * in.n;
    a.src_idx = in.src_idx ? in.src_idx + s0 : nullptr;
    a.inj_y = in.inj_y ? in.inj_y + (size_t)s0 * (in.n / in.inj_hc) : nullptr;
    a.inj = in.inj ? in.inj + (size_t)s0 * in.inj_hc : nullptr;
    a.g.w = in.w;
    a.g.out = in.out + (size_t)s0 * xr * in.N;
    a.g.add = in.add;
    a.g.row0 = s0 * xr;
    a.w2 = in.w2;
    a.out2 = in.out2 ? in.out2 + (size_t)s0 * xr * in.N2 : nullptr;
    a.h_out = in.h_out ? in.h_out + (size_t)s0 * in.n : nullptr;
    a.x_out = in.x_out ? in.x_out + (size_t)s0 * in.n : nullptr;
    a.mean_hn = in.mean_hn ? in.mean_hn + (size_t)s0 * in.n : nullptr;
    a.mean_out = in.mean_out ? in.mean_out + (size_t)s0 * xr * in.mean_H : nullptr;
    // the grouped pre-step: every norm group of this launch to one wave (at most four groups of 2048 elements, norm
    // weights given, K 2048 or 8192, an injection width of whole 512-element pieces). Larger groups stay staged: one
    // wave over a group of 8192 measured slower than the staged step (10.5 against 9.6 us for the head's fc_hidden
    // launch).
    const bool grouped = !in.mean_out && in.G == 2048 && in.norm_w && in.n % 512 == 0 && a.Sl * in.n <= 4 * in.G &&
                         (in.K == 2048 || in.K == 8192) && (!in.inj || (in.n / in.inj_hc) % 512 == 0);
    auto kern = !grouped       ? head_gemv_kernel<0, false, 16>
                : in.K == 2048 ? (in.inj ? head_gemv_kernel<4, true, 4> : head_gemv_kernel<4, false, 4>)
                               : (in.inj ? head_gemv_kernel<4, true, 16> : head_gemv_kernel<4, false, 16>);
    KernelCfg cfg;  // allows the largest staging (64 KB) as dynamic LDS, once per device and instantiation
    hipError_t ce = kernel_cfg(reinterpret_cast<const void*>(kern), 256, (size_t)kHeadLds * 2, &cfg);
    if (ce != hipSuccess) return ce;
    const int grid = in.mean_out ? (in.mean_H + 3) / 4 : (in.N + in.N2 + 3) / 4;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), (size_t)a.Sl * in.n * 2, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_hc_mean(const uint16_t* m, const uint16_t* hn, int S, int hc, int H, uint16_t* mixed,
                          hipStream_t st) {
  const int64_t n = (int64_t)S * H;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(hc_mean_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, m, hn, S, hc, H, mixed);
  return hipGetLastError();
}

hipError_t launch_hc_inject(const uint16_t* hyp, const uint16_t* y, const uint16_t* inj, int S, int hc, int H,
                            uint16_t* out, hipStream_t st) {
  const int64_t n = (int64_t)S * hc * H;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(hc_inject_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, hyp, y, inj, S, hc, H, out);
  return hipGetLastError();
}

hipError_t launch_gather_rows(const void* src, int64_t n_src, int64_t row_bytes, const int32_t* idx, int n,
                              int idx_add, void* dst, int* err, hipStream_t st) {
  const bool wide = row_bytes % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(dst) % 16 == 0;
  const int64_t row_u = row_bytes / (wide ? 16 : 4);
  const int64_t total = (int64_t)n * row_u;
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (wide)
    hipLaunchKernelGGL(gather_rows_kernel<uint4>, grid, dim3(256), 0, st, static_cast<const uint4*>(src), n_src, row_u,
                       idx, n, idx_add, static_cast<uint4*>(dst), err);
  else
    hipLaunchKernelGGL(gather_rows_kernel<uint32_t>, grid, dim3(256), 0, st, static_cast<const uint32_t*>(src), n_src,
                       row_u, idx, n, idx_add, static_cast<uint32_t*>(dst), err);
  return hipGetLastError();
}

}  // namespace ss
