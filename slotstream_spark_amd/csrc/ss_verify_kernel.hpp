// One persistent launch per MoE layer of a verify step (T <= 4 tokens), or per block of 4 rows of moe_decode.
//
// Phases (every workgroup resident: the grid is one workgroup per CU; 4 waves each):
//   A  verify mode. Dense bf16 rows in the fixed fp32 order of dense_rows_kernel (the E router rows, the Is shared
//      gate/up row pairs, the shared_expert_gate row) spread over every wave of the grid, while the layer's map and
//      slot_ptr tables are staged into LDS. Each workgroup publishes its finished row counts (release).
//   B  Each workgroup waits for all router rows (acquire) and computes the router tail for every token itself
//      (softmax, top-k, renormalisation: the same bits everywhere), then the unique expert list of the block.
//      Workgroups that own output rows then start direct-to-LDS loads of their down-projection weights for the
//      first P experts, which stream while phase C runs.
//   C  Routed gate/up items, one (unique expert u, 8-row tile p) per wave at a time over the full K: 16 columns =
//      8 gate rows + 8 up rows, 16 x 16-byte loads per lane in flight, x A-fragments from LDS. The epilogue writes
//      h as bf16 hi/lo MFMA A-fragments (the layout the down phase consumes), 8-element partial sums of h for the
//      per-group bias term, and h_buf. Each workgroup publishes its item count.
//   D  Workgroup b < H/16 owns output rows 16b..16b+15 for every expert. After all items (and, in verify mode, the
//      shared rows) are published, it stages the h fragments into LDS, each wave runs the down MFMAs of the experts
//      u = w (mod 4), the shared-expert down rows are added, and the rank-order combine writes o, out and y. No
//      floating-point sum uses atomics; every sum has a fixed order.
// The kernel is written with rolled loops and small unroll factors: each workgroup runs it once per launch, so its
// instruction footprint, not only its arithmetic, bounds the time.
// Device counters live at the start of the scratch; the last workgroup to leave resets them, so every launch starts
// from zero. Waits are bounded: on timeout the kernel raises SS_ERR_TIMEOUT and finishes.
//
// Reference semantics: kernels/moe_gemv_affine.py:56-147, model/layers.py:336-402, reference_torch.py:118-134,
// runtime/graphs.py:160-169.
#pragma once
#include "ss_verify_dev.hpp"

namespace ss {

template <int NJG, int NJD, bool XF32, bool SHQ4>
__global__ __launch_bounds__(256) void verify_kernel(VerifyArgs a, SsRecord rec) {
  extern __shared__ uint4 dsm[];
  __shared__ VSmem s;
  uint8_t* dl = reinterpret_cast<uint8_t*>(dsm);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int G = gridDim.x, bid = blockIdx.x;
  const int n = lane & 15, g = lane >> 4;
  const int T = a.T, H = a.H, I = a.I, K = a.K, E = a.E;
  const bool verify = a.mode == 0;
  const VLayout L = vlayout(T, H, I, verify ? a.Is : 0, K, verify ? E : 0);
  const DLayout D = dlayout(T, H, I, K, E, XF32 ? 1 : 0, verify ? 1 : 0);
  uint8_t* scr = static_cast<uint8_t*>(a.scratch);
  int* ctr = reinterpret_cast<int*>(scr + L.ctr);
  uint64_t* logits = reinterpret_cast<uint64_t*>(scr + L.logits);
  const uint32_t tag = (uint32_t)ld_ag(shard(ctr, CTR_EPOCH, 0)) + 1u;  // this launch's logit tag
  uint16_t* gsh = reinterpret_cast<uint16_t*>(scr + L.gsh);
  uint16_t* ush = reinterpret_cast<uint16_t*>(scr + L.ush);
  uint16_t* sgl = reinterpret_cast<uint16_t*>(scr + L.sgl);
  uint4* hfrag = reinterpret_cast<uint4*>(scr + L.hfrag);
  float* hsum8 = reinterpret_cast<float*>(scr + L.hsum8);
  uint4* xfl = reinterpret_cast<uint4*>(dl + D.xfrag);
  uint4* hfl = reinterpret_cast<uint4*>(dl + D.hfrag);
  float* partl = reinterpret_cast<float*>(dl + D.part);
  uint8_t* prefl = dl + D.pref;
  const int nt = T;
#define SS_TRACE(k)                                                                               \
  do {                                                                                            \
    if (a.trace && tid == 0) a.trace[(size_t)bid * 16 + (k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)

  SS_TRACE(0);
  for (int i = tid; i < kMaxQv * kTBv; i += 256) (&s.umask[0][0])[i] = 0u;
  if (tid < 4) s.zero_h[tid] = make_uint4(0u, 0u, 0u, 0u);
  if (tid == 0) s.nt = nt;

  // ------------------------------------------------------------ phase A + B (verify) / ids (decode)
  // Dense-row jobs (verify mode): j < E is router row j; E <= j < E + Is the shared gate and up rows j - E, and the
  // last of those jobs also takes the shared_expert_gate row, so no workgroup that holds router rows waits for a
  // second job. The rows of a wave's first job, this workgroup's map entries and x are all requested before any of
  // them is used, so phase A costs one memory round trip.
  constexpr int NJX = NJG / 4;  // 16-byte words per lane of one dense row (H / 512)
  const int Is = a.Is, J = verify ? E + Is : 0, W = G * 4;
  const int j_first = bid * 4 + w;
  const bool has_tile = bid < (H >> 4);
  uint4 r0[NJX], r1[NJX], r2[NJX];
  constexpr bool sh_q4 = SHQ4;  // affine 4-bit shared gate / up / down (sh_gs .. sh_db set), else bf16 rows
  auto load_job = [&](int j) {
    if (j >= E && sh_q4) {
      // affine 4-bit shared gate and up rows: q4_chunk registers
      const size_t r = (size_t)(j - E);
#pragma unroll
      for (int jj = 0; jj < NJX; ++jj) {
        r0[jj] = q4_chunk(a.sh_gate + r * (H / 4), a.sh_gs + r * (H / 64), a.sh_gb + r * (H / 64), jj, lane);
        r1[jj] = q4_chunk(a.sh_up + r * (H / 4), a.sh_us + r * (H / 64), a.sh_ub + r * (H / 64), jj, lane);
      }
    } else {
      const uint16_t* w0 = j < E ? a.router_w + (size_t)j * H : a.sh_gate + (size_t)(j - E) * H;
#pragma unroll
      for (int jj = 0; jj < NJX; ++jj) r0[jj] = ldg16(w0 + 8 * (64 * jj + lane));
      if (j >= E) {
        const uint16_t* w1 = a.sh_up + (size_t)(j - E) * H;
#pragma unroll
        for (int jj = 0; jj < NJX; ++jj) r1[jj] = ldg16(w1 + 8 * (64 * jj + lane));
      }
    }
    if (j == J - 1) {
#pragma unroll
      for (int jj = 0; jj < NJX; ++jj) r2[jj] = ldg16(a.sh_g + 8 * (64 * jj + lane));
    }
  };
  if (verify && j_first < J) load_job(j_first);
  int slot_e[2] = {-1, -1};
  if (verify) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int e = tid + 256 * k;
      const int64_t mi = a.map_base + e;
      const bool ok = e < E && mi < a.map_len;
      const int v = gp(a.map)[ok ? mi : 0];
      slot_e[k] = ok ? v : -1;
    }
  }
  stage_x<NJG, XF32>(a, xfl, s.gx, s.rnorm, nt);
  __syncthreads();
  if (verify) {
#pragma unroll 1
    for (int j = j_first; j < J; j += W) {
      if (j != j_first) load_job(j);
      // The job's rows (router or shared gate, then shared up, then the shared_expert_gate row) pass through r0 in
      // turn, so the dot product has one copy in the code: each workgroup runs this phase once per launch, and its
      // instruction footprint counts with its arithmetic.
      const int nrow = j < E ? 1 : (j == J - 1 ? 3 : 2);
#pragma unroll 1
      for (int q = 0; q < nrow; ++q) {
        float d[kTBv];
        if (sh_q4 && j >= E && q < 2)
          affine_dot<NJX>(r0, xfl, nt, d);
        else
          dense_dot<NJX>(r0, xfl, nt, d);
        if (lane == 0) {
          if (j < E) {
#pragma unroll 1
            for (int t = 0; t < nt; ++t)
              st_ag(logits + (size_t)t * E + j, ((uint64_t)tag << 32) | (uint64_t)ss_f32_to_bf16(d[t]));
          } else {
            uint16_t* dst = q == 0 ? gsh + (j - E) : (q == 1 ? ush + (j - E) : sgl);
            const size_t ts = q == 2 ? 1 : (size_t)Is;
#pragma unroll 1
            for (int t = 0; t < nt; ++t) st_ag(dst + (size_t)t * ts, (uint16_t)ss_f32_to_bf16(d[t]));
          }
        }
#pragma unroll
        for (int jj = 0; jj < NJX; ++jj) {
          r0[jj] = r1[jj];
          r1[jj] = r2[jj];
        }
      }
    }
    stores_done();
    __syncthreads();
    if (tid == 0) {
      int ns = 0;
      for (int ww = 0; ww < 4; ++ww)
        for (int j = bid * 4 + ww; j < J; j += W)
          if (j >= E) ns += j == J - 1 ? 2 : 1;
      if (ns) signal_add(ctr, CTR_SHARED, ns);
      SS_TRACE(1);
    }
    // The layer's slot pointers into LDS and the routing bias into the tail waves' registers while the other
    // workgroups finish their router rows.
    const uint8_t* base_k[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const bool ok = slot_e[k] >= 0 && (int64_t)slot_e[k] < a.n_slots;
      const int64_t p = gp(a.slot_ptr)[ok ? slot_e[k] : 0];
      base_k[k] = ok ? reinterpret_cast<const uint8_t*>(p) : nullptr;
    }
    constexpr int NV = kMaxEv / 64;
    float bias_r[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + 64 * i;
      bias_r[i] = a.bias ? gp(a.bias)[e < E ? e : 0] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int e = tid + 256 * k;
      if (e < E) {
        s.map[e] = slot_e[k];
        s.base_e[e] = base_k[k];
      }
    }
    SS_TRACE(2);
    if (w < nt) {
      router_tail_wave(a, logits, tag, w, s, bias_r);
      if (a.trace && tid == 0) a.trace[(size_t)bid * 16 + 12] = __builtin_amdgcn_s_memrealtime();
    }
    __syncthreads();
    SS_TRACE(3);
    if (bid == 0 && tid < nt * K) {
      a.ids_out[tid] = s.ids[tid];
      a.w_out[tid] = s.wts[tid];
    }
  } else {
    if (tid < nt * K) {
      s.ids[tid] = a.ids_in[tid];
      s.wts[tid] = a.w_in[tid];
    }
    __syncthreads();
  }
  if (tid < 64) {
    unique_setup(a, s, verify);
  } else {
    // Zeros that phase C's A lanes outside their row block read instead of x (the router-tail candidates that
    // share this memory are dead; phase D writes hsum only after every item is done).
    for (int i = tid - 64; i < kXZero; i += 192) reinterpret_cast<uint4*>(s.hsum)[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();
  SS_TRACE(4);
  const int nu = s.nu;
  const int tiles = I >> 3;
  const int n_items = nu * tiles;
  const int my_half = g >> 1, my_part = g & 1;
  const int drow = 16 * bid + n;  // down row of this lane
  const int64_t drow_b = I >> 1, dsb_b = (I >> 6) * 2;

  // ------------------------------------------------------------ down prefetch: P experts into LDS
  // Slot layout (per expert): [NJD][64 lanes] weight uint4, then [NJD][64 lanes] scale dword, [NJD][64] bias dword.
  auto issue_down = [&](int u, int slotp) {
    uint8_t* sl = prefl + (size_t)slotp * D.slot;
    const uint8_t* base = s.base[u];
    for (int j = 0; j < NJD; ++j) dma16(base + rec.dw + drow * drow_b + 64 * j + 16 * g, sl + (size_t)j * 1024);
    // scale and bias dwords: entry idx = row * NJD + j of the 16 rows (NJD dwords each)
    for (int k0 = 0; k0 < 16 * NJD; k0 += 64) {
      const int idx = k0 + lane;
      if (idx < 16 * NJD) {
        const int row = idx / NJD, jj = idx - row * NJD;
        const int64_t ro = (int64_t)(16 * bid + row) * dsb_b + 4 * jj;
        dma4(base + rec.ds + ro, sl + (size_t)NJD * 1024 + (size_t)k0 * 4);
        dma4(base + rec.db + ro, sl + (size_t)NJD * 1024 + (size_t)16 * NJD * 4 + (size_t)k0 * 4);
      }
    }
  };

  // ------------------------------------------------------------ phase C: gate/up, one item per wave at a time
  // Items go first to the workgroups without down rows (bid >= H/16), one per wave, then wrap around.
  const int gw = ((bid - (H >> 4) + G) % G) * 4 + w;
  int my_items = 0;
  for (int ww = 0; ww < 4; ++ww) {
    const int gq = ((bid - (H >> 4) + G) % G) * 4 + ww;
    for (int it = gq; it < n_items; it += W) ++my_items;
  }
  if (my_items) {
    SS_TRACE(6);
    const int m = lane & 15, at = m & 3, agrp = m >> 2, ahh = agrp >> 1, apart = agrp & 1;
    const bool a_act = ahh == (g >> 1) && at < nt && (XF32 || apart == 0);
    const int64_t row_b = H >> 1, sb_b = (H >> 6) * 2;
    float* xch = s.xch[w];
#pragma unroll 1
    for (int item = gw; item < n_items; item += W) {
      const int u = item / tiles, p = item - u * tiles;
      const int r8 = 8 * p + (n & 7);
      const uint8_t* base = s.base[u];
      const uint8_t* wrow = base + (n < 8 ? rec.gw : rec.uw) + r8 * row_b + 16 * g;
      const SS_G uint32_t* srow = (const SS_G uint32_t*)gp(base + (n < 8 ? rec.gs : rec.us) + r8 * sb_b);
      const SS_G uint32_t* brow = (const SS_G uint32_t*)gp(base + (n < 8 ? rec.gb : rec.ub) + r8 * sb_b);
      uint4 wv[NJG];
      uint32_t sv[NJG], bv[NJG];
#pragma unroll
      for (int j = 0; j < NJG; ++j) {
        wv[j] = ldg16(wrow + 64 * j);
        sv[j] = srow[j];
        bv[j] = brow[j];
      }
      // Keep every load of the item ahead of the first MFMA: otherwise the scheduler spreads them over the loop
      // and the item pays one memory latency per batch.
      __builtin_amdgcn_sched_barrier(0);
      if (item == gw && w == 0) {
        __builtin_amdgcn_s_waitcnt(0);
        SS_TRACE(14);
      }
      float acc[kTBv] = {0.f, 0.f, 0.f, 0.f};
      constexpr int JB = NJG % 4 == 0 ? 4 : 1;  // K iterations whose LDS operands are read before their MFMAs
#pragma unroll
      for (int j0 = 0; j0 < NJG; j0 += JB) {
        uint4 av4[JB][4];
        float4 gxv[JB];
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
          const int j = j0 + jj;
          const uint4* fp = a_act ? xfl + (size_t)(((j * 4) * 4 + g) * kTBv + at) * (XF32 ? 2 : 1) + (XF32 ? apart : 0)
                                  : reinterpret_cast<const uint4*>(s.hsum);  // zeros (kXZero entries)
#pragma unroll
          for (int i = 0; i < 4; ++i) av4[jj][i] = fp[(size_t)i * 16 * (XF32 ? 2 : 1)];  // in bounds for every lane
          gxv[jj] = reinterpret_cast<const float4*>(s.gx)[2 * j + my_half];
        }
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
          const int j = j0 + jj;
          ss_f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            ss_u32x4 av = as_v(av4[jj][i]);
            const uint32_t wd = i == 0 ? wv[j].x : i == 1 ? wv[j].y : i == 2 ? wv[j].z : wv[j].w;
            d = ss_mfma(av, ss_nibbles_to_bf16(wd), d);
          }
          const float sf = pick_half(sv[j], my_half);
          const float bf = pick_half(bv[j], my_half);
          const float s16 = sf * kNibbleScale;
          const float bp = my_part ? 0.f : __builtin_fmaf(-kNibbleScale, sf, bf);
          const float gxa[kTBv] = {gxv[jj].x, gxv[jj].y, gxv[jj].z, gxv[jj].w};
#pragma unroll
          for (int r = 0; r < kTBv; ++r) {
            acc[r] = __builtin_fmaf(s16, d[r], acc[r]);
            acc[r] = __builtin_fmaf(bp, gxa[r], acc[r]);
          }
        }
      }
      if (item == gw && w == 0) SS_TRACE(15);
#pragma unroll
      for (int r = 0; r < kTBv; ++r) {
        acc[r] = ss_rows_sum(acc[r]);
        if (g == 0) xch[n * kTBv + r] = acc[r];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      {
        // h = silu(gate) * up of one (token r, row c) per lane 8 r + c, written over that gate value.
        const int r = lane >> 3, c = lane & 7;
        if (r < nt) {
          const float gv = xch[c * kTBv + r], uv = xch[(c + 8) * kTBv + r];
          xch[c * kTBv + r] = gv / (1.f + ss_expf(-gv)) * uv;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (lane < nt) {
        const int r = lane;
        float hv[8];
        float sum8 = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          hv[c] = xch[c * kTBv + r];
          sum8 = sum8 + hv[c];
        }
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t a0 = ss_f32_to_bf16(hv[d]), a1 = ss_f32_to_bf16(hv[d + 4]);
          hw[d] = a0 | (a1 << 16);
          lw[d] = ss_f32_to_bf16(hv[d] - ss_bf16_to_f32(a0)) | (ss_f32_to_bf16(hv[d + 4] - ss_bf16_to_f32(a1)) << 16);
        }
        const uint4 fhi = make_uint4(hw[0], hw[1], hw[2], hw[3]), flo = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        const int jf = p >> 4, gf = (p & 15) >> 2, ifr = p & 3;
        uint32_t mk = s.umask[u][r];
        while (mk) {
          const int k = __ffs(mk) - 1;
          mk &= mk - 1;
          const int q = r * K + k;
          uint4* fpo = hfrag + (((size_t)q * NJD + jf) * 4 + gf) * 8 + ifr;
          st_ag16(fpo, fhi);
          st_ag16(fpo + 4, flo);
          st_ag(reinterpret_cast<uint32_t*>(hsum8) + (size_t)q * (I >> 3) + p, __float_as_uint(sum8));
          if (a.h_buf) {
            float* hp = a.h_buf + ((size_t)r * K + k) * I + 8 * p;
            stg16(hp, make_uint4(__float_as_uint(hv[0]), __float_as_uint(hv[1]), __float_as_uint(hv[2]),
                                 __float_as_uint(hv[3])));
            stg16(hp + 4, make_uint4(__float_as_uint(hv[4]), __float_as_uint(hv[5]), __float_as_uint(hv[6]),
                                     __float_as_uint(hv[7])));
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    stores_done();
    __syncthreads();
    if (tid == 0) signal_add(ctr, CTR_ITEMS, my_items);
    SS_TRACE(7);
  }

  // Shared-expert down rows (verify mode): their weights and the first batch of down-projection weights are
  // requested only now, after the gate/up items are published (requested earlier they would queue ahead of the
  // items' own loads); the gate / up inputs follow the DMAs, and the rows are computed after the down experts, when
  // every load has landed, so nothing here waits on the critical path.
  constexpr int NSC = NJD > 4 ? 2 : 1;  // 512-element chunks of a shared down row per lane (Is <= 512 * NSC)
  uint4 shw[4][NSC];
  SharedIn shin;
  if (verify && has_tile) load_shared_down<4, NSC, SHQ4>(a, 16 * bid + 4 * w, shw);
  if (has_tile) {
#pragma unroll 1
    for (int u = w; u < nu && u < D.P; u += 4) issue_down(u, u);
  }
  if (verify && has_tile) {
    wait_ge(ctr, CTR_SHARED, a.Is + 1, a.err);
    shin = shared_load(a, gsh, ush, nt);
  }

  // ------------------------------------------------------------ phase D: down + combine
  if (has_tile) {
    if (w == 0) wait_ge(ctr, CTR_ITEMS, n_items, a.err);
    __syncthreads();
    SS_TRACE(8);
    // The combine's shared-expert gate logit, requested now and used at the end.
    const uint16_t sgl_pre = verify && tid < 16 * kTBv ? ld_ag(sgl + ((tid & 3) < nt ? (tid & 3) : 0)) : 0;
    const int nq = nt * K;
    // Stage the h fragments of every use into LDS (1 KB per wave instruction) and the h group sums.
    const int hchunks = D.stage_h ? nq * I * 4 / 1024 : 0;
#pragma unroll 1
    for (int c = w; c < hchunks; c += 4) dma16_ag(reinterpret_cast<const uint8_t*>(hfrag) + (size_t)c * 1024 + 16 * lane,
                                               reinterpret_cast<uint8_t*>(hfl) + (size_t)c * 1024);
    for (int idx = tid; idx < nq * (I >> 6); idx += 256) {
      const int q = idx / (I >> 6), Gi = idx - q * (I >> 6);
      float sum = 0.f;
      if (s.use_u[q] >= 0) {
        const float* hp = hsum8 + (size_t)q * (I >> 3) + 8 * Gi;
        const uint4 h0 = ld_ag16(hp), h1 = ld_ag16(hp + 4);
        const float hv[8] = {__uint_as_float(h0.x), __uint_as_float(h0.y), __uint_as_float(h0.z), __uint_as_float(h0.w),
                             __uint_as_float(h1.x), __uint_as_float(h1.y), __uint_as_float(h1.z), __uint_as_float(h1.w)};
#pragma unroll
        for (int c = 0; c < 8; ++c) sum = sum + hv[c];
      }
      s.hsum[q][Gi] = sum;
    }
    stores_done();
    __syncthreads();
    SS_TRACE(9);
    const int m = lane & 15, at = m & 3, agrp = m >> 2, ahh = agrp >> 1, apart = agrp & 1;
    const bool a_lane = ahh == (g >> 1) && at < nt;
#pragma unroll 1
    for (int u0 = 0; u0 < nu; u0 += D.P) {
      if (u0 > 0) {
        __syncthreads();
#pragma unroll 1
        for (int u = u0 + w; u < nu && u < u0 + D.P; u += 4) issue_down(u, u - u0);
        stores_done();
        __syncthreads();
      }
      // One expert: every operand is read up front (weights, scales, h fragments, h group sums; inactive lanes read
      // in-bounds index 0 and are zeroed by a select), then the MFMA chains run without intervening waits.
      // NTK = 2 when T <= 2: the accumulators, h group sums and row sums of the two absent token rows are skipped
      // (the combine reads rows r < T only).
      auto expert = [&](int u, auto staged, auto ntk) {
        constexpr bool STAGED = decltype(staged)::value;
        constexpr int NTK = decltype(ntk)::value;
        const uint8_t* sl = prefl + (size_t)(u - u0) * D.slot;
        const uint32_t am = a_lane ? s.umask[u][at] : 0u;
        const int aq = am ? at * K + __ffs(am) - 1 : 0;
        int qr[kTBv];
        bool vr[kTBv];
#pragma unroll
        for (int r = 0; r < NTK; ++r) {
          const uint32_t mr = r < nt ? s.umask[u][r] : 0u;
          vr[r] = mr != 0u;
          qr[r] = mr ? r * K + __ffs(mr) - 1 : 0;
        }
        uint4 wq[NJD], av4[NJD][4];
        uint32_t svw[NJD], bvw[NJD];
        float hsv[NJD][kTBv];
#pragma unroll
        for (int j = 0; j < NJD; ++j) {
          wq[j] = reinterpret_cast<const uint4*>(sl + (size_t)j * 1024)[lane];
          svw[j] = reinterpret_cast<const uint32_t*>(sl + (size_t)NJD * 1024)[n * NJD + j];
          bvw[j] = reinterpret_cast<const uint32_t*>(sl + (size_t)NJD * 1024 + (size_t)16 * NJD * 4)[n * NJD + j];
          const size_t fo = (((size_t)aq * NJD + j) * 4 + g) * 8 + apart * 4;
#pragma unroll
          for (int i = 0; i < 4; ++i) av4[j][i] = STAGED ? (am ? hfl + fo : s.zero_h)[i] : ld_ag16(hfrag + fo + i);
#pragma unroll
          for (int r = 0; r < NTK; ++r) hsv[j][r] = s.hsum[qr[r]][2 * j + my_half];
        }
        float acc[kTBv] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NJD; ++j) {
          ss_f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            ss_u32x4 av = as_v(av4[j][i]);
            if (!STAGED && !am) av = ss_u32x4{0u, 0u, 0u, 0u};  // staged: zero_h was read instead
            const uint32_t wd = i == 0 ? wq[j].x : i == 1 ? wq[j].y : i == 2 ? wq[j].z : wq[j].w;
            d = ss_mfma(av, ss_nibbles_to_bf16(wd), d);
          }
          const float sf = pick_half(svw[j], my_half);
          const float bf = pick_half(bvw[j], my_half);
          const float s16 = sf * kNibbleScale;
          const float bp = my_part ? 0.f : __builtin_fmaf(-kNibbleScale, sf, bf);
#pragma unroll
          for (int r = 0; r < NTK; ++r) {
            acc[r] = __builtin_fmaf(s16, d[r], acc[r]);
            acc[r] = __builtin_fmaf(bp, vr[r] ? hsv[j][r] : 0.f, acc[r]);
          }
        }
#pragma unroll
        for (int r = 0; r < NTK; ++r) {
          acc[r] = ss_rows_sum(acc[r]);
          if (g == 0) partl[((size_t)u * 16 + n) * kTBv + r] = acc[r];
        }
      };
      using Two = std::integral_constant<int, 2>;
      using Four = std::integral_constant<int, kTBv>;
      if (D.stage_h && nt <= 2) {
#pragma unroll 1
        for (int u = u0 + w; u < nu && u < u0 + D.P; u += 4) expert(u, std::true_type{}, Two{});
      } else if (D.stage_h) {
#pragma unroll 1
        for (int u = u0 + w; u < nu && u < u0 + D.P; u += 4) expert(u, std::true_type{}, Four{});
      } else {
#pragma unroll 1
        for (int u = u0 + w; u < nu && u < u0 + D.P; u += 4) expert(u, std::false_type{}, Four{});
      }
    }
    SS_TRACE(10);
    if (verify) {
      // The prefetch region is free once every wave is past its down experts; hs goes there.
      __syncthreads();
      float* hsl = reinterpret_cast<float*>(prefl);
      shared_hs_all<NSC>(a, shin, gsh, ush, w, nt, hsl);
      __syncthreads();
      float o[4][kTBv];
      shared_down_rows<4, NSC, SHQ4>(a, hsl, shw, nt, o);
      if (a.trace && tid == 0) a.trace[(size_t)bid * 16 + 13] = __builtin_amdgcn_s_memrealtime();
      if (lane == 0)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
#pragma unroll
          for (int t = 0; t < kTBv; ++t) s.shv[4 * w + rr][t] = o[rr][t];
    }
    __syncthreads();
    if (tid < 16 * kTBv) {
      const int c = tid >> 2, r = tid & 3;
      if (r < nt) {
        // Every operand of the K terms is read before the first sum (K <= kMaxQv / kTBv; absent terms read entry 0
        // and are dropped by the select), then the terms are added in rank order.
        constexpr int KM = kMaxQv / kTBv;
        float ov[KM];
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          const int q = r * K + (k < K ? k : 0), u = s.use_u[q];
          const float pv = partl[((size_t)(u >= 0 ? u : 0) * 16 + c) * kTBv + r];
          ov[k] = k < K && u >= 0 ? pv * s.wts[q] : 0.f;
        }
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          if (k < K) {
            if (a.o_buf) a.o_buf[((size_t)r * K + k) * H + 16 * bid + c] = ov[k];
            acc = k == 0 ? ov[k] : acc + ov[k];
          }
        }
        if (a.out) a.out[(size_t)r * H + 16 * bid + c] = acc;
        if (verify) {
          const float shb = ss_round_bf16(s.shv[c][r]);
          const float sgx = ss_bf16_to_f32(sgl_pre);
          const float sgv = ss_round_bf16(1.f / (1.f + ss_expf(-sgx)));
          const float sh2 = ss_round_bf16(sgv * shb);
          const uint32_t yb = ss_f32_to_bf16(ss_round_bf16(acc) + sh2);
          a.y[(size_t)r * H + 16 * bid + c] = (uint16_t)yb;
          if (a.x_plus_y) {  // the residual stream of the next layer
            const float xv = ss_bf16_to_f32(static_cast<const uint16_t*>(a.x)[(size_t)r * H + 16 * bid + c]);
            a.x_plus_y[(size_t)r * H + 16 * bid + c] = (uint16_t)ss_f32_to_bf16(xv + ss_bf16_to_f32(yb));
          }
        }
      }
    }
  }

  // ------------------------------------------------------------ exit: the last workgroup resets the counters
  __syncthreads();
  SS_TRACE(11);
#undef SS_TRACE
  if (tid == 0) {
    // Two-level exit ticket: the last workgroup of each shard takes a ticket on the top counter; the last of those
    // resets every shard (all other workgroups have made their last counter access).
    const int sh = bid % kShards;
    const int in_shard = (G - sh + kShards - 1) / kShards;
    const int t1 = __hip_atomic_fetch_add(shard(ctr, CTR_EXIT, sh), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t1 == in_shard - 1) {
      const int t2 = __hip_atomic_fetch_add(shard(ctr, CTR_TOP, 0), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (t2 == (G < kShards ? G : kShards) - 1) {
        for (int c = 0; c < CTR_COUNT; ++c)
          if (c != CTR_EPOCH)
            for (int q = 0; q < kShards; ++q)
              __hip_atomic_store(shard(ctr, c, q), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(shard(ctr, CTR_EPOCH, 0), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <int NJG, int NJD, bool XF32, bool SHQ4>
static hipError_t launch_nj(const VerifyArgs& a, hipStream_t st) {
  const SsRecord rec = ss_record_layout(a.H, a.I);
  auto kern = verify_kernel<NJG, NJD, XF32, SHQ4>;
  const DLayout dly = dlayout(a.T, a.H, a.I, a.K, a.E, XF32 ? 1 : 0, a.mode == 0 ? 1 : 0);
  // Every workgroup waits on the others, so the grid is one workgroup per CU and is launched only if a workgroup
  // with the largest dynamic LDS this kernel takes fits on a CU (checked once per device).
  KernelCfg cfg;
  hipError_t e = kernel_cfg(reinterpret_cast<const void*>(kern), 256, kLdsBudget, &cfg);
  if (e != hipSuccess) return e;
  if (cfg.per_cu < 1) return hipErrorCooperativeLaunchTooLarge;
  // A workgroup may hold at most 160 KB of LDS on gfx950; refuse any shape whose layout would exceed it.
  if (dly.P < 1 || dly.total > kLdsBudget || cfg.lds_static + dly.total > 160 * 1024) return hipErrorInvalidConfiguration;
  // The shared expert's hs [T][Is] fp32 reuses the prefetch region at the end of phase D.
  if (a.mode == 0 && (size_t)a.T * a.Is * 4 > dly.total - dly.pref) return hipErrorInvalidConfiguration;
  const int grid = cfg.cus;
  if (grid < a.H / 16) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), dly.total, st, a, rec);
  return hipGetLastError();
}

}  // namespace ss
