// A chain of MoE verify layers in one persistent launch (T <= 4 tokens): the verify step's MoE layers, each with
// the RMSNorm before it and the residual add after it (GraphSet._moe, runtime/graphs.py:160-169, one stream and
// unit injection; model/layers.py:336-402; reference_torch.py:30-38, 118-134).
//
// Each layer runs the phases of the single-layer verify kernel (ss_verify.hip) with the same operations in the same
// order, so every layer's ids, weights, y and stream carry the bits of separate ssmoe_moe_verify_layer_chain
// launches. What the chain changes is what waits for what:
//   * the stream passes from layer to layer as tagged words (tag << 32 | two bf16), double-buffered by layer
//     parity: the next layer polls the words themselves, one memory round trip, no counter and no launch;
//   * while a layer's experts stream, every wave issues the reads the next layer starts with: its router or
//     shared-expert rows, the map entries and routing bias of the next layer, and (workgroups with output rows) the
//     next layer's shared down rows, so the next layer's dense rows need only the stream;
//   * the shared expert's down rows are formed by the workgroups without output rows once their items are done
//     (workgroup H/16 + b for the rows of workgroup b), gated by sigmoid(x w_sg) there, and handed to the combine as
//     tagged words, so the workgroups with output rows only wait for the routed items;
//   * items are counted per wave, so a wave's items are visible without waiting for the other waves of its
//     workgroup.
// Counters are cumulative over the layers of a launch and tags are the launch epoch plus the layer index, so no
// state is reset between layers. Router logits are double-buffered by layer parity as well: a workgroup without
// items may still read layer l's logits while layer l + 1 writes its own. Every wave owns a router or shared row in
// every layer (the host checks E + Is >= 4 * grid), and that row needs the previous layer's whole stream, so no
// workgroup falls more than one layer behind the slowest.
// Waits are bounded: on timeout a kernel raises SS_ERR_TIMEOUT and goes on, so every workgroup reaches the exit.
#include "ss_verify_dev.hpp"

namespace ss {

namespace {

// Chain counters have one shard per lane of the wave that polls them (64), and each wave adds to shard
// (4 * workgroup + wave) % 64: with about a thousand waves signalling the items at once, 16 shards queued some 60
// atomic adds on each line at the memory-side atomic unit, which delayed the moment the count was complete.
constexpr int kCShards = 64;
SS_DEV int* cshard(int* ctr, int c, int s) { return ctr + (c * kCShards + s) * kShardStride; }
SS_DEV void csignal_add(int* ctr, int c, int v, int who) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __hip_atomic_fetch_add(cshard(ctr, c, who % kCShards), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct CLayout {
  size_t ctr, logits, sw, shx, gsh, ush, sgl, hfrag, hsum8, total;
};

__host__ __device__ inline CLayout clayout(int T, int H, int I, int Is, int K, int E) {
  (void)T;
  CLayout l;
  size_t o = 0;
  l.ctr = o;
  o = al256(o + (size_t)CTR_COUNT * kCShards * kShardStride * 4);
  l.logits = o;  // [2][kTBv][E] words: tag << 32 | bf16 logit
  o = al256(o + (size_t)2 * kTBv * E * 8);
  l.sw = o;  // [2][kTBv][H / 2] words: tag << 32 | two bf16 of the stream
  o = al256(o + (size_t)2 * kTBv * (H / 2) * 8);
  l.shx = o;  // [kTBv][H] words: tag << 32 | the gated shared-expert output bf16(bf16(sigmoid(sgl)) * bf16(sh))
  o = al256(o + (size_t)kTBv * H * 8);
  l.gsh = o;
  o = al256(o + (size_t)kTBv * Is * 2);
  l.ush = o;
  o = al256(o + (size_t)kTBv * Is * 2);
  l.sgl = o;
  o = al256(o + (size_t)kTBv * 2);
  l.hfrag = o;
  o = al256(o + (size_t)kTBv * K * I * 4);
  l.hsum8 = o;
  o = al256(o + (size_t)kTBv * K * (I / 8) * 4);
  l.total = o;
  return l;
}

// Dynamic LDS: per-expert partial dots | one region holding, in turn, the stream copy (x staging), the shared
// expert's hs (before the routed down rows) and the staged h fragments | the x fragments and the layer's norm
// weights, then the down prefetch.
struct CDLayout {
  size_t part, hreg, pref, total, slot;
  int P, stage_h;
};

__host__ __device__ inline CDLayout cdlayout(int T, int H, int I, int Is, int K, int E) {
  CDLayout d;
  const int nq = T * K;
  const int nu_max = nq < E ? nq : E;
  const size_t xf = (size_t)(H / 128) * 4 * 4 * kTBv * 16;
  d.slot = dslot_bytes(I);
  d.part = 0;
  size_t o = (size_t)nu_max * 16 * kTBv * 4;
  d.hreg = o;
  const size_t hf = (size_t)nq * I * 4;
  const size_t scopy = (size_t)kTBv * H * 2, hsl = (size_t)kTBv * Is * 4;
  size_t small = scopy > hsl ? scopy : hsl;
  const size_t tail = xf > d.slot ? xf : d.slot;
  d.stage_h = o + (hf > small ? hf : small) + tail <= kLdsBudget;
  o += d.stage_h ? (hf > small ? hf : small) : small;
  d.pref = o;
  const long room = (long)kLdsBudget - (long)o;
  int P = room > 0 ? (int)(room / (long)d.slot) : 0;
  if (P > nu_max) P = nu_max;
  d.P = P;
  const size_t pb = (size_t)P * d.slot, xw = xf + (size_t)H * 2;  // x fragments, then the norm weights
  d.total = o + (pb > xw ? pb : xw);
  return d;
}

// x fragments and group sums of T tokens from `src` ([T][H] bf16 in global memory or LDS), replacing every element by
// bf16((x * r_t) * norm_w) when `norm` (r_t = 1 / sqrt(sum(x^2) / H + eps) of token t in the ssmoe_residual_rmsnorm
// order): the operations of stage_x for bf16 x.
template <int NJG>
SS_DEV void stage_x_src(const uint16_t* src, bool norm, const uint16_t* nw_lds, float eps, int H, uint4* xfl,
                        float (*gx)[kTBv], float* rnorm, int nt) {
  const int tid = threadIdx.x;
  constexpr int NJX = NJG / 4;
  uint4 nv[NJX];
  if (norm) {
    const int tn = (tid >> 6) < nt ? (tid >> 6) : 0;
#pragma unroll
    for (int jj = 0; jj < NJX; ++jj)
      nv[jj] = *reinterpret_cast<const uint4*>(src + (size_t)tn * H + 8 * (64 * jj + (tid & 63)));
  }
  constexpr int NF = NJG * 16 * kTBv;
  constexpr int FPT = NF / 256;
  static_assert(NF % 256 == 0, "whole fragment entries per thread");
  uint4 fv[FPT];
#pragma unroll
  for (int k = 0; k < FPT; ++k) {
    const int f = tid + 256 * k;
    const int t = f & 3, gg = (f >> 2) & 3, i = (f >> 4) & 3, j = f >> 6;
    const int tt = t < nt ? t : 0;
    fv[k] = *reinterpret_cast<const uint4*>(src + (size_t)tt * H + 128 * j + 32 * gg + 8 * i);
  }
  uint4 gv[8];
  const int q = tid < (H >> 6) * kTBv ? tid : 0;
  const int gt = (q & 3) < nt ? (q & 3) : 0;
  const int Gi = q >> 2;
  if (!norm) {
#pragma unroll
    for (int k = 0; k < 8; ++k) gv[k] = *reinterpret_cast<const uint4*>(src + (size_t)gt * H + 64 * Gi + 8 * k);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (norm) {
    float acc = 0.f;
#pragma unroll
    for (int jj = 0; jj < NJX; ++jj) {
      const uint32_t v[4] = {nv[jj].x, nv[jj].y, nv[jj].z, nv[jj].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float e0 = bf_lo(v[c]), e1 = bf_hi(v[c]);
        acc = fmaf(e0, e0, acc);
        acc = fmaf(e1, e1, acc);
      }
    }
    const float ssum = ss_wave_sum(acc);
    if ((tid & 63) == 0) rnorm[tid >> 6] = 1.f / sqrtf(ssum / (float)H + eps);
    __syncthreads();
    auto scale8 = [&](uint4 v, float r, int k0) {
      const uint32_t x4[4] = {v.x, v.y, v.z, v.w};
      uint32_t o[4];
      if (nw_lds) {
        const uint4 wv = *reinterpret_cast<const uint4*>(nw_lds + k0);
        const uint32_t w4[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          o[c] = ss_f32_to_bf16((bf_lo(x4[c]) * r) * bf_lo(w4[c])) |
                 (ss_f32_to_bf16((bf_hi(x4[c]) * r) * bf_hi(w4[c])) << 16);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          o[c] = ss_f32_to_bf16(bf_lo(x4[c]) * r) | (ss_f32_to_bf16(bf_hi(x4[c]) * r) << 16);
      }
      return make_uint4(o[0], o[1], o[2], o[3]);
    };
#pragma unroll
    for (int k = 0; k < FPT; ++k) {
      const int f = tid + 256 * k;
      const int t = f & 3, gg = (f >> 2) & 3, i = (f >> 4) & 3, j = f >> 6;
      const int tt = t < nt ? t : 0;
      fv[k] = scale8(fv[k], rnorm[tt], 128 * j + 32 * gg + 8 * i);
    }
  }
#pragma unroll
  for (int k = 0; k < FPT; ++k) {
    const int f = tid + 256 * k;
    const bool live = (f & 3) < nt;
    const uint4 pv = perm_pairs(fv[k]);
    xfl[f] = make_uint4(live ? pv.x : 0u, live ? pv.y : 0u, live ? pv.z : 0u, live ? pv.w : 0u);
  }
  if (norm) return;  // the group sums come from the staged fragments later (xfrag_group_sums)
  if (tid < (H >> 6) * kTBv) {
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint4 v = gv[k];
      sum = sum + bf_lo(v.x);
      sum = sum + bf_hi(v.x);
      sum = sum + bf_lo(v.y);
      sum = sum + bf_hi(v.y);
      sum = sum + bf_lo(v.z);
      sum = sum + bf_hi(v.z);
      sum = sum + bf_lo(v.w);
      sum = sum + bf_hi(v.w);
    }
    gx[Gi][q & 3] = (q & 3) < nt ? sum : 0.f;
  }
}

// Group sum q (group q >> 2 of token q & 3, sequential in element order) of the normalized x, from the staged
// fragments: the stage_x_src sums when it normalizes, formed once the fragments are visible to the whole workgroup.
SS_DEV void xfrag_group_sums(const uint4* xfl, float (*gx)[kTBv], int q, int nt) {
  const int Gi = q >> 2, gt = (q & 3) < nt ? (q & 3) : 0;
  uint4 v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = xfl[xfrag_index(64 * Gi + 8 * k, gt)];
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    sum = sum + bf_lo(v[k].x);
    sum = sum + bf_lo(v[k].y);
    sum = sum + bf_lo(v[k].z);
    sum = sum + bf_lo(v[k].w);
    sum = sum + bf_hi(v[k].x);
    sum = sum + bf_hi(v[k].y);
    sum = sum + bf_hi(v[k].z);
    sum = sum + bf_hi(v[k].w);
  }
  gx[Gi][q & 3] = (q & 3) < nt ? sum : 0.f;
}

// The fields the shared device helpers read, for one layer.
SS_DEV VerifyArgs helper_args(const ChainArgs& a, const ssmoe_chain_layer& lp) {
  VerifyArgs v{};
  v.mode = 0;
  v.bias = lp.router_bias;
  v.sh_down = lp.sh_down;
  v.sh_gs = lp.sh_gate_s;
  v.sh_gb = lp.sh_gate_b;
  v.sh_us = lp.sh_up_s;
  v.sh_ub = lp.sh_up_b;
  v.sh_ds = lp.sh_down_s;
  v.sh_db = lp.sh_down_b;
  v.map = a.map;
  v.map_len = a.map_len;
  v.slot_ptr = a.slot_ptr;
  v.n_slots = a.n_slots;
  v.map_base = lp.layer * a.E;
  v.T = a.T;
  v.H = a.H;
  v.I = a.I;
  v.Is = a.Is;
  v.K = a.K;
  v.E = a.E;
  v.err = a.err;
  v.trace = nullptr;
  return v;
}

// A layer entry staged in LDS (by read_layer_dma) into scalar registers.
constexpr int kLayerDwords = sizeof(ssmoe_chain_layer) / 4;
static_assert(sizeof(ssmoe_chain_layer) % 4 == 0 && kLayerDwords <= 64, "whole dwords, one per lane");
SS_DEV ssmoe_chain_layer layer_from_lds(const uint32_t* lds) {
  uint32_t v[kLayerDwords];
#pragma unroll
  for (int i = 0; i < kLayerDwords; ++i) v[i] = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds[i]);
  ssmoe_chain_layer r;
  __builtin_memcpy(&r, v, sizeof r);
  return r;
}

}  // namespace

size_t chain_scratch_bytes(int T, int H, int I, int Is, int K, int E) { return clayout(T, H, I, Is, K, E).total; }

// A wait of the chain kernel gives up after kChainSpin polls (each a memory round trip, well under a second in all),
// raises SS_ERR_TIMEOUT and marks the workgroup dead: every later wait of that workgroup returns at once, so a launch
// whose hand-offs failed still ends within about a second. The polls do not sleep between round trips: measured on
// MI355X, the hand-offs complete about 0.15 us sooner per layer than with a short sleep in each poll.
constexpr int kChainSpin = 1 << 18;

template <int NJG, int NJD, bool SHQ4>
__global__ __launch_bounds__(256) void chain_kernel(ChainArgs a, SsRecord rec) {
  extern __shared__ uint4 dsm[];
  __shared__ VSmem s0;
  __shared__ int s_dead;
  __shared__ alignas(16) uint32_t s_next[64];  // the next layer's entry, read by a direct-to-LDS load
  // Trace stamps of the last two layers, kept in LDS and written out at the exit, so that no stamp is a global
  // store the next wait for memory would include.
  __shared__ uint64_t s_tr[2][32];
  uint8_t* dl = reinterpret_cast<uint8_t*>(dsm);
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, bid = blockIdx.x;
  const int n = lane & 15, g = lane >> 4;
  const int T = a.T, H = a.H, I = a.I, K = a.K, E = a.E, Is = a.Is, NL = a.NL;
  const CLayout L = clayout(T, H, I, Is, K, E);
  uint8_t* scr = static_cast<uint8_t*>(a.scratch);
  int* ctr = reinterpret_cast<int*>(scr + L.ctr);
  if (tid == 0) s_dead = 0;
  if (tid < 64) (&s_tr[0][0])[tid] = 0ull;
  __syncthreads();
  auto give_up = [&]() {
    if (lane == 0) {
      ss_raise(a.err, SS_ERR_TIMEOUT);
      __hip_atomic_store(&s_dead, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  auto dead = [&]() { return __hip_atomic_load(&s_dead, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0; };
  // One full wave waits until the shards of counter c sum to at least target (the order of wait_ge).
  auto wait_ctr = [&](int c, int target) {
    int* p = cshard(ctr, c, lane);
    for (int it = 0;; ++it) {
      if (dead()) break;
      const int v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int total = (int)ss_butterfly((uint32_t)v, [](uint32_t x, uint32_t y) { return x + y; });
      if (total >= target) break;
      if (it >= kChainSpin) {
        give_up();
        break;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  };
  const int nt = T;
  const CDLayout D = cdlayout(T, H, I, Is, K, E);
  const uint32_t tag0 = (uint32_t)ld_ag(cshard(ctr, CTR_EPOCH, 0)) + 1u;  // layer l's tag: tag0 + l
  constexpr int NJX = NJG / 4;
  constexpr int NV = kMaxEv / 64;
  const int J = E + Is, W = G * 4;
  // Router rows go to the workgroups without output rows: they finish a layer first, so the next layer's logits do
  // not wait for the workgroups that write its stream.
  const int j_first = ((bid + G - (H >> 4)) % G) * 4 + w;
  const bool has_tile = bid < (H >> 4);
  const int tiles = I >> 3;
  const int my_half = g >> 1, my_part = g & 1;
  const int drow = 16 * bid + n;
  const int64_t drow_b = I >> 1, dsb_b = (I >> 6) * 2;
  const int64_t row_b = H >> 1, sb_b = (H >> 6) * 2;

  ssmoe_chain_layer lp = a.l0;
  uint4 r0[NJX], r1[NJX], r2[NJX];
  // Dense-row jobs: j < E is router row j; E <= j < E + Is the shared gate and up rows j - E; the last job also takes
  // the shared_expert_gate row (as the single-layer kernel).
  auto load_job = [&](const ssmoe_chain_layer& q, int j) {
    if (SHQ4 && j >= E) {
      // affine 4-bit shared gate and up rows: q4_chunk registers
      const size_t r = (size_t)(j - E);
#pragma unroll
      for (int jj = 0; jj < NJX; ++jj) {
        r0[jj] = q4_chunk(q.sh_gate + r * (H / 4), q.sh_gate_s + r * (H / 64), q.sh_gate_b + r * (H / 64), jj, lane);
        r1[jj] = q4_chunk(q.sh_up + r * (H / 4), q.sh_up_s + r * (H / 64), q.sh_up_b + r * (H / 64), jj, lane);
      }
    } else {
      const uint16_t* w0 = j < E ? q.router_w + (size_t)j * H : q.sh_gate + (size_t)(j - E) * H;
#pragma unroll
      for (int jj = 0; jj < NJX; ++jj) r0[jj] = ldg16(w0 + 8 * (64 * jj + lane));
      if (j >= E) {
        const uint16_t* w1 = q.sh_up + (size_t)(j - E) * H;
#pragma unroll
        for (int jj = 0; jj < NJX; ++jj) r1[jj] = ldg16(w1 + 8 * (64 * jj + lane));
      }
    }
    if (j == J - 1) {
#pragma unroll
      for (int jj = 0; jj < NJX; ++jj) r2[jj] = ldg16(q.sh_g + 8 * (64 * jj + lane));
    }
  };
  int slot_e[2] = {-1, -1};
  auto load_map = [&](const ssmoe_chain_layer& q) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int e = tid + 256 * k;
      const int64_t mi = q.layer * E + e;
      const bool ok = e < E && mi >= 0 && mi < a.map_len;
      const int v = gp(a.map)[ok ? mi : 0];
      slot_e[k] = ok ? v : -1;
    }
  };
  // The slot pointers are loaded without a select on the loaded value (an entry outside the table reads slot 0 and
  // is cleared where the tables are written), so no wait for them follows the load.
  int64_t base_k[2] = {0, 0};
  auto slot_ok = [&](int k) { return slot_e[k] >= 0 && (int64_t)slot_e[k] < a.n_slots; };
  auto load_bases = [&]() {
#pragma unroll
    for (int k = 0; k < 2; ++k) base_k[k] = gp(a.slot_ptr)[slot_ok(k) ? slot_e[k] : 0];
  };
  float bias_r[NV];
  auto load_bias = [&](const ssmoe_chain_layer& q) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + 64 * i;
      bias_r[i] = q.router_bias ? gp(q.router_bias)[e < E ? e : 0] : 0.f;
    }
  };
  constexpr int NSC = NJD > 4 ? 2 : 1;  // 512-element chunks of a shared down row per lane (Is <= 512 * NSC)
  uint4 shw[4][NSC];

  if (j_first < J) load_job(lp, j_first);
  load_map(lp);
  load_bias(lp);
  int items_target = 0;

#pragma unroll 1
  for (int l = 0; l < NL; ++l) {
    const uint32_t tag = tag0 + (uint32_t)l;
    const bool tr = a.trace && l >= NL - 2;
    uint64_t* trs = s_tr[l == NL - 1 ? 1 : 0];  // stamps 0-15 go to the layer's row, 16-31 to its extra row
#define SS_TRACE(k)                                                   \
  do {                                                                \
    if (tr && tid == 0) trs[(k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
    SS_TRACE(0);
    // Offsets of the dynamic LDS regions, made opaque to the compiler at every layer so that the LDS addresses
    // derived from them are formed where they are used rather than hoisted out of the layer loop (where dozens of
    // them would stay live across every phase and spill).
    size_t o_part = D.part, o_hreg = D.hreg, o_pref = D.pref;
    uint32_t o_s = 0;
    size_t o_w = 0;
    asm volatile("" : "+s"(o_part), "+s"(o_hreg), "+s"(o_pref), "+s"(o_s), "+s"(o_w));
    VSmem& s = *reinterpret_cast<VSmem*>(reinterpret_cast<uint8_t*>(&s0) + o_s);
    uint8_t* scw = scr + o_w;
    uint64_t* logits_all = reinterpret_cast<uint64_t*>(scw + L.logits);
    uint64_t* sw_all = reinterpret_cast<uint64_t*>(scw + L.sw);
    uint16_t* gsh = reinterpret_cast<uint16_t*>(scw + L.gsh);
    uint16_t* ush = reinterpret_cast<uint16_t*>(scw + L.ush);
    uint16_t* sgl = reinterpret_cast<uint16_t*>(scw + L.sgl);
    uint64_t* shx = reinterpret_cast<uint64_t*>(scw + L.shx);
    uint4* hfrag = reinterpret_cast<uint4*>(scw + L.hfrag);
    float* hsum8 = reinterpret_cast<float*>(scw + L.hsum8);
    uint4* xfl = reinterpret_cast<uint4*>(dl + o_pref);
    uint4* hfl = reinterpret_cast<uint4*>(dl + o_hreg);
    uint16_t* scopy = reinterpret_cast<uint16_t*>(dl + o_hreg);
    float* hsl = reinterpret_cast<float*>(dl + o_hreg);
    float* partl = reinterpret_cast<float*>(dl + o_part);
    uint8_t* prefl = dl + o_pref;
    const VerifyArgs va = helper_args(a, lp);
    // The next layer's entry: one dword per lane of wave 3 straight into LDS, read at the end of this layer (no
    // register waits for it in between; wave 3 has no stores in flight at the end of a layer).
    if (l + 1 < NL && w == 3 && lane < kLayerDwords)
      dma4(reinterpret_cast<const uint32_t*>(a.more + l) + lane, s_next);
    // The layer's norm weights go straight into LDS behind the x fragments (wave 2, waited for before the staging),
    // so the staging that follows the stream's arrival reads no global memory.
    uint16_t* nwl = reinterpret_cast<uint16_t*>(xfl + NJG * 16 * kTBv);
    if (lp.norm_w && w == 2)
      for (int i = 0; i < (H >> 9); ++i) dma16(lp.norm_w + 8 * (64 * i + lane), reinterpret_cast<uint8_t*>(nwl) + 1024 * i);
    for (int i = tid; i < kMaxQv * kTBv; i += 256) (&s.umask[0][0])[i] = 0u;
    if (tid < 4) s.zero_h[tid] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 0) s.nt = nt;

    // ---------------------------------------------------------- x: the stream of the previous layer
    // Always staged from the LDS copy, so that every read of x below is an LDS read (a read through a pointer that
    // may be global is a flat access, which waits for every load the wave has in flight, the next layer's prefetches
    // included).
    const bool norm = l > 0 || a.norm_in != 0;
    if (l == 0) {
      const int nw = nt * (H >> 3);  // 16-byte words of the input rows
      uint4* dst = reinterpret_cast<uint4*>(scopy);
      for (int idx = tid; idx < nw; idx += 256) dst[idx] = ldg16(a.stream_in + 8 * (size_t)idx);
      __syncthreads();
    } else {
      // Copy the previous layer's stream words into LDS as plain bf16 [T][H], polling until each word carries that
      // layer's tag.
      const uint64_t* src = sw_all + (size_t)((l - 1) & 1) * kTBv * (H / 2);
      const uint32_t want = tag - 1u;
      const int nw = nt * (H >> 1);
      uint32_t* dst = reinterpret_cast<uint32_t*>(scopy);
      SS_TRACE(16 + 2);
#pragma unroll 1
      for (int k0 = 0; k0 < nw; k0 += 256 * 8) {
        uint64_t v[8];
        for (int it = 0;; ++it) {
          bool fresh = true;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const int idx = k0 + tid + 256 * k;
            v[k] = idx < nw ? ld_ag(src + idx) : 0ull;
            fresh = fresh && (idx >= nw || (uint32_t)(v[k] >> 32) == want);
          }
          if (it == 0) SS_TRACE(16 + 1);
          if (__all(fresh) || dead()) {
            if (tr && tid == 0) trs[14] = (uint64_t)it;
            break;
          }
          if (it >= kChainSpin) {
            give_up();
            break;
          }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int idx = k0 + tid + 256 * k;
          if (idx < nw) dst[idx] = (uint32_t)v[k];
        }
      }
      SS_TRACE(5);
      __syncthreads();
    }
    const uint16_t* xsrc = scopy;
    if (w == 2) __builtin_amdgcn_s_waitcnt(0);  // the norm weights have landed in LDS
    stage_x_src<NJG>(xsrc, norm, lp.norm_w ? nwl : nullptr, a.eps, H, xfl, s.gx, s.rnorm, nt);
    // The residual stream value of the combine's (row, token), read before the shared region is reused.
    uint32_t xres = 0;
    if (has_tile && tid < 16 * kTBv && (tid & 3) < nt) xres = xsrc[(size_t)(tid & 3) * H + 16 * bid + (tid >> 2)];
    __syncthreads();
    SS_TRACE(1);

    // ---------------------------------------------------------- phase A: dense rows
    uint64_t* logits = logits_all + (size_t)(l & 1) * kTBv * E;
#pragma unroll 1
    for (int j = j_first; j < J; j += W) {
      if (j != j_first) load_job(lp, j);
      const int nrow = j < E ? 1 : (j == J - 1 ? 3 : 2);
#pragma unroll 1
      for (int q = 0; q < nrow; ++q) {
        float d[kTBv];
        if (SHQ4 && j >= E && q < 2)
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
    SS_TRACE(16 + 4);
    // Router rows need no wait (their words carry the tag). A wave with shared rows publishes them once its own
    // stores are acknowledged: at once, or, for a wave that runs a router tail, after the tail (the shared rows are
    // first read after the items, so the tail does not wait for the acknowledgement).
    int ns = 0;
    for (int j = j_first; j < J; j += W)
      if (j >= E) ns += j == J - 1 ? 2 : 1;
    auto publish_shared = [&]() {
      if (ns) {
        stores_done();
        if (lane == 0) csignal_add(ctr, CTR_SHARED, ns, 4 * bid + w);
      }
    };
    if (w >= nt) publish_shared();
    // The slot pointers go out now; the waves without a router tail store the table entries while the tail waves
    // work, the tail waves after their tail (the tables are first read by the unique-expert list).
    load_bases();
    auto write_tables = [&]() {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int e = tid + 256 * k;
        if (e < E) {
          s.map[e] = slot_e[k];
          s.base_e[e] = slot_ok(k) ? reinterpret_cast<const uint8_t*>(base_k[k]) : nullptr;
        }
      }
    };
    if (w >= nt) write_tables();
    SS_TRACE(2);

    // ---------------------------------------------------------- phase B: router tail, unique experts
    if (w < nt && !dead()) router_tail_wave(va, logits, tag, w, s, bias_r, tr && w == 0 ? trs + 24 : nullptr);
    if (w < nt) {
      SS_TRACE(16 + 10);
      write_tables();
      publish_shared();
    }
    __syncthreads();
    SS_TRACE(3);
    if (bid == 0 && tid < nt * K) {
      gp(lp.ids)[tid] = s.ids[tid];
      gp(lp.weights)[tid] = s.wts[tid];
    }
    if (tid < 64) {
      unique_setup(va, s, true);
    } else {
      // While wave 0 forms the unique list: the x group sums of a normalized stream (first read by the items) and
      // the zeros of the items' h sums.
      if (norm)
        for (int q = tid - 64; q < (H >> 6) * kTBv; q += 192) xfrag_group_sums(xfl, s.gx, q, nt);
      for (int i = tid - 64; i < kXZero; i += 192) reinterpret_cast<uint4*>(s.hsum)[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();
    SS_TRACE(4);
    const int nu = s.nu;
    const int n_items = nu * tiles;
    items_target += n_items;

    // ---------------------------------------------------------- phase C: gate/up items
    const int gw = ((bid - (H >> 4) + G) % G) * 4 + w;
    int wave_items = 0;
    for (int it = gw; it < n_items; it += W) ++wave_items;
    if (wave_items) {
      const int m = lane & 15, at = m & 3, agrp = m >> 2, ahh = agrp >> 1, apart = agrp & 1;
      const bool a_act = ahh == (g >> 1) && at < nt && apart == 0;
      // One instantiation per token count (2 or 4 accumulators): the dots, row sums and SwiGLU of absent tokens are
      // not formed.
      auto run_items = [&](auto ntk_c, auto lds_c) {
        constexpr int NTK = decltype(ntk_c)::value;
        constexpr bool LDS_SWIGLU = decltype(lds_c)::value;
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
          // The row's scales and biases in 16-byte loads first (four dwords each: a quarter of the requests of
          // dword loads), then the packed words in chunk order.
          static_assert(NJG % 4 == 0, "whole 16-byte scale loads");
#pragma unroll
          for (int j4 = 0; j4 < NJG / 4; ++j4) {
            const ss_u32x4 s4 = *(const SS_G ss_u32x4*)(srow + 4 * j4), b4 = *(const SS_G ss_u32x4*)(brow + 4 * j4);
            sv[4 * j4] = s4.x;
            sv[4 * j4 + 1] = s4.y;
            sv[4 * j4 + 2] = s4.z;
            sv[4 * j4 + 3] = s4.w;
            bv[4 * j4] = b4.x;
            bv[4 * j4 + 1] = b4.y;
            bv[4 * j4 + 2] = b4.z;
            bv[4 * j4 + 3] = b4.w;
          }
#pragma unroll
          for (int j = 0; j < NJG; ++j) wv[j] = ldg16(wrow + 64 * j);
          __builtin_amdgcn_sched_barrier(0);
          if (NJG == 16 && tr && item == gw) {
            // diagnostics (traced layers of the BASELINE shape only): the item's loads issued, then landed
            SS_TRACE(16 + 5);
            __builtin_amdgcn_s_waitcnt(0);
            SS_TRACE(16 + 6);
          }
          float acc[NTK];
#pragma unroll
          for (int r = 0; r < NTK; ++r) acc[r] = 0.f;
          constexpr int JB = NJG % 4 == 0 ? 4 : 1;
#pragma unroll
          for (int j0 = 0; j0 < NJG; j0 += JB) {
            uint4 av4[JB][4];
            float4 gxv[JB];
#pragma unroll
            for (int jj = 0; jj < JB; ++jj) {
              const int j = j0 + jj;
              const uint4* fp = a_act ? xfl + (size_t)(((j * 4) * 4 + g) * kTBv + at)
                                      : reinterpret_cast<const uint4*>(s.hsum);
#pragma unroll
              for (int i = 0; i < 4; ++i) av4[jj][i] = fp[(size_t)i * 16];
              gxv[jj] = reinterpret_cast<const float4*>(s.gx)[2 * j + my_half];
            }
            // The JB chunks' MFMA chains interleaved (slice i of every chunk, then slice i + 1), so that a chunk's
            // dependent MFMAs overlap the other chunks' instead of waiting on each other; each chunk's sum and the
            // accumulation below keep their order.
            ss_f32x4 dj[JB];
#pragma unroll
            for (int jj = 0; jj < JB; ++jj) dj[jj] = ss_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
              for (int jj = 0; jj < JB; ++jj) {
                const int j = j0 + jj;
                const uint32_t wd = i == 0 ? wv[j].x : i == 1 ? wv[j].y : i == 2 ? wv[j].z : wv[j].w;
                dj[jj] = ss_mfma(as_v(av4[jj][i]), ss_nibbles_to_bf16(wd), dj[jj]);
              }
            }
#pragma unroll
            for (int jj = 0; jj < JB; ++jj) {
              const int j = j0 + jj;
              const ss_f32x4 d = dj[jj];
              const float sf = pick_half(sv[j], my_half);
              const float bf = pick_half(bv[j], my_half);
              const float s16 = sf * kNibbleScale;
              const float bp = my_part ? 0.f : __builtin_fmaf(-kNibbleScale, sf, bf);
              const float gxa[kTBv] = {gxv[jj].x, gxv[jj].y, gxv[jj].z, gxv[jj].w};
#pragma unroll
              for (int r = 0; r < NTK; ++r) {
                acc[r] = __builtin_fmaf(s16, d[r], acc[r]);
                acc[r] = __builtin_fmaf(bp, gxa[r], acc[r]);
              }
            }
          }
          if (NJG == 16 && tr && item == gw) SS_TRACE(16 + 14);  // the item's dots formed
          if constexpr (!LDS_SWIGLU) {
            // Every lane of column n now gets row n's dot of each token (gate row n for n < 8, up row n - 8 above),
            // and the lanes n < 8 form h = silu(gate) * up of their row c = n from the up dot 8 lanes up: no LDS.
            float hq[NTK];
#pragma unroll
            for (int r = 0; r < NTK; ++r) {
              const float gd = ss_rows_sum(acc[r]);
              const float ud = ss_uf(ss_xor_lane<8>(ss_fu(gd)));
              hq[r] = gd / (1.f + ss_expf(-gd)) * ud;
            }
            const int jf = p >> 4, gf = (p & 15) >> 2, ifr = p & 3;
            const uint32_t mk_l = lane < nt ? s.umask[u][lane] : 0u;
#pragma unroll
            for (int r = 0; r < NTK; ++r) {
              if (r >= nt) break;
              uint32_t mk = (uint32_t)__builtin_amdgcn_readlane((int)mk_l, r);
              if (!mk) continue;
              // h of token r as bf16 high parts and bf16 residuals: lanes 0-3 hold word c of the high parts (rows c,
              // c + 4), lanes 4-7 word c - 4 of the residuals; lane 8 the sequential sum of the 8 h values.
              const float h = hq[r];
              const uint32_t a0 = ss_f32_to_bf16(h), lo = ss_f32_to_bf16(h - ss_bf16_to_f32(a0));
              const uint32_t a0p = ss_xor_lane<4>(a0), lop = ss_xor_lane<4>(lo);
              const uint32_t word = n < 4 ? (a0 | (a0p << 16)) : (lop | (lo << 16));
              float sum8 = 0.f;
#pragma unroll
              for (int c = 0; c < 8; ++c) sum8 = sum8 + ss_readlane_f(h, c);
              while (mk) {
                const int k = __ffs(mk) - 1;
                mk &= mk - 1;
                const int q = r * K + k;
                uint32_t* fpo = reinterpret_cast<uint32_t*>(hfrag + (((size_t)q * NJD + jf) * 4 + gf) * 8 + ifr);
                if (lane < 8)
                  st_ag(fpo + (lane < 4 ? lane : 12 + lane), word);
                else if (lane == 8)
                  st_ag(reinterpret_cast<uint32_t*>(hsum8) + (size_t)q * (I >> 3) + p, __float_as_uint(sum8));
              }
            }
          } else {
            // more tokens: the SwiGLU and h packing through the wave's LDS rows (one (token, row) per lane)
            float* xch = s.xch[w];
#pragma unroll
            for (int r = 0; r < NTK; ++r) {
              acc[r] = ss_rows_sum(acc[r]);
              if (g == 0) xch[n * kTBv + r] = acc[r];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            {
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
                lw[d] = ss_f32_to_bf16(hv[d] - ss_bf16_to_f32(a0)) |
                        (ss_f32_to_bf16(hv[d + 4] - ss_bf16_to_f32(a1)) << 16);
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
              }
            }
            __builtin_amdgcn_wave_barrier();
          }
          if (item == gw) SS_TRACE(16 + 7);
        }
      };
      // Up to two tokens: SwiGLU and h packing in registers. More: through the wave's LDS rows, which measured
      // faster at H 2048; at H 2560 the register file holds only the register form.
      if (nt <= 2)
        run_items(std::integral_constant<int, 2>{}, std::false_type{});
      else if constexpr (NJG > 16)
        run_items(std::integral_constant<int, kTBv>{}, std::false_type{});
      else
        run_items(std::integral_constant<int, kTBv>{}, std::true_type{});
      // Each wave publishes its own items as soon as its stores are acknowledged.
      stores_done();
      if (lane == 0) csignal_add(ctr, CTR_ITEMS, wave_items, 4 * bid + w);
    }
    SS_TRACE(7);

    __syncthreads();  // every wave is past its items: the x fragments are dead, the prefetch slots may be written

    if (!has_tile) {
      // ---------------------------------------------------------- the shared expert's rows of output blocks
      // ob = bid - H/16, + (G - H/16), ... (< H/16; the operations of the single-layer kernel's shared rows), gated and
      // published for the combines of those workgroups
      const int nfree = G - (H >> 4);
      int ob = bid - (H >> 4);
      load_shared_down<4, NSC, SHQ4>(va, 16 * ob + 4 * w, shw);
      wait_ctr(CTR_SHARED, (l + 1) * (Is + 1));
      const SharedIn shin = shared_load(va, gsh, ush, nt);
      const uint16_t sgl_t = ld_ag(sgl + ((lane & 3) < nt ? (lane & 3) : 0));
      shared_hs_all<NSC>(va, shin, gsh, ush, w, nt, hsl);
      __syncthreads();
      const float sgv = ss_round_bf16(1.f / (1.f + ss_expf(-ss_bf16_to_f32(sgl_t))));
#pragma unroll 1
      for (; ob < (H >> 4); ob += nfree) {
        if (ob != bid - (H >> 4)) load_shared_down<4, NSC, SHQ4>(va, 16 * ob + 4 * w, shw);
        float o[4][kTBv];
        shared_down_rows<4, NSC, SHQ4>(va, hsl, shw, nt, o);
        // lane 4 rr + t publishes row 16 ob + 4 w + rr of token t
        const int rr = (lane >> 2) & 3, t = lane & 3;
        float shv = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int u = 0; u < kTBv; ++u) shv = (q == rr && u == t) ? o[q][u] : shv;
        if (lane < 16 && t < nt) {
          const float shb = ss_round_bf16(shv);
          const uint32_t sh2 = ss_f32_to_bf16(sgv * shb);
          st_ag(shx + (size_t)t * H + 16 * ob + 4 * w + rr, ((uint64_t)tag << 32) | (uint64_t)sh2);
        }
      }
      SS_TRACE(13);
    }

    if (has_tile) {
      // ---------------------------------------------------------- down prefetch
      auto issue_down = [&](int u, int slotp) {
        uint8_t* sl = prefl + (size_t)slotp * D.slot;
        const uint8_t* base = s.base[u];
        for (int j = 0; j < NJD; ++j) dma16(base + rec.dw + drow * drow_b + 64 * j + 16 * g, sl + (size_t)j * 1024);
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
#pragma unroll 1
      for (int u = w; u < nu && u < D.P; u += 4) issue_down(u, u);

      // ---------------------------------------------------------- phase D: down + combine
      if (w == 0) wait_ctr(CTR_ITEMS, items_target);
      __syncthreads();
      SS_TRACE(8);
      // The gated shared-expert output of the combine's (row, token), requested now, checked at the combine.
      const size_t shx_i = (size_t)(tid & 3) * H + 16 * bid + (tid >> 2);
      uint64_t shx_w = tid < 16 * kTBv && (tid & 3) < nt ? ld_ag(shx + shx_i) : 0ull;
      const int nq = nt * K;
      const int hchunks = D.stage_h ? nq * I * 4 / 1024 : 0;
#pragma unroll 1
      for (int c = w; c < hchunks; c += 4)
        dma16_ag(reinterpret_cast<const uint8_t*>(hfrag) + (size_t)c * 1024 + 16 * lane,
                 reinterpret_cast<uint8_t*>(hfl) + (size_t)c * 1024);
      for (int idx = tid; idx < nq * (I >> 6); idx += 256) {
        const int q = idx / (I >> 6), Gi = idx - q * (I >> 6);
        float sum = 0.f;
        if (s.use_u[q] >= 0) {
          const float* hp = hsum8 + (size_t)q * (I >> 3) + 8 * Gi;
          const uint4 h0 = ld_ag16(hp), h1 = ld_ag16(hp + 4);
          const float hv[8] = {__uint_as_float(h0.x), __uint_as_float(h0.y), __uint_as_float(h0.z),
                               __uint_as_float(h0.w), __uint_as_float(h1.x), __uint_as_float(h1.y),
                               __uint_as_float(h1.z), __uint_as_float(h1.w)};
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
          // The NJD chunks' MFMA chains interleaved (slice i of every chunk, then slice i + 1); each chunk's sum and
          // the accumulation below keep their order.
          ss_f32x4 dj[NJD];
#pragma unroll
          for (int j = 0; j < NJD; ++j) dj[j] = ss_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < NJD; ++j) {
              ss_u32x4 av = as_v(av4[j][i]);
              if (!STAGED && !am) av = ss_u32x4{0u, 0u, 0u, 0u};
              const uint32_t wd = i == 0 ? wq[j].x : i == 1 ? wq[j].y : i == 2 ? wq[j].z : wq[j].w;
              dj[j] = ss_mfma(av, ss_nibbles_to_bf16(wd), dj[j]);
            }
          }
#pragma unroll
          for (int j = 0; j < NJD; ++j) {
            const ss_f32x4 d = dj[j];
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
          for (int u = u0 + w; u < nu && u < u0 + D.P; u += 4) {
            expert(u, std::true_type{}, Two{});
            if (u < 12) SS_TRACE(16 + 11 + (u >> 2));
          }
        } else if (D.stage_h) {
#pragma unroll 1
          for (int u = u0 + w; u < nu && u < u0 + D.P; u += 4) expert(u, std::true_type{}, Four{});
        } else {
#pragma unroll 1
          for (int u = u0 + w; u < nu && u < u0 + D.P; u += 4) expert(u, std::false_type{}, Four{});
        }
      }
      // No global load is issued inside the expert loop: a load in flight there makes every LDS read of the loop
      // wait for it (the loop's reads may alias the direct-to-LDS prefetch, so the compiler waits for all loads).
      // The shared word is requested again here, if the first request (issued with the h staging) was stale.
      if (w == 0 && tid < 16 * kTBv && (tid & 3) < nt && (uint32_t)(shx_w >> 32) != tag) shx_w = ld_ag(shx + shx_i);
      SS_TRACE(10);
      __syncthreads();
      SS_TRACE(12);
      if (tid < 16 * kTBv) {
        const int c = tid >> 2, r = tid & 3;
        uint32_t sb = 0;
        if (r < nt) {
          constexpr int KM = kMaxQv / kTBv;
          // Every LDS read is issued before any is used (two dependent rounds, no branch per term).
          int uq[KM];
          float wq[KM], pv[KM], ov[KM];
#pragma unroll
          for (int k = 0; k < KM; ++k) {
            const int q = r * K + (k < K ? k : 0);
            uq[k] = s.use_u[q];
            wq[k] = s.wts[q];
          }
#pragma unroll
          for (int k = 0; k < KM; ++k) pv[k] = partl[((size_t)(uq[k] >= 0 ? uq[k] : 0) * 16 + c) * kTBv + r];
#pragma unroll
          for (int k = 0; k < KM; ++k) {
            const float prod = pv[k] * wq[k];
            ov[k] = k < K && uq[k] >= 0 ? prod : 0.f;
          }
          float acc = 0.f;
#pragma unroll
          for (int k = 0; k < KM; ++k)
            if (k < K) acc = k == 0 ? ov[k] : acc + ov[k];
          if (lp.routed_out) gp(lp.routed_out)[(size_t)r * H + 16 * bid + c] = acc;
          SS_TRACE(16 + 3);
          for (int it = 0; (uint32_t)(shx_w >> 32) != tag; ++it) {
            if (dead()) break;
            if (it >= kChainSpin) {
              ss_raise(a.err, SS_ERR_TIMEOUT);
              break;
            }
            shx_w = ld_ag(shx + shx_i);
          }
          SS_TRACE(15);
          const float sh2 = ss_bf16_to_f32((uint32_t)shx_w & 0xFFFFu);
          const uint32_t yb = ss_f32_to_bf16(ss_round_bf16(acc) + sh2);
          gp(lp.y)[(size_t)r * H + 16 * bid + c] = (uint16_t)yb;
          sb = ss_f32_to_bf16(ss_bf16_to_f32(xres) + ss_bf16_to_f32(yb));
          if (lp.stream_out) gp(lp.stream_out)[(size_t)r * H + 16 * bid + c] = (uint16_t)sb;
        }
        // the stream word of rows (c, c + 1) of token r: the partner row sits 4 lanes up
        const uint32_t sb_hi = (uint32_t)__shfl_xor((int)sb, 4);
        if (r < nt && (c & 1) == 0 && l + 1 < NL)
          st_ag(sw_all + (size_t)(l & 1) * kTBv * (H / 2) + (size_t)r * (H / 2) + 8 * bid + (c >> 1),
                ((uint64_t)tag << 32) | (uint64_t)(sb | (sb_hi << 16)));
      }
      SS_TRACE(6);
      if (tr && tid == 0) {
        __builtin_amdgcn_s_waitcnt(0);
        trs[16] = __builtin_amdgcn_s_memrealtime();
      }
    }

    // ---------------------------------------------------------- into the next layer
    // The next layer's first reads (its router or shared rows, map entries and routing bias) go out now and land
    // while the workgroup waits for this layer's stream; its slot pointers follow its dense rows.
    if (l + 1 < NL) {
      if (w == 3) __builtin_amdgcn_s_waitcnt(0);  // the entry has landed in LDS
      __syncthreads();
      const ssmoe_chain_layer ln = layer_from_lds(s_next);
      if (j_first < J) load_job(ln, j_first);
      load_map(ln);
      if (w < nt) load_bias(ln);
      lp = ln;
    }
    __syncthreads();
    SS_TRACE(11);
#undef SS_TRACE
  }

  // ------------------------------------------------------------ exit: the last workgroup resets the counters
  __syncthreads();
  if (a.trace && tid < 64) {
    // Rows: last layer at bid, the layer before at 512 + bid; their extra stamps at 256 + bid and 768 + bid.
    const int q = lane >> 5, k = lane & 31;
    const size_t row = (size_t)(q ? 0 : 512) + (k < 16 ? 0 : 256) + bid;
    if (NL - 2 + q >= 0) a.trace[row * 16 + (k & 15)] = s_tr[q][k];
  }
  if (tid == 0) {
    const int sh = bid % kCShards;
    const int in_shard = (G - sh + kCShards - 1) / kCShards;
    const int t1 = __hip_atomic_fetch_add(cshard(ctr, CTR_EXIT, sh), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t1 == in_shard - 1) {
      const int t2 = __hip_atomic_fetch_add(cshard(ctr, CTR_TOP, 0), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (t2 == (G < kCShards ? G : kCShards) - 1) {
        for (int c = 0; c < CTR_COUNT; ++c)
          if (c != CTR_EPOCH)
            for (int q = 0; q < kCShards; ++q)
              __hip_atomic_store(cshard(ctr, c, q), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(cshard(ctr, CTR_EPOCH, 0), NL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <int NJG, int NJD, bool SHQ4>
static hipError_t launch_chain_nj(const ChainArgs& a, hipStream_t st) {
  const SsRecord rec = ss_record_layout(a.H, a.I);
  auto kern = chain_kernel<NJG, NJD, SHQ4>;
  const CDLayout dly = cdlayout(a.T, a.H, a.I, a.Is, a.K, a.E);
  // Every workgroup waits on the others: one workgroup per CU, launched only if a workgroup with the largest dynamic
  // LDS the kernel takes fits on a CU (checked once per device).
  KernelCfg cfg;
  hipError_t e = kernel_cfg(reinterpret_cast<const void*>(kern), 256, kLdsBudget, &cfg);
  if (e != hipSuccess) return e;
  if (cfg.per_cu < 1) return hipErrorCooperativeLaunchTooLarge;
  if (dly.P < 1 || dly.total > kLdsBudget || cfg.lds_static + dly.total > 160 * 1024) return hipErrorInvalidConfiguration;
  const int grid = cfg.cus;
  if (grid <= a.H / 16 || a.E + a.Is < 4 * grid) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), dly.total, st, a, rec);
  return hipGetLastError();
}

bool chain_shape_supported(int H, int I) { return (H == 2048 && I == 512) || (H == 2560 && I == 640); }

const char* chain_shapes_text() {
  return "the chain kernel is built for H 2048 with I 512 (BASELINE) and H 2560 with I 640 (the reference model)";
}

hipError_t launch_chain(const ChainArgs& a, hipStream_t st) {
  // One instantiated shape: H 2048 x I 512, the BASELINE layer (the layer loop is sized to the register file for it);
  // other shapes run one ssmoe_moe_verify_layer_chain launch per layer.
  const int njg = a.H / 128, njd = a.I / 128;
  const bool q4 = a.l0.sh_gate_s != nullptr;  // every layer alike (checked by the entry point)
  if (njg == 16 && njd == 4) return q4 ? launch_chain_nj<16, 4, true>(a, st) : launch_chain_nj<16, 4, false>(a, st);
  if (njg == 20 && njd == 5) return q4 ? launch_chain_nj<20, 5, true>(a, st) : launch_chain_nj<20, 5, false>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace ss
