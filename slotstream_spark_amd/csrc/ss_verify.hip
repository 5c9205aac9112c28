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
#include <type_traits>

#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

constexpr int kTBv = 4;          // tokens per launch
constexpr int kMaxEv = 512;      // experts per layer (LDS tables)
constexpr int kMaxQv = 64;       // kTBv * K, K <= 16
constexpr int kSpinMax = 1 << 22;
constexpr int kXZero = 98;       // uint4 zeros an inactive A lane reads in phase C: offsets 0 .. 48 * 2 (fp32 x)
constexpr int SS_ERR_TIMEOUT = 16;
constexpr size_t kLdsBudget = 160 * 1024 - 16 * 1024;  // dynamic LDS left after the static part (< 16 KB)

// Counters are sharded: workgroup b adds to shard b % kShards of a counter, and a waiter sums the shards. Each
// shard has a 128-byte line of its own; many workgroups adding to one address serialise at the memory-side atomic
// unit (tens of ns each), which with 256 workgroups delays the moment the count is complete by microseconds.
constexpr int kShards = 16;
constexpr int kShardStride = 32;  // ints
// CTR_EPOCH counts launches on this workspace: it is never reset, and the last workgroup of a launch adds one.
enum { CTR_SHARED = 0, CTR_ITEMS = 1, CTR_EXIT = 2, CTR_TOP = 3, CTR_EPOCH = 4, CTR_COUNT = 5 };
SS_DEV int* shard(int* ctr, int c, int s) { return ctr + (c * kShards + s) * kShardStride; }

typedef __attribute__((address_space(3))) void lds_void_t;
struct VLayout {
  size_t ctr, logits, gsh, ush, sgl, hfrag, hsum8, total;
};

static __host__ __device__ inline size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

static __host__ __device__ inline VLayout vlayout(int T, int H, int I, int Is, int K, int E) {
  VLayout l;
  size_t o = 0;
  l.ctr = o;
  o = al256(o + (size_t)CTR_COUNT * kShards * kShardStride * 4);
  l.logits = o;  // [T][E] words: tag << 32 | bf16 logit
  o = al256(o + (size_t)T * E * 8);
  l.gsh = o;
  o = al256(o + (size_t)T * Is * 2);
  l.ush = o;
  o = al256(o + (size_t)T * Is * 2);
  l.sgl = o;
  o = al256(o + (size_t)T * 2);
  l.hfrag = o;
  o = al256(o + (size_t)T * K * I * 4);
  l.hsum8 = o;
  o = al256(o + (size_t)T * K * (I / 8) * 4);
  l.total = o;
  return l;
}

size_t verify_scratch_bytes(int T, int H, int I, int Is, int K, int E) {
  return vlayout(T, H, I, Is, K, E).total;
}

// Dynamic LDS layout (bytes): per-expert partial dots, staged h fragments, then one region that holds the x
// fragments while phases A-C run and the down-weight prefetch slots afterwards (a workgroup issues its prefetch only
// once its own gate/up items are done, the last use of x).
// Prefetch slot (one expert, the workgroup's 16 down rows): [NJD][64 lanes] 16-byte weight words, then the scale
// dwords [16 rows][NJD] and the bias dwords [16 rows][NJD] (dword j of a row holds groups 2j, 2j + 1).
struct DLayout {
  size_t xfrag, hfrag, pref, part, total;
  int P;           // experts whose down weights are prefetched per batch
  int stage_h;     // 1: the h fragments are staged in LDS for the down phase; 0: read from global memory
  size_t slot;     // bytes per prefetch slot
};

static __host__ __device__ inline size_t dslot_bytes(int I) { return (size_t)(I / 128) * (1024 + 2 * 16 * 4); }

static __host__ __device__ inline DLayout dlayout(int T, int H, int I, int K, int E, int x_f32, int verify) {
  (void)verify;
  DLayout d;
  const int nq = T * K;
  const int nu_max = nq < E ? nq : E;
  const size_t xf = (size_t)(H / 128) * 4 * 4 * kTBv * (x_f32 ? 2 : 1) * 16;
  d.slot = dslot_bytes(I);
  size_t o = 0;
  d.part = o;
  o += (size_t)nu_max * 16 * kTBv * 4;
  d.hfrag = o;
  const size_t hf = (size_t)nq * I * 4;
  const size_t tail = xf > d.slot ? xf : d.slot;  // the shared region holds x, or at least one slot
  d.stage_h = o + hf + tail <= kLdsBudget;
  if (d.stage_h) o += hf;
  d.pref = d.xfrag = o;
  const long room = (long)kLdsBudget - (long)o;
  int P = room > 0 ? (int)(room / (long)d.slot) : 0;
  if (P > nu_max) P = nu_max;
  d.P = P;
  const size_t pb = (size_t)P * d.slot;
  d.total = o + (pb > xf ? pb : xf);
  return d;
}

// Cross-workgroup hand-off. The data that crosses workgroups (router logits, shared-expert rows, h fragments and
// sums, counters) is written and read only with monotonic agent-scope accesses: on gfx950 these carry the sc1
// scope bit, so they are coherent across the eight XCDs' L2 caches by themselves, and no whole-cache write-back
// (buffer_wbl2) or invalidate (buffer_inv), which agent-scope release and acquire fences would emit, is needed.
// Producer: every wave waits for its own stores to be acknowledged (s_waitcnt), the workgroup barrier orders them,
// then one thread adds to the counter. Consumer: one thread polls the counter, then the workgroup barrier; the data
// loads are issued after the poll has seen the count.
SS_DEV void stores_done() { __builtin_amdgcn_s_waitcnt(0); }

SS_DEV void signal_add(int* ctr, int c, int v) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __hip_atomic_fetch_add(shard(ctr, c, blockIdx.x % kShards), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every lane of one wave: lanes 0 .. kShards-1 read one shard each, the butterfly sums them.
SS_DEV void wait_ge(int* ctr, int c, int target, int* err) {
  const int lane = threadIdx.x & 63;
  int* p = shard(ctr, c, lane < kShards ? lane : 0);
  for (int it = 0;; ++it) {
    const int v = lane < kShards ? __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    const int total = (int)ss_butterfly((uint32_t)v, [](uint32_t x, uint32_t y) { return x + y; });
    if (total >= target) break;
    if (it >= kSpinMax) {
      if (lane == 0) ss_raise(err, SS_ERR_TIMEOUT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <class T>
SS_DEV void st_ag(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
SS_DEV T ld_ag(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
SS_DEV void st_ag16(void* p, uint4 v) {
  uint64_t* q = static_cast<uint64_t*>(p);
  st_ag(q, ((uint64_t)v.y << 32) | v.x);
  st_ag(q + 1, ((uint64_t)v.w << 32) | v.z);
}
SS_DEV uint4 ld_ag16(const void* p) {
  const uint64_t* q = static_cast<const uint64_t*>(p);
  const uint64_t a = ld_ag(q), b = ld_ag(q + 1);
  return make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
}

// Direct-to-LDS loads: lane l's `size` bytes land at lds_wave_base + size * l (lds_wave_base is wave-uniform).
SS_DEV void dma16(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_wave_base, 16, 0, 0);
}
// The same with the sc1 (agent) scope bit, for data written by other workgroups in this launch.
SS_DEV void dma16_ag(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_wave_base, 16, 0, 16);
}
SS_DEV void dma4(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_wave_base, 4, 0, 0);
}

struct VSmem {
  int map[kMaxEv];
  const uint8_t* base_e[kMaxEv];  // record of every expert of the layer (verify mode)
  const uint8_t* base[kMaxQv];    // per unique expert
  uint32_t umask[kMaxQv][kTBv];
  int use_u[kMaxQv];
  int ids[kMaxQv];
  float wts[kMaxQv];
  float gx[64][kTBv];             // x group sums (H <= 4096)
  union alignas(16) {
    float hsum[kMaxQv][16];       // h group sums per use (I <= 1024), phase D
    uint64_t cand[kTBv][64];      // router-tail candidates of each token, phase B
  };
  float shv[16][kTBv];
  float rnorm[kTBv];              // 1 / rms of each token (chained layers)
  float xch[4][16 * kTBv];        // per-wave exchange of one item's 16 columns x 4 tokens
  alignas(16) int ekey[64];       // unique_setup keys
  alignas(16) uint4 zero_h[4];    // zeros: the h operand of A rows that do not use the expert (phase D)
  int nt, nu;
};

static_assert(kXZero * sizeof(uint4) <= sizeof(float) * kMaxQv * 16, "phase C zeros fit in hsum");

SS_DEV float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
SS_DEV float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
SS_DEV float pick_half(uint32_t pair, int hi) { return hi ? bf_hi(pair) : bf_lo(pair); }

// bf16 pair (element d, element d+4) of 8 consecutive bf16 held as 4 words (e0e1, e2e3, e4e5, e6e7).
SS_DEV uint4 perm_pairs(uint4 v) {
  uint4 f;
  f.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
  f.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
  f.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
  f.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  return f;
}

SS_DEV ss_u32x4 as_v(uint4 v) {
  ss_u32x4 r;
  r.x = v.x;
  r.y = v.y;
  r.z = v.z;
  r.w = v.w;
  return r;
}

// Unique experts of the block in first-occurrence order from s.ids. Wave 0 only; caller syncs.
// Each lane publishes a key (its expert, or a negative value no other lane has when the entry is unusable) and
// finds the first lane with the same key by broadcast LDS reads.
SS_DEV void unique_setup(const VerifyArgs& a, VSmem& s, bool tables_in_lds) {
  const int lane = threadIdx.x;
  const int nq = s.nt * a.K;
  int e = -1, slot = -1;
  bool valid = false;
  if (lane < nq) {
    e = s.ids[lane];
    if (e >= 0 && e < a.E) {
      if (tables_in_lds) {
        slot = s.map[e];
      } else {
        const int64_t mi = a.map_base + e;
        if (mi >= 0 && mi < a.map_len) slot = a.map[mi];
      }
      valid = slot >= 0 && (int64_t)slot < a.n_slots;
      if (!valid) ss_raise(a.err, SS_ERR_SLOT);
    } else {
      ss_raise(a.err, SS_ERR_EXPERT_ID);
    }
  }
  const int key = valid ? e : -1 - lane;
  s.ekey[lane] = key;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int j0 = 64;
#pragma unroll 4
  for (int j = 0; j < nq; j += 4) {
    const int4 k4 = *reinterpret_cast<const int4*>(&s.ekey[j]);
    if (j0 == 64 && k4.x == key) j0 = j;
    if (j0 == 64 && k4.y == key) j0 = j + 1;
    if (j0 == 64 && k4.z == key) j0 = j + 2;
    if (j0 == 64 && k4.w == key) j0 = j + 3;
  }
  const bool first = valid && j0 == lane;
  const uint64_t mask = __ballot(first);
  const int uidx = valid ? __popcll(mask & ((1ull << j0) - 1ull)) : -1;
  if (first) s.base[uidx] = tables_in_lds ? s.base_e[e] : reinterpret_cast<const uint8_t*>(a.slot_ptr[slot]);
  if (lane < nq) {
    s.use_u[lane] = uidx;
    if (valid) atomicOr(&s.umask[uidx][lane / a.K], 1u << (lane % a.K));
  }
  if (lane == 0) s.nu = __popcll(mask);
}

// Router tail of token t in one wave (the operations and order of router_topk_kernel): lane l holds the entries
// e = l + 64 i. The top K in (probability desc, index asc) order come from a threshold and a rank count (below);
// the K dependent rounds of router_topk_kernel remain for the rows that path does not take. Both give the same
// ids, and the weights are summed in rank order either way.
SS_DEV void router_tail_wave(const VerifyArgs& a, const uint64_t* logits, uint32_t tag, int t, VSmem& s,
                             const float (&bias_r)[kMaxEv / 64]) {
  const int lane = threadIdx.x & 63;
  const int E = a.E, K = a.K;
  constexpr int NV = kMaxEv / 64;
  const uint64_t* lg = logits + (size_t)t * E;
  // Every logit word carries the launch's tag: the wave polls the words themselves until all of its token's E
  // logits are this launch's (bounded like wait_ge), so no counter round trip precedes the data.
  uint64_t wv[NV];
  for (int it = 0;; ++it) {
    bool fresh = true;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + 64 * i;
      wv[i] = ld_ag(lg + (e < E ? e : 0));
      fresh = fresh && (e >= E || (uint32_t)(wv[i] >> 32) == tag);
    }
    if (__all(fresh)) break;
    if (it >= kSpinMax) {
      if (lane == 0) ss_raise(a.err, SS_ERR_TIMEOUT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (a.trace && threadIdx.x == 0) a.trace[(size_t)blockIdx.x * 16 + 5] = __builtin_amdgcn_s_memrealtime();  // logits in
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = ss_bf16_to_f32((uint16_t)wv[i]);
  if (a.bias) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = v[i] + bias_r[i];
  }
  // Selects instead of branches; an absent entry adds +0 to a non-negative sum, which changes no bit.
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
  // kp = key + 1 for a present, untaken entry (NaN probabilities have key 0, so kp 1), 0 once taken or absent.
  uint32_t kp[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    v[i] = v[i] / z;
    kp[i] = lane + 64 * i < E ? ss_key(v[i]) + 1u : 0u;
  }
  // tau: the largest threshold with zero low 16 bits that at least K lane maxima reach. Those K entries are >= tau,
  // so every entry of the top K is too. The entries >= tau (a few more than K on router rows) go to LDS in index
  // order as (kp << 32 | 0xFFFF - e), a key whose order is the selection order; each candidate's rank is the number
  // of larger keys. With more than 64 candidates, or no such tau (NaN probabilities have kp 1), the rounds run.
  {
    uint32_t lmax = kp[0];
#pragma unroll
    for (int i = 1; i < NV; ++i) lmax = kp[i] > lmax ? kp[i] : lmax;
    uint32_t tau = 0;
#pragma unroll
    for (int b = 31; b >= 16; --b) {
      const uint32_t c = tau | (1u << b);
      tau = __popcll(__ballot(lmax >= c)) >= K ? c : tau;
    }
    uint64_t bal[NV];
    int nc = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      bal[i] = __ballot(kp[i] >= tau);
      nc += __popcll(bal[i]);
    }
    if (tau != 0 && nc <= 64) {
      uint64_t* cs = s.cand[t];
      int off = 0;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const uint64_t b = bal[i];
        const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        if ((b >> lane) & 1ull) cs[off + below] = ((uint64_t)kp[i] << 32) | (uint64_t)(0xFFFFu - (uint32_t)(lane + 64 * i));
        off += __popcll(b);
      }
      const int ncp = (nc + 7) & ~7;  // zero keys pad the list to whole groups of 8; they rank below every key
      if (lane >= nc && lane < ncp) cs[lane] = 0ull;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint64_t my = lane < nc ? cs[lane] : 0ull;
      int rank = 0;
#pragma unroll 1
      for (int j = 0; j < ncp; j += 8) {
        const ulonglong2* q = reinterpret_cast<const ulonglong2*>(cs + j);
        const ulonglong2 q0 = q[0], q1 = q[1], q2 = q[2], q3 = q[3];
        rank += (q0.x > my) + (q0.y > my) + (q1.x > my) + (q1.y > my) + (q2.x > my) + (q2.y > my) + (q3.x > my) +
                (q3.y > my);
      }
      if (lane < nc && rank < K) {
        s.ids[t * K + rank] = (int)(0xFFFFu - (uint32_t)my);
        s.wts[t * K + rank] = ss_unkey((uint32_t)(my >> 32) - 1u);  // the probability itself (kp = key + 1)
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const float pv = lane < K ? s.wts[t * K + lane] : 0.f;
      float sum = 0.f;
#pragma unroll 1
      for (int r = 0; r < K; ++r) sum = sum + ss_readlane_f(pv, r);  // rank-order sum of the top-k probabilities
      if (lane < K) s.wts[t * K + lane] = pv / sum;
      return;
    }
  }
  float mine = 0.f, sum = 0.f;
  int my_id = 0;
#pragma unroll 1
  for (int r = 0; r < K; ++r) {
    uint32_t lm = kp[0];
#pragma unroll
    for (int i = 1; i < NV; ++i) lm = kp[i] > lm ? kp[i] : lm;
    const uint32_t mx = ss_wave_max_u32(lm);
    // The lowest index e = lane + 64 i holding mx: per lane the lowest such i, then across lanes the lowest e.
    int li = NV;
#pragma unroll
    for (int i = NV - 1; i >= 0; --i) li = kp[i] == mx ? i : li;
    const uint32_t code = (uint32_t)(li * 64 + lane);  // = e where this lane holds mx, >= 64 NV otherwise
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
    const bool own = lane == wl;
#pragma unroll
    for (int i = 0; i < NV; ++i) kp[i] = own && i == wi ? 0u : kp[i];
    sum = sum + pv;  // rank-order sum of the top-k probabilities
    mine = lane == r ? pv : mine;
    my_id = lane == r ? bi : my_id;
  }
  if (lane < K) {
    s.ids[t * K + lane] = my_id;
    s.wts[t * K + lane] = mine / sum;
  }
}

// x A-fragment entry f = (((j * 4 + i) * 4 + g) * kTBv + t) holds elements kb .. kb + 7 of token t, kb = 128 j +
// 32 g + 8 i, as the bf16 pairs (e0, e4) (e1, e5) (e2, e6) (e3, e7) (perm_pairs); with fp32 x the entry is two uint4,
// the bf16 high parts and the bf16 residuals. Element e of an entry is word e & 3, half e >> 2.
SS_DEV int xfrag_index(int kb, int t) {
  return ((((kb >> 7) * 4 + ((kb >> 3) & 3)) * 4 + ((kb >> 5) & 3)) * kTBv) + t;
}

// Stage the x fragments (into xfl) and the 64-element group sums of x (into s.gx, sequential in element order).
// Every global load of a thread is issued before its first use; tokens t >= nt read token 0 and are zeroed.
// With a.norm_in (bf16 x only) every element is first replaced by bf16((x * r_t) * norm_w): wave w computes r of
// token w in the ssmoe_residual_rmsnorm order (lane l: elements 512 j + 8 l .. + 7 by fma from 0, then the
// butterfly), so every workgroup stages the same values the separate norm kernel would write.
template <int NJG, bool XF32>
SS_DEV void stage_x(const VerifyArgs& a, uint4* xfl, float (*gx)[kTBv], float* rnorm, int nt) {
  const int tid = threadIdx.x;
  const int H = a.H;
  constexpr int NJX = NJG / 4;
  const bool norm = !XF32 && a.norm_in;
  uint4 nv[NJX];
  if (norm) {
    const int tn = (tid >> 6) < nt ? (tid >> 6) : 0;
#pragma unroll
    for (int jj = 0; jj < NJX; ++jj)
      nv[jj] = ldg16(static_cast<const uint16_t*>(a.x) + (size_t)tn * H + 8 * (64 * jj + (tid & 63)));
  }
  constexpr int NF = NJG * 16 * kTBv;  // (j, i, g, t)
  constexpr int FPT = NF / 256;
  static_assert(NF % 256 == 0, "whole fragment entries per thread");
  uint4 fv[FPT][XF32 ? 2 : 1];
#pragma unroll
  for (int k = 0; k < FPT; ++k) {
    const int f = tid + 256 * k;
    const int t = f & 3, gg = (f >> 2) & 3, i = (f >> 4) & 3, j = f >> 6;
    const int tt = t < nt ? t : 0;
    const int kb = 128 * j + 32 * gg + 8 * i;
    if (XF32) {
      const float* xp = static_cast<const float*>(a.x) + (size_t)tt * H + kb;
      fv[k][0] = ldg16(xp);
      fv[k][XF32 ? 1 : 0] = ldg16(xp + 4);
    } else {
      fv[k][0] = ldg16(static_cast<const uint16_t*>(a.x) + (size_t)tt * H + kb);
    }
  }
  // Group sums: thread q < (H / 64) * kTBv sums group q >> 2 of token q & 3.
  constexpr int GV = XF32 ? 16 : 8;
  uint4 gv[GV];
  const int q = tid < (H >> 6) * kTBv ? tid : 0;
  const int gt = (q & 3) < nt ? (q & 3) : 0;
  const int Gi = q >> 2;
#pragma unroll
  for (int k = 0; k < GV; ++k) {
    if (norm) break;  // the norm path sums the staged values instead
    if (XF32)
      gv[k] = ldg16(static_cast<const float*>(a.x) + (size_t)gt * H + 64 * Gi + 4 * k);
    else
      gv[k] = ldg16(static_cast<const uint16_t*>(a.x) + (size_t)gt * H + 64 * Gi + 8 * k);
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
    if ((tid & 63) == 0) rnorm[tid >> 6] = 1.f / sqrtf(ssum / (float)H + a.norm_eps);
    __syncthreads();
    // bf16((v * r) * w) of the 8 elements of a 16-byte word (w = norm_w at element k0; without norm_w, bf16(v * r))
    auto scale8 = [&](uint4 v, float r, int k0) {
      const uint32_t x4[4] = {v.x, v.y, v.z, v.w};
      uint32_t o[4];
      if (a.norm_w) {
        const uint4 wv = ldg16(a.norm_w + k0);
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
      fv[k][0] = scale8(fv[k][0], rnorm[tt], 128 * j + 32 * gg + 8 * i);
    }
  }
#pragma unroll
  for (int k = 0; k < FPT; ++k) {
    const int f = tid + 256 * k;
    const bool live = (f & 3) < nt;
    if (XF32) {
      const uint4 v0 = fv[k][0], v1 = fv[k][XF32 ? 1 : 0];
      const float e0[4] = {__uint_as_float(v0.x), __uint_as_float(v0.y), __uint_as_float(v0.z), __uint_as_float(v0.w)};
      const float e1[4] = {__uint_as_float(v1.x), __uint_as_float(v1.y), __uint_as_float(v1.z), __uint_as_float(v1.w)};
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t b0 = ss_f32_to_bf16(e0[d]), b1 = ss_f32_to_bf16(e1[d]);
        hw[d] = b0 | (b1 << 16);
        lw[d] = ss_f32_to_bf16(e0[d] - ss_bf16_to_f32(b0)) | (ss_f32_to_bf16(e1[d] - ss_bf16_to_f32(b1)) << 16);
      }
      xfl[2 * f] = make_uint4(live ? hw[0] : 0u, live ? hw[1] : 0u, live ? hw[2] : 0u, live ? hw[3] : 0u);
      xfl[2 * f + 1] = make_uint4(live ? lw[0] : 0u, live ? lw[1] : 0u, live ? lw[2] : 0u, live ? lw[3] : 0u);
    } else {
      const uint4 pv = perm_pairs(fv[k][0]);
      xfl[f] = make_uint4(live ? pv.x : 0u, live ? pv.y : 0u, live ? pv.z : 0u, live ? pv.w : 0u);
    }
  }
  if (norm) {
    // The group sums of the normalised values, read back in element order from the staged fragments (entry
    // elements e0..e7 are the halves lo(x) lo(y) lo(z) lo(w) hi(x) hi(y) hi(z) hi(w)).
    __syncthreads();
    if (tid < (H >> 6) * kTBv) {
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint4 v = xfl[xfrag_index(64 * Gi + 8 * k, gt)];
        sum = sum + bf_lo(v.x);
        sum = sum + bf_lo(v.y);
        sum = sum + bf_lo(v.z);
        sum = sum + bf_lo(v.w);
        sum = sum + bf_hi(v.x);
        sum = sum + bf_hi(v.y);
        sum = sum + bf_hi(v.z);
        sum = sum + bf_hi(v.w);
      }
      gx[Gi][q & 3] = (q & 3) < nt ? sum : 0.f;
    }
    return;
  }
  if (tid < (H >> 6) * kTBv) {
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < GV; ++k) {
      const uint4 v = gv[k];
      if (XF32) {
        sum = sum + __uint_as_float(v.x);
        sum = sum + __uint_as_float(v.y);
        sum = sum + __uint_as_float(v.z);
        sum = sum + __uint_as_float(v.w);
      } else {
        sum = sum + bf_lo(v.x);
        sum = sum + bf_hi(v.x);
        sum = sum + bf_lo(v.y);
        sum = sum + bf_hi(v.y);
        sum = sum + bf_lo(v.z);
        sum = sum + bf_hi(v.z);
        sum = sum + bf_lo(v.w);
        sum = sum + bf_hi(v.w);
      }
    }
    gx[Gi][q & 3] = (q & 3) < nt ? sum : 0.f;
  }
}

// One dense bf16 row (16-byte words wv[jj] = elements 512 jj + 8 lane .. +7, already in registers) against the
// staged bf16 x fragments, in the dense_rows_kernel order: per lane, fused multiply-adds over its elements in order,
// then the wave butterfly.
template <int NJX>
SS_DEV void dense_dot(const uint4 (&wv)[NJX], const uint4* xfl, int nt, float out[kTBv]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int t = 0; t < kTBv; ++t) {
    if (t >= nt) break;
    float ac = 0.f;
#pragma unroll
    for (int jj = 0; jj < NJX; ++jj) {
      const uint4 xv = xfl[xfrag_index(512 * jj + 8 * lane, t)];
      const uint32_t ww[4] = {wv[jj].x, wv[jj].y, wv[jj].z, wv[jj].w};
      const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float wf = (e & 1) ? bf_hi(ww[e >> 1]) : bf_lo(ww[e >> 1]);
        const float xf = (e >> 2) ? bf_hi(xx[e & 3]) : bf_lo(xx[e & 3]);
        ac = __builtin_fmaf(xf, wf, ac);
      }
    }
    out[t] = ss_wave_sum(ac);
  }
}

// The shared-expert gate / up projections of this lane's 8 elements for every token (tokens >= nt read token 0).
struct SharedIn {
  uint4 g[kTBv], u[kTBv];
};

SS_DEV SharedIn shared_load(const VerifyArgs& a, const uint16_t* gsh, const uint16_t* ush, int nt) {
  const int lane = threadIdx.x & 63;
  const int li = 8 * lane < a.Is ? lane : 0;
  SharedIn in;
#pragma unroll
  for (int t = 0; t < kTBv; ++t) {
    const int tt = t < nt ? t : 0;
    in.g[t] = ld_ag16(gsh + (size_t)tt * a.Is + 8 * li);
    in.u[t] = ld_ag16(ush + (size_t)tt * a.Is + 8 * li);
  }
  return in;
}

// hs = bf16(bf16(silu(g)) * u) of the shared expert (the F.silu and product of the reference, in bf16), split over
// the workgroup's four waves: wave w computes elements 8 l + 2 w and 8 l + 2 w + 1 of lane l's eight for every
// token and stores them to hsl [nt][Is] (LDS).
SS_DEV void shared_hs_part(const VerifyArgs& a, const SharedIn& in, int w, int nt, float* hsl) {
  const int lane = threadIdx.x & 63;
  if (8 * lane >= a.Is) return;
#pragma unroll
  for (int t = 0; t < kTBv; ++t) {
    if (t >= nt) break;
    const uint32_t gw4[4] = {in.g[t].x, in.g[t].y, in.g[t].z, in.g[t].w};
    const uint32_t uw4[4] = {in.u[t].x, in.u[t].y, in.u[t].z, in.u[t].w};
    const uint32_t gw = w == 0 ? gw4[0] : w == 1 ? gw4[1] : w == 2 ? gw4[2] : gw4[3];
    const uint32_t uw = w == 0 ? uw4[0] : w == 1 ? uw4[1] : w == 2 ? uw4[2] : uw4[3];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float gv = h ? bf_hi(gw) : bf_lo(gw);
      const float uv = h ? bf_hi(uw) : bf_lo(uw);
      const float sv = ss_round_bf16(gv / (1.f + ss_expf(-gv)));
      hsl[t * a.Is + 8 * lane + 2 * w + h] = ss_round_bf16(sv * uv);
    }
  }
}

// Shared-expert down rows of one wave, in the dense_rows order: the dot of hs (hsl) with the bf16 down rows;
// out[rr][t] receives the fp32 sums (every lane). sh_w holds each row's 8 elements of this lane (Is <= 512).
template <int NR>
SS_DEV void shared_down_rows(const VerifyArgs& a, const float* hsl, const uint4 (&sh_w)[NR], int nt,
                             float (&out)[NR][kTBv]) {
  const int lane = threadIdx.x & 63;
  float sacc[NR][kTBv];
#pragma unroll
  for (int rr = 0; rr < NR; ++rr)
#pragma unroll
    for (int t = 0; t < kTBv; ++t) sacc[rr][t] = 0.f;
  if (8 * lane < a.Is) {
#pragma unroll
    for (int t = 0; t < kTBv; ++t) {
      if (t >= nt) break;
      float hsv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) hsv[e] = hsl[t * a.Is + 8 * lane + e];
#pragma unroll
      for (int rr = 0; rr < NR; ++rr) {
        const uint32_t ww[4] = {sh_w[rr].x, sh_w[rr].y, sh_w[rr].z, sh_w[rr].w};
        float ac = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ac = __builtin_fmaf(hsv[e], (e & 1) ? bf_hi(ww[e >> 1]) : bf_lo(ww[e >> 1]), ac);
#pragma unroll
        for (int q = 0; q < kTBv; ++q)
          if (q == t) sacc[rr][q] = ac;
      }
    }
  }
#pragma unroll
  for (int rr = 0; rr < NR; ++rr)
#pragma unroll
    for (int t = 0; t < kTBv; ++t) out[rr][t] = t < nt ? ss_wave_sum(sacc[rr][t]) : 0.f;
}

template <int NJG, int NJD, bool XF32>
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
  auto load_job = [&](int j) {
    const uint16_t* w0 = j < E ? a.router_w + (size_t)j * H : a.sh_gate + (size_t)(j - E) * H;
#pragma unroll
    for (int jj = 0; jj < NJX; ++jj) r0[jj] = ldg16(w0 + 8 * (64 * jj + lane));
    if (j >= E) {
      const uint16_t* w1 = a.sh_up + (size_t)(j - E) * H;
#pragma unroll
      for (int jj = 0; jj < NJX; ++jj) r1[jj] = ldg16(w1 + 8 * (64 * jj + lane));
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
  uint4 shw[4];
  SharedIn shin;
  if (verify && has_tile) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      shw[rr] = ldg16(a.sh_down + (size_t)(16 * bid + 4 * w + rr) * a.Is + 8 * (8 * lane < a.Is ? lane : 0));
  }
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
      shared_hs_part(a, shin, w, nt, hsl);
      __syncthreads();
      float o[4][kTBv];
      shared_down_rows<4>(a, hsl, shw, nt, o);
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

template <int NJG, int NJD, bool XF32>
static hipError_t launch_nj(const VerifyArgs& a, hipStream_t st) {
  const SsRecord rec = ss_record_layout(a.H, a.I);
  auto kern = verify_kernel<NJG, NJD, XF32>;
  const DLayout dly = dlayout(a.T, a.H, a.I, a.K, a.E, XF32 ? 1 : 0, a.mode == 0 ? 1 : 0);
  static size_t lds_set = 0, lds_static = 0;
  static int grid = 0;
  if (lds_set == 0) {
    hipFuncAttributes attr;
    hipError_t e = hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kern));
    if (e != hipSuccess) return e;
    lds_static = attr.sharedSizeBytes;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)kLdsBudget);
    if (e != hipSuccess) return e;
    lds_set = kLdsBudget;
  }
  // A workgroup may hold at most 160 KB of LDS on gfx950; refuse any shape whose layout would exceed it.
  if (dly.P < 1 || dly.total > kLdsBudget || lds_static + dly.total > 160 * 1024) return hipErrorInvalidConfiguration;
  // The shared expert's hs [T][Is] fp32 reuses the prefetch region at the end of phase D.
  if (a.mode == 0 && (size_t)a.T * a.Is * 4 > dly.total - dly.pref) return hipErrorInvalidConfiguration;
  if (grid == 0) {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    grid = cus;
  }
  if (grid < a.H / 16) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), dly.total, st, a, rec);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void zero16_kernel(uint4* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

hipError_t launch_zero16(void* p, size_t bytes, hipStream_t st) {
  const size_t n = bytes / 16;
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(zero16_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, st,
                     static_cast<uint4*>(p), n);
  return hipGetLastError();
}

template <int NJG, int NJD>
static hipError_t launch_x(const VerifyArgs& a, hipStream_t st) {
  return a.x_f32 ? launch_nj<NJG, NJD, true>(a, st) : launch_nj<NJG, NJD, false>(a, st);
}

hipError_t launch_verify(const VerifyArgs& a, hipStream_t st) {
  // Shapes with instantiated kernels: H in {1024, 2048, 2560, 4096} x I in {128, 256, 512, 640, 1024}.
  const int njg = a.H / 128, njd = a.I / 128;
#define SS_CASE(G_, D_) \
  if (njg == G_ && njd == D_) return launch_x<G_, D_>(a, st);
#define SS_ROW(G_) SS_CASE(G_, 1) SS_CASE(G_, 2) SS_CASE(G_, 4) SS_CASE(G_, 5) SS_CASE(G_, 8)
  SS_ROW(8)
  SS_ROW(16)
  SS_ROW(20)
  SS_ROW(32)
#undef SS_ROW
#undef SS_CASE
  return hipErrorInvalidValue;
}

}  // namespace ss
