// Device helpers of the persistent MoE verify kernels (ss_verify.hip: one layer per launch, and decode mode;
// ss_chain.hip: a chain of layers per launch): workspace and LDS layouts, cross-workgroup hand-off primitives, x
// staging, dense rows, the router tail, the unique-expert list and the shared expert's rows.
#pragma once
#include <type_traits>

#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

constexpr int kTBv = 4;          // tokens per launch
constexpr int kMaxEv = 512;      // experts per layer (LDS tables)
constexpr int kMaxQv = 64;       // kTBv * K, K <= 16
constexpr int kSpinMax = 1 << 22;
constexpr int kXZero = 98;       // uint4 zeros an inactive A lane reads in phase C: offsets 0 .. 48 * 2 (fp32 x)
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
  alignas(16) uint4 zero_h[4];    // zeros: the h operand of A rows that do not use the expert (phase D)
  int nt, nu;
};

static_assert(kXZero * sizeof(uint4) <= sizeof(float) * kMaxQv * 16, "phase C zeros fit in hsum");

SS_DEV float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
SS_DEV float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
// The high or low bf16 of a pair as fp32 in one byte permute (the selector depends on hi only, so it is formed once
// per lane): bytes 3, 2 or 1, 0 of the pair to the top, zeros below.
SS_DEV float pick_half(uint32_t pair, int hi) {
  return __uint_as_float(__builtin_amdgcn_perm(pair, pair, hi ? 0x07060C0Cu : 0x05040C0Cu));
}

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
// The lanes holding the same expert come from ballots of the expert id's bits (ids < kMaxEv = 2^9; an unusable
// entry matches no lane), so the step has no LDS exchange and no branch per entry: the first lane of each expert
// takes the next unique index, stores its record pointer and the expert's (token, rank) bits for every token, and
// errors are raised from one uniform branch.
SS_DEV void unique_setup(const VerifyArgs& a, VSmem& s, bool tables_in_lds) {
  static_assert(kMaxEv <= 512 && kMaxQv <= 64, "9 id bits, one wave of entries");
  const int lane = threadIdx.x;
  const int nq = s.nt * a.K;
  int e = -1, slot = -1;
  bool in_e = false, valid = false;
  if (lane < nq) {
    e = s.ids[lane];
    in_e = e >= 0 && e < a.E;
    if (in_e) {
      if (tables_in_lds) {
        slot = s.map[e];
      } else {
        const int64_t mi = a.map_base + e;
        if (mi >= 0 && mi < a.map_len) slot = a.map[mi];
      }
      valid = slot >= 0 && (int64_t)slot < a.n_slots;
    }
  }
  const uint64_t bad_e = __ballot(lane < nq && !in_e), bad_s = __ballot(in_e && !valid);
  if ((bad_e | bad_s) != 0ull && lane == 0)
    ss_raise(a.err, (bad_e ? SS_ERR_EXPERT_ID : 0) | (bad_s ? SS_ERR_SLOT : 0));
  uint64_t same = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 9; ++b) {
    const bool bit = ((e >> b) & 1) != 0;
    const uint64_t bb = __ballot(valid && bit);
    same &= bit ? bb : ~bb;
  }
  const int j0 = valid ? (int)__builtin_ctzll(same) : 64;  // a valid lane is in its own set
  const bool first = valid && j0 == lane;
  const uint64_t fm = __ballot(first);
  const int uidx = valid ? __popcll(fm & ((1ull << j0) - 1ull)) : -1;
  if (first) {
    s.base[uidx] = tables_in_lds ? s.base_e[e] : reinterpret_cast<const uint8_t*>(a.slot_ptr[slot]);
    const uint32_t km = (uint32_t)((1ull << a.K) - 1ull);
#pragma unroll
    for (int t = 0; t < kTBv; ++t) s.umask[uidx][t] = t * a.K < 64 ? (uint32_t)(same >> (t * a.K)) & km : 0u;
  }
  if (lane < nq) s.use_u[lane] = uidx;
  if (lane == 0) s.nu = __popcll(fm);
}

// Router tail of token t in one wave (the operations and order of router_topk_kernel): lane l holds the entries
// e = l + 64 i. The top K in (probability desc, index asc) order come from a threshold and a rank count (below);
// the K dependent rounds of router_topk_kernel remain for the rows that path does not take. Both give the same
// ids, and the weights are summed in rank order either way.
SS_DEV void router_tail_wave(const VerifyArgs& a, const uint64_t* logits, uint32_t tag, int t, VSmem& s,
                             const float (&bias_r)[kMaxEv / 64], uint64_t* stamps = nullptr) {
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
  }
  if (a.trace && threadIdx.x == 0) a.trace[(size_t)blockIdx.x * 16 + 5] = __builtin_amdgcn_s_memrealtime();  // logits in
  if (stamps && lane == 0) stamps[0] = __builtin_amdgcn_s_memrealtime();
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
  float ve[NV];  // the exponentials, kept for the rare entries whose quotient takes the division
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    v[i] = ss_expf_le0(v[i] - m);  // v - m <= 0 (an absent entry holds entry 0's value, which is at most m)
    ve[i] = v[i];
    acc = acc + (lane + 64 * i < E ? v[i] : 0.f);
  }
  const float z = ss_wave_sum(acc);
  // v / z for every entry from one division: q = RN(v * RN(1/z)) is within an ulp of v / z, the remainder
  // v - q z is exact (fma), and RN(q + rem * RN(1/z)) is the correctly rounded quotient (Markstein's theorem; here
  // v is in [0, 1] and z in [1, E], and a v in (0, 2^-64), where the remainder could underflow, takes the
  // division itself). NaN inputs give NaN either way.
  const float rz = 1.f / z;
  bool tiny = false;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const float vi = v[i];
    const float q = vi * rz;
    const float rem = __builtin_fmaf(-q, z, vi);
    v[i] = __builtin_fmaf(rem, rz, q);
    tiny = tiny || (vi > 0.f && vi < 0x1p-64f);
  }
  if (__any(tiny)) {
    // rare (a probability below 2^-64 somewhere in the wave): every entry of the wave takes the division
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = ve[i] / z;
  }
  // kp = key + 1 for a present, untaken entry (NaN probabilities have key 0, so kp 1), 0 once taken or absent.
  uint32_t kp[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) kp[i] = lane + 64 * i < E ? ss_key(v[i]) + 1u : 0u;
  if (stamps && lane == 0) stamps[1] = __builtin_amdgcn_s_memrealtime();
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
// then the wave butterfly. Tokens go in pairs, two independent chains side by side (a token t >= nt of a pair holds
// token 0's fragments; its sum is formed and not used).
template <int NJX>
SS_DEV void dense_dot(const uint4 (&wv)[NJX], const uint4* xfl, int nt, float out[kTBv]) {
  static_assert(kTBv % 2 == 0, "token pairs");
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int t = 0; t < kTBv; t += 2) {
    if (t >= nt) break;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int jj = 0; jj < NJX; ++jj) {
      const uint4 x0 = xfl[xfrag_index(512 * jj + 8 * lane, t)];
      const uint4 x1 = xfl[xfrag_index(512 * jj + 8 * lane, t + 1)];
      const uint32_t ww[4] = {wv[jj].x, wv[jj].y, wv[jj].z, wv[jj].w};
      const uint32_t xx0[4] = {x0.x, x0.y, x0.z, x0.w};
      const uint32_t xx1[4] = {x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float wf = (e & 1) ? bf_hi(ww[e >> 1]) : bf_lo(ww[e >> 1]);
        const float xf0 = (e >> 2) ? bf_hi(xx0[e & 3]) : bf_lo(xx0[e & 3]);
        const float xf1 = (e >> 2) ? bf_hi(xx1[e & 3]) : bf_lo(xx1[e & 3]);
        a0 = __builtin_fmaf(xf0, wf, a0);
        a1 = __builtin_fmaf(xf1, wf, a1);
      }
    }
    ss_wave_sum2(a0, a1);
    out[t] = a0;
    out[t + 1] = a1;
  }
}

// Affine 4-bit (gs 64) dense rows (the shared expert's projections when the checkpoint keeps them quantized): the
// dense-row register of chunk jj holds {the word of elements 512 jj + 8 lane .. + 7 (nibble e at bits 4e), its
// group's bf16 scale | bf16 bias << 16, 0, 0}. q4_chunk loads it from words uint32 [K/8] and s, b bf16 [K/64] of
// one row.
SS_DEV uint4 q4_chunk(const uint16_t* words, const uint16_t* sc, const uint16_t* bi, int jj, int lane) {
  const int w8 = 64 * jj + lane, grp = w8 >> 3;
  const uint32_t wd = *gp(reinterpret_cast<const uint32_t*>(words + 2 * (size_t)w8));
  const uint32_t sv = *gp(sc + grp);
  const uint32_t bv = *gp(bi + grp);
  return make_uint4(wd, sv | (bv << 16), 0u, 0u);
}

// dense_dot over q4_chunk registers: each weight dequantized in fp32 first (q * s, then + b), then the dense_dot
// order (or_dense_rows_q4).
template <int NJX>
SS_DEV void affine_dot(const uint4 (&wv)[NJX], const uint4* xfl, int nt, float out[kTBv]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int t = 0; t < kTBv; t += 2) {
    if (t >= nt) break;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int jj = 0; jj < NJX; ++jj) {
      const uint4 x0 = xfl[xfrag_index(512 * jj + 8 * lane, t)];
      const uint4 x1 = xfl[xfrag_index(512 * jj + 8 * lane, t + 1)];
      const uint32_t xx0[4] = {x0.x, x0.y, x0.z, x0.w};
      const uint32_t xx1[4] = {x1.x, x1.y, x1.z, x1.w};
      const float sc = bf_lo(wv[jj].y), bi = bf_hi(wv[jj].y);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q = (float)((wv[jj].x >> (4 * e)) & 0xFu);
        const float wf = q * sc + bi;
        const float xf0 = (e >> 2) ? bf_hi(xx0[e & 3]) : bf_lo(xx0[e & 3]);
        const float xf1 = (e >> 2) ? bf_hi(xx1[e & 3]) : bf_lo(xx1[e & 3]);
        a0 = __builtin_fmaf(xf0, wf, a0);
        a1 = __builtin_fmaf(xf1, wf, a1);
      }
    }
    ss_wave_sum2(a0, a1);
    out[t] = a0;
    out[t + 1] = a1;
  }
}

// The shared-expert gate / up projections of this lane's 8 elements for every token (tokens >= nt read token 0).
struct SharedIn {
  uint4 g[kTBv], u[kTBv];
};

// Chunk c (elements 512 c + 8 l .. + 7 of lane l; Is <= 1024) of the projections.
SS_DEV SharedIn shared_load(const VerifyArgs& a, const uint16_t* gsh, const uint16_t* ush, int nt, int c = 0) {
  const int lane = threadIdx.x & 63;
  const int e0 = 512 * c + 8 * lane < a.Is ? 512 * c + 8 * lane : 0;
  SharedIn in;
#pragma unroll
  for (int t = 0; t < kTBv; ++t) {
    const int tt = t < nt ? t : 0;
    in.g[t] = ld_ag16(gsh + (size_t)tt * a.Is + e0);
    in.u[t] = ld_ag16(ush + (size_t)tt * a.Is + e0);
  }
  return in;
}

// hs = bf16(bf16(silu(g)) * u) of the shared expert (the F.silu and product of the reference, in bf16), split over
// the workgroup's four waves: wave w computes elements e0 + 2 w and e0 + 2 w + 1 of lane l's eight (e0 = 512 c + 8 l)
// for every token and stores them to hsl [nt][Is] (LDS).
SS_DEV void shared_hs_part(const VerifyArgs& a, const SharedIn& in, int w, int nt, float* hsl, int c = 0) {
  const int lane = threadIdx.x & 63;
  const int e0 = 512 * c + 8 * lane;
  if (e0 >= a.Is) return;
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
      hsl[t * a.Is + e0 + 2 * w + h] = ss_round_bf16(sv * uv);
    }
  }
}

// All of hs (both chunks when Is > 512; the second chunk's projections are loaded here, one more round trip).
template <int NSC>
SS_DEV void shared_hs_all(const VerifyArgs& a, const SharedIn& in0, const uint16_t* gsh, const uint16_t* ush, int w,
                          int nt, float* hsl) {
  shared_hs_part(a, in0, w, nt, hsl, 0);
  if (NSC > 1 && a.Is > 512) {
    const SharedIn in1 = shared_load(a, gsh, ush, nt, 1);
    shared_hs_part(a, in1, w, nt, hsl, 1);
  }
}

// The shared-expert down row registers of one wave, chunk c of row r in sh_w[r][c]: bf16 rows (the lane's 8
// elements 512 c + 8 l .. + 7), or with an affine 4-bit down projection (Q4: sh_ds, sh_db set) the q4_chunk register
// of those elements. NSC chunks per row (512 * NSC >= Is): the kernels take NSC = 2 with I > 512, else 1.
template <int NR, int NSC, bool Q4>
SS_DEV void load_shared_down(const VerifyArgs& a, int row0, uint4 (&sh_w)[NR][NSC]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int rr = 0; rr < NR; ++rr)
#pragma unroll
    for (int c = 0; c < NSC; ++c) {
      const int w8 = 64 * c + lane;
      const bool ok = 8 * w8 < a.Is;
      const size_t row = (size_t)(row0 + rr);
      sh_w[rr][c] = !ok ? make_uint4(0u, 0u, 0u, 0u)
                    : Q4 ? q4_chunk(a.sh_down + row * (a.Is / 4), a.sh_ds + row * (a.Is / 64),
                                         a.sh_db + row * (a.Is / 64), c, lane)
                              : ldg16(a.sh_down + row * a.Is + 8 * w8);
    }
}

// Shared-expert down rows of one wave, in the dense_rows order (lane l: chunk 0's elements, then chunk 1's, by fma
// from 0; then the butterfly): the dot of hs (hsl) with the down rows; out[rr][t] receives the fp32 sums (every lane).
template <int NR, int NSC, bool Q4>
SS_DEV void shared_down_rows(const VerifyArgs& a, const float* hsl, const uint4 (&sh_w)[NR][NSC], int nt,
                             float (&out)[NR][kTBv]) {
  const int lane = threadIdx.x & 63;
  float sacc[NR][kTBv];
#pragma unroll
  for (int rr = 0; rr < NR; ++rr)
#pragma unroll
    for (int t = 0; t < kTBv; ++t) sacc[rr][t] = 0.f;
#pragma unroll
  for (int c = 0; c < NSC; ++c) {
    const int e0 = 512 * c + 8 * lane;
    if (e0 >= a.Is) break;
#pragma unroll
    for (int t = 0; t < kTBv; ++t) {
      if (t >= nt) break;
      float hsv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) hsv[e] = hsl[t * a.Is + e0 + e];
#pragma unroll
      for (int rr = 0; rr < NR; ++rr) {
        const uint32_t ww[4] = {sh_w[rr][c].x, sh_w[rr][c].y, sh_w[rr][c].z, sh_w[rr][c].w};
        float ac = 0.f;
#pragma unroll
        for (int q = 0; q < kTBv; ++q)
          if (q == t) ac = sacc[rr][q];
        if (Q4) {
          const float sc = bf_lo(ww[1]), bi = bf_hi(ww[1]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float q = (float)((ww[0] >> (4 * e)) & 0xFu);
            const float wf = q * sc + bi;
            ac = __builtin_fmaf(hsv[e], wf, ac);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) ac = __builtin_fmaf(hsv[e], (e & 1) ? bf_hi(ww[e >> 1]) : bf_lo(ww[e >> 1]), ac);
        }
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

}  // namespace ss
