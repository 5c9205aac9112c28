/* CPU restatement of the bit-exact parts of the MTP-verify MoE path. TEST INFRASTRUCTURE ONLY: the checker that
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP kernels against; nothing in the
 * product links or calls it.
 *
 * Every function states the reference file:line whose semantics it follows and the fixed operation order it
 * defines. Compiled with -ffp-contract=off: a*b+c is fused only where the code says fmaf.
 *
 * Pinned by (tests/test_oracle.py, tests/test_golden.py):
 *   or_expf          fp64 exp over a dense sweep (<= 2 ulp), special values, exp(0) = 1.
 *   or_bf16_*        every one of the 65536 bf16 patterns round-trips; RNE ties against numpy/torch.
 *   or_dense_rows    fp64 dot + one rounding (agreement away from rounding boundaries); torch F.linear bf16
 *                    golden fixtures written from reference_torch.moe_ref.
 *   or_router_topk   ids: brute force stable sort of the probabilities; golden fixtures (moe_ref's torch.topk).
 *   or_topk_stable   the reference's CPU spec _ref_row (tests/t0/test_topk_stable.py:14-31) with ties, NaN,
 *                    +-inf, +-0, n_valid.
 *   or_accept_greedy np.argmax + the accept-while-equal loop, brute force.
 *   or_accept_pq     distributional check (chi-square: emitted token ~ p) on a small vocabulary, p == q always
 *                    accepts, q(x) = 0 / p(x) = 0 edge cases, hierarchical sums vs fp64 totals.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- scalars */
static float f_from_u(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t u_from_f(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

float or_bf16_to_f32(uint16_t b) { return f_from_u((uint32_t)b << 16); }

/* Round to nearest even; NaN -> quiet NaN keeping the sign. */
uint16_t or_f32_to_bf16(float f) {
  uint32_t u = u_from_f(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)(((u >> 16) | 0x40u) & 0xFFFFu);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float round_bf16(float f) { return or_bf16_to_f32(or_f32_to_bf16(f)); }

/* exp: Cody-Waite reduction with a 15-bit ln2 head, degree-7 Taylor polynomial (Horner, fmaf), 2^n scale. */
float or_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return f_from_u(0x7F800000u);
  if (x < -103.97208404541015625f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187045037746429443359375e-06f, r);
  float p = 1.98412701138295233249664306640625e-04f;
  p = fmaf(p, r, 1.38888892251998186111450195312500e-03f);
  p = fmaf(p, r, 8.33333376795053482055664062500000e-03f);
  p = fmaf(p, r, 4.16666679084300994873046875000000e-02f);
  p = fmaf(p, r, 1.66666671633720397949218750000000e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) {
    p = p * 2.0f;
    ni -= 1;
  } else if (ni < -120) {
    p = p * 5.42101086242752217003726400434970855712890625e-20f;
    ni += 64;
  }
  return p * f_from_u((uint32_t)(ni + 127) << 23);
}

/* Order-preserving key: kernels/topk_stable.py:1-13 (NaN -> 0, negatives bitwise not, positives sign flip). */
uint32_t or_key(float f) {
  const uint32_t u = u_from_f(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0u;
  return (u & 0x80000000u) ? ~u : (u ^ 0x80000000u);
}

/* 64-lane xor butterfly: lane l += lane l^32, then ^16 ... ^1; returns lane 0. */
static float butterfly_sum(const float* v64) {
  float a[64], b[64];
  memcpy(a, v64, sizeof a);
  for (int m = 32; m >= 1; m >>= 1) {
    for (int l = 0; l < 64; ++l) b[l] = a[l] + a[l ^ m];
    memcpy(a, b, sizeof a);
  }
  return a[0];
}

/* ---------------------------------------------------------------- dense bf16 rows
 * out[t, n] = bf16(sum_k x[t, k] w[n, k]) (model/layers.py:62-76, reference_torch.py:121). Order: lane l of 64
 * accumulates chunks j = 0, 1, ...: elements 512j + 8l .. 512j + 8l + 7 with fmaf from 0; then the butterfly. */
void or_dense_rows(const uint16_t* x, const uint16_t* w, uint16_t* out, int T, int H, int N) {
  const int h8 = H / 8, nj = (H + 511) / 512;
  for (int t = 0; t < T; ++t) {
    for (int n = 0; n < N; ++n) {
      float lanes[64];
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int j = 0; j < nj; ++j) {
          const int k8 = 64 * j + l;
          if (k8 >= h8) break;
          for (int e = 0; e < 8; ++e) {
            const int k = 8 * k8 + e;
            acc = fmaf(or_bf16_to_f32(x[(size_t)t * H + k]), or_bf16_to_f32(w[(size_t)n * H + k]), acc);
          }
        }
        lanes[l] = acc;
      }
      out[(size_t)t * N + n] = or_f32_to_bf16(butterfly_sum(lanes));
    }
  }
}

/* Dense rows over affine 4-bit (gs 64) weights, the dot products of the shared expert when the checkpoint keeps it
 * quantized (reference: lin -> gemv on an AffineWeight, model/layers.py:62-76, kernels/gemv_affine.py:214-262,
 * w = q * s + b of kernels/affine_ref.py:10-30). words uint32 [N][K/8] (nibble i of a word at bits 4i), s, b bf16
 * [N][K/64]. The or_dense_rows order with each weight dequantized in fp32 first (a multiply, then an add: two
 * roundings): lane l accumulates elements 512 j + 8 l .. + 7 by fmaf from 0, then the butterfly, one rounding to
 * bf16. With s = 1 and b = 0 every weight is the integer q and the result equals or_dense_rows on bf16(q) bit for
 * bit. */
void or_dense_rows_q4(const uint16_t* x, const uint32_t* words, const uint16_t* s, const uint16_t* b, uint16_t* out,
                      int T, int K, int N) {
  const int k8 = K / 8, nj = (K + 511) / 512, ng = K / 64;
  for (int t = 0; t < T; ++t) {
    for (int n = 0; n < N; ++n) {
      float lanes[64];
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int j = 0; j < nj; ++j) {
          const int w8 = 64 * j + l;
          if (w8 >= k8) break;
          const uint32_t wd = words[(size_t)n * k8 + w8];
          const int grp = (8 * w8) / 64;
          const float sc = or_bf16_to_f32(s[(size_t)n * ng + grp]), bi = or_bf16_to_f32(b[(size_t)n * ng + grp]);
          for (int e = 0; e < 8; ++e) {
            const int k = 8 * w8 + e;
            const float q = (float)((wd >> (4 * e)) & 0xFu);
            const float prod = q * sc;
            const float wgt = prod + bi;
            acc = fmaf(or_bf16_to_f32(x[(size_t)t * K + k]), wgt, acc);
          }
        }
        lanes[l] = acc;
      }
      out[(size_t)t * N + n] = or_f32_to_bf16(butterfly_sum(lanes));
    }
  }
}

/* ---------------------------------------------------------------- router tail
 * model/layers.py:340-347, reference_torch.py:122-124. scores s = bf16 logit (+ bias, one fp32 add);
 * m = max (NaN ignored); e = exp(s - m); Z: lane l sums e[l], e[l+64], ... sequentially from 0, then the butterfly;
 * p = e / Z; top-k: K rounds of (largest key, lowest index) among the untaken; w = p / S, S the sequential
 * rank-order sum of the K probabilities. */
void or_router_topk(const uint16_t* logits, const float* bias, float* probs, int32_t* ids, float* weights, int T,
                    int E, int K, float* scratch /* [2E] */) {
  float* s = scratch;
  uint8_t* taken = (uint8_t*)(scratch + E);
  for (int t = 0; t < T; ++t) {
    float m = -INFINITY;
    for (int e = 0; e < E; ++e) {
      float v = or_bf16_to_f32(logits[(size_t)t * E + e]);
      if (bias) v = v + bias[e];
      s[e] = v;
      m = fmaxf(m, v);
      taken[e] = 0;
    }
    float lanes[64];
    for (int l = 0; l < 64; ++l) lanes[l] = 0.0f;
    for (int e = 0; e < E; ++e) {
      const float v = or_expf(s[e] - m);
      s[e] = v;
      lanes[e % 64] = lanes[e % 64] + v;
    }
    const float z = butterfly_sum(lanes);
    for (int e = 0; e < E; ++e) {
      s[e] = s[e] / z;
      if (probs) probs[(size_t)t * E + e] = s[e];
    }
    float tv[64];
    for (int r = 0; r < K; ++r) {
      uint32_t bk = 0;
      int bi = 0x7FFFFFFF;
      for (int e = 0; e < E; ++e) {
        if (taken[e]) continue;
        const uint32_t k = or_key(s[e]);
        if (k > bk || (k == bk && e < bi)) {
          bk = k;
          bi = e;
        }
      }
      taken[bi] = 1;
      ids[(size_t)t * K + r] = bi;
      tv[r] = s[bi];
    }
    float S = 0.0f;
    for (int r = 0; r < K; ++r) S = S + tv[r];
    for (int r = 0; r < K; ++r) weights[(size_t)t * K + r] = tv[r] / S;
  }
}

/* ---------------------------------------------------------------- topk_stable
 * kernels/topk_stable.py:85-113 with the CPU spec of tests/t0/test_topk_stable.py:14-31: stable order by
 * (key desc, index asc) over the first n_valid entries; k <= 16 keeps that order, larger k re-sorts the selected
 * indices ascending; missing entries are -1 / -inf. O(N * k) selection, fine for test sizes. */
void or_topk_stable(const float* scores, const int32_t* n_valid, int32_t* idx, float* val, int R, int N, int k,
                    uint8_t* taken /* [N] */) {
  for (int r = 0; r < R; ++r) {
    const float* x = scores + (size_t)r * N;
    int nv = N;
    if (n_valid) nv = n_valid[r] < 0 ? 0 : (n_valid[r] > N ? N : n_valid[r]);
    const int want = k < nv ? k : nv;
    memset(taken, 0, (size_t)N);
    int32_t* oi = idx + (size_t)r * k;
    for (int a = 0; a < want; ++a) {
      uint32_t bk = 0;
      int bi = -1;
      for (int i = 0; i < nv; ++i) {
        if (taken[i]) continue;
        const uint32_t kk = or_key(x[i]);
        if (bi < 0 || kk > bk) {
          bk = kk;
          bi = i;
        }
      }
      taken[bi] = 1;
      oi[a] = bi;
    }
    if (k > 16) { /* by index ascending */
      int p = 0;
      for (int i = 0; i < nv; ++i)
        if (taken[i]) oi[p++] = i;
    }
    for (int a = 0; a < want; ++a)
      if (val) val[(size_t)r * k + a] = x[oi[a]];
    for (int a = want; a < k; ++a) {
      oi[a] = -1;
      if (val) val[(size_t)r * k + a] = -INFINITY;
    }
  }
}

/* ---------------------------------------------------------------- acceptance */
#define SUB 16
#define CHUNK 1024

static int is_finite_f(float v) { return (u_from_f(v) & 0x7F800000u) != 0x7F800000u; }

/* Greedy: engine/generate.py:208-229, engine/sampler.py:83-84 (np.argmax: first maximum). out as ssmoe.h. */
void or_accept_greedy(const float* target, const int32_t* drafts, int D, int V, int32_t* out) {
  int good = 0, emit = 0, flags = 0;
  for (int i = 0; i <= D; ++i) {
    const float* x = target + (size_t)i * V;
    int bad = 0, bi = 0;
    float best = -INFINITY;
    int have = 0;
    for (int j = 0; j < V; ++j) {
      if (!is_finite_f(x[j])) bad = 1;
      if (!have || x[j] > best) {
        if (x[j] == x[j]) {
          best = x[j];
          bi = j;
          have = 1;
        }
      }
    }
    if (bad) {
      flags |= 1;
      break;
    }
    out[4 + emit++] = bi;
    if (i < D && bi == drafts[i]) {
      ++good;
      continue;
    }
    break;
  }
  for (int i = emit; i <= D; ++i) out[4 + i] = -1;
  out[0] = good;
  out[1] = emit;
  out[2] = 0;
  out[3] = flags;
}

/* Hierarchical sum of f(j): sub-chunk totals (sequential from 0), chunk totals (butterfly), row (sequential). */
typedef float (*ValFn)(const void* ctx, int j);

static float chunk_total(ValFn f, const void* ctx, int c, int V, float* sub /* [64] or NULL */) {
  float lanes[64];
  for (int b = 0; b < 64; ++b) {
    float s = 0.0f;
    for (int i = 0; i < SUB; ++i) {
      const int j = c * CHUNK + b * SUB + i;
      if (j < V) s = s + f(ctx, j);
    }
    lanes[b] = s;
    if (sub) sub[b] = s;
  }
  return butterfly_sum(lanes);
}

/* ---------------------------------------------------------------- p/q acceptance (Leviathan et al. 2023, Alg. 1)
 * No reference counterpart. Every sum has a fixed order made of two pieces, so that the kernels form it with
 * lane-parallel operations:
 *   scan64: the inclusive prefix of 64 nonnegative values: Hillis-Steele steps d = 1, 2, 4, 8 inside each row of
 *   16 (P_l += P_{l-d} when l - d is in the row, each step from the previous step's values), then rows 1 and 3 add
 *   the last value of the row before (P_15, P_47), then rows 2 and 3 add P_31 of that step; every addition is
 *   (own + other); total64 = the last prefix. (The kernels form it with DPP row shifts and row broadcasts.)
 *   a "lane layout" of n values with k per lane: lane l holds values k l .. k l + k - 1 (those < n); its local sum is
 *   the sequential sum from 0; the layout's prefixes are scan64 of the local sums.
 * Per row (logits x, V entries, 1024-entry chunks c, invT = 1 / T in fp32):
 *   y_j = x_j * invT; m_c = max of y_j over the chunk (NaN ignored); e_j = exp(y_j - m_c);
 *   s_c = total64 of the chunk's 64 sub-chunks of 16 (lane layout k = 16: sub-chunk l = entries 16 l .. 16 l + 15);
 *   M = max m_c; g_c = exp(m_c - M); Z = total64 of t_c = s_c * g_c in the lane layout k = ceil(nch / 64);
 *   a_c = g_c / Z; p_j = e_j * a_c.
 * The drafts: x_i is accepted iff u_i * q_i(x_i) < p_i(x_i) (p, q of target row i and draft row i); the first
 * rejection samples from v_j = max(0, p_j - q_j) of row i, and every draft accepted from v_j = p_j of row D. A
 * non-finite logit in a row the round reaches stops it; a draft outside [0, V) is flagged and rejected.
 * The sample after a rejection: r_c = total64 of the chunk's sub-chunk sums of v; S = total64 of r_c in the chunk
 * lane layout; target u * S. descend() on the chunk layout gives the chunk cs and its base b; descend() on chunk cs's
 * sub-chunks with target (u * S - b) gives the entry. With every draft accepted, the sample from p_D is drawn as
 * or_draw_rows draws: the chunk by its mass r_c = s_c * a_c, the entry by its e with target (u * S - b) / a_cs. */
#define PQ_MAX_NCH 1024

static void scan64(const float* L, float* P) {
  float a[64], b[64];
  memcpy(a, L, sizeof a);
  for (int d = 1; d < 16; d <<= 1) {
    for (int l = 0; l < 64; ++l) b[l] = (l & 15) >= d ? a[l] + a[l - d] : a[l];
    memcpy(a, b, sizeof a);
  }
  for (int l = 0; l < 64; ++l) b[l] = (l >> 4) == 1 ? a[l] + a[15] : (l >> 4) == 3 ? a[l] + a[47] : a[l];
  memcpy(a, b, sizeof a);
  for (int l = 0; l < 64; ++l) b[l] = (l >> 4) >= 2 ? a[l] + a[31] : a[l];
  memcpy(P, b, sizeof b);
}

/* Local sums of a lane layout of n values with k per lane. */
static void lane_sums(const float* v, int n, int k, float* L) {
  for (int l = 0; l < 64; ++l) {
    float s = 0.0f;
    for (int i = 0; i < k && k * l + i < n; ++i) s = s + v[k * l + i];
    L[l] = s;
  }
}

/* The search over a lane layout (n values, k per lane) for target t: the first lane holding values whose prefix
 * exceeds t (else the last lane with a nonzero local sum, else lane 0), then inside it the first value whose running
 * sum from the lane's exclusive prefix exceeds t (else its last nonzero value, else its first); *base receives the
 * running sum before the chosen value. Returns the value's index, clamped to n - 1. (The scan's prefixes need not
 * rise with l by the last ulp, so an empty lane past the values could otherwise be the first to exceed t.) */
static int descend(const float* v, int n, int k, float t, float* base) {
  float L[64], P[64];
  lane_sums(v, n, k, L);
  scan64(L, P);
  int ls = -1;
  for (int l = 0; l < 64 && ls < 0 && k * l < n; ++l)
    if (P[l] > t) ls = l;
  if (ls < 0) {
    for (int l = 0; l < 64; ++l)
      if (L[l] > 0.0f) ls = l;
    if (ls < 0) ls = 0;
  }
  const float e = ls > 0 ? P[ls - 1] : 0.0f;
  float run = e;
  int pick = -1, last = -1;
  for (int i = 0; i < k && k * ls + i < n; ++i) {
    const float x = v[k * ls + i];
    if (x > 0.0f) last = i;
    const float nx = run + x;
    if (nx > t) {
      pick = i;
      break;
    }
    run = nx;
  }
  if (pick < 0) {
    pick = last >= 0 ? last : 0;
    run = e;
    for (int i = 0; i < pick; ++i) run = run + v[k * ls + i];
  }
  *base = run;
  const int idx = k * ls + pick;
  return idx < n ? idx : n - 1;
}

typedef struct {
  float m[PQ_MAX_NCH], a[PQ_MAX_NCH], s[PQ_MAX_NCH];
  float M, Z;
  int bad;
} PqRow;

static float pq_inv(float temp) { return 1.0f / temp; }

/* e_j of chunk c's maximum for one row (y = x * invT). */
static float pq_e(const float* x, int j, float invT, float mc) { return or_expf(x[j] * invT - mc); }

static void pq_row(const float* x, int V, float invT, PqRow* r) {
  const int nch = (V + CHUNK - 1) / CHUNK, kc = (nch + 63) / 64;
  float s[PQ_MAX_NCH], t[PQ_MAX_NCH], g[PQ_MAX_NCH];
  r->bad = 0;
  r->M = -INFINITY;
  for (int c = 0; c < nch; ++c) {
    float mc = -INFINITY;
    for (int j = c * CHUNK; j < V && j < (c + 1) * CHUNK; ++j) {
      if (!is_finite_f(x[j])) r->bad = 1;
      mc = fmaxf(mc, x[j] * invT);
    }
    float e[CHUNK], L[64], P[64];
    for (int i = 0; i < CHUNK; ++i) {
      const int j = c * CHUNK + i;
      e[i] = j < V ? pq_e(x, j, invT, mc) : 0.0f;
    }
    lane_sums(e, CHUNK, SUB, L);
    scan64(L, P);
    r->m[c] = mc;
    s[c] = P[63];
    r->s[c] = s[c];
    r->M = fmaxf(r->M, mc);
  }
  for (int c = 0; c < nch; ++c) {
    g[c] = or_expf(r->m[c] - r->M);
    t[c] = s[c] * g[c];
  }
  float L[64], P[64];
  lane_sums(t, nch, kc, L);
  scan64(L, P);
  r->Z = P[63];
  for (int c = 0; c < nch; ++c) r->a[c] = g[c] / r->Z;
}

static float pq_p(const float* x, int j, float invT, const PqRow* r) {
  const int c = j / CHUNK;
  return pq_e(x, j, invT, r->m[c]) * r->a[c];
}

/* out as ssmoe.h; work is unused (kept for the binding). */
void or_accept_pq(const float* target, const float* draft, const int32_t* drafts, const float* uniforms, int D,
                  int V, float temp, int32_t* out, float* work) {
  (void)work;
  const int nch = (V + CHUNK - 1) / CHUNK, kc = (nch + 63) / 64;
  const float invT = pq_inv(temp);
  PqRow* rt = (PqRow*)calloc((size_t)(D + 1), sizeof(PqRow));
  PqRow* rd = (PqRow*)calloc((size_t)(D > 0 ? D : 1), sizeof(PqRow));
  for (int i = 0; i <= D; ++i) pq_row(target + (size_t)i * V, V, invT, &rt[i]);
  for (int i = 0; i < D; ++i) pq_row(draft + (size_t)i * V, V, invT, &rd[i]);
  int good = 0, flags = 0, stop = 0, srow = D, sdraft = -1;
  for (int i = 0; i < D; ++i) {
    if (rt[i].bad || rd[i].bad) {
      flags |= 1;
      stop = 1;
      break;
    }
    const int x = drafts[i];
    if (x < 0 || x >= V) {
      flags |= 2;
      srow = i;
      sdraft = i;
      break;
    }
    const float p = pq_p(target + (size_t)i * V, x, invT, &rt[i]);
    const float q = pq_p(draft + (size_t)i * V, x, invT, &rd[i]);
    if (uniforms[i] * q < p) {
      ++good;
      continue;
    }
    srow = i;
    sdraft = i;
    break;
  }
  if (!stop && sdraft < 0 && rt[D].bad) {
    flags |= 1;
    stop = 1;
  }
  const int uidx = good + (sdraft >= 0 ? 1 : 0);
  for (int i = 0; i < good; ++i) out[4 + i] = drafts[i];
  int emit = good;
  if (!stop && sdraft < 0) {
    const PqRow* pr = &rt[D];
    const float* x = target + (size_t)D * V;
    float rc[PQ_MAX_NCH], L[64], P[64], e[CHUNK];
    for (int c = 0; c < nch; ++c) rc[c] = pr->s[c] * pr->a[c];
    lane_sums(rc, nch, kc, L);
    scan64(L, P);
    if (!(P[63] > 0.0f)) flags |= 4;
    const float tu = uniforms[uidx] * P[63];
    float cbase = 0.0f, ebase = 0.0f;
    const int cs = descend(rc, nch, kc, tu, &cbase);
    const int n_in = V - cs * CHUNK < CHUNK ? V - cs * CHUNK : CHUNK;
    for (int i = 0; i < n_in; ++i) e[i] = pq_e(x, cs * CHUNK + i, invT, pr->m[cs]);
    out[4 + emit++] = cs * CHUNK + descend(e, n_in, SUB, (tu - cbase) / pr->a[cs], &ebase);
  } else if (!stop) {
    const float* tp = target + (size_t)srow * V;
    const float* dq = draft + (size_t)sdraft * V;
    float* v = (float*)malloc(sizeof(float) * (size_t)nch * CHUNK);
    float r[PQ_MAX_NCH];
    for (int c = 0; c < nch; ++c) {
      for (int i = 0; i < CHUNK; ++i) {
        const int j = c * CHUNK + i;
        float x = 0.0f;
        if (j < V) {
          const float d = pq_p(tp, j, invT, &rt[srow]) - pq_p(dq, j, invT, &rd[sdraft]);
          x = d > 0.0f ? d : 0.0f;
        }
        v[(size_t)c * CHUNK + i] = x;
      }
      float L[64], P[64];
      lane_sums(v + (size_t)c * CHUNK, CHUNK, SUB, L);
      scan64(L, P);
      r[c] = P[63];
    }
    float L[64], P[64];
    lane_sums(r, nch, kc, L);
    scan64(L, P);
    const float S = P[63];
    if (!(S > 0.0f)) flags |= 4;
    const float tu = uniforms[uidx] * S;
    float cbase = 0.0f, ebase = 0.0f;
    const int cs = descend(r, nch, kc, tu, &cbase);
    const int n_in = V - cs * CHUNK < CHUNK ? V - cs * CHUNK : CHUNK;
    const int e = descend(v + (size_t)cs * CHUNK, n_in, SUB, tu - cbase, &ebase);
    out[4 + emit++] = cs * CHUNK + e;
    free(v);
  }
  for (int i = emit; i <= D; ++i) out[4 + i] = -1;
  out[0] = good;
  out[1] = emit;
  out[2] = stop ? uidx : uidx + 1;
  out[3] = flags;
  free(rt);
  free(rd);
}

/* Draws x_r ~ softmax(logits[r] / temp) for R rows (ssmoe_sample_rows, the proposal of the p/q round; no reference
 * counterpart), with the p/q round's row statistics: the chunk by descend() over the chunk masses r_c = s_c * a_c
 * (k = ceil(nch / 64)) with target t = u_r * S, S their layout total; inside chunk cs the entry by descend() over its
 * e values (k = 16) with target (t - base) / a_cs. A row with a non-finite logit yields an index in [0, V) of no
 * meaning (the p/q round stops at that row). */
void or_draw_rows(const float* logits, int R, int V, float temp, const float* uniforms, int32_t* tokens) {
  const int nch = (V + CHUNK - 1) / CHUNK, kc = (nch + 63) / 64;
  const float invT = pq_inv(temp);
  PqRow* pr = (PqRow*)malloc(sizeof(PqRow));
  for (int r = 0; r < R; ++r) {
    const float* x = logits + (size_t)r * V;
    pq_row(x, V, invT, pr);
    float rc[PQ_MAX_NCH], L[64], P[64], e[CHUNK];
    for (int c = 0; c < nch; ++c) rc[c] = pr->s[c] * pr->a[c];
    lane_sums(rc, nch, kc, L);
    scan64(L, P);
    const float t = uniforms[r] * P[63];
    float cbase = 0.0f, ebase = 0.0f;
    const int cs = descend(rc, nch, kc, t, &cbase);
    const int n_in = V - cs * CHUNK < CHUNK ? V - cs * CHUNK : CHUNK;
    for (int i = 0; i < n_in; ++i) e[i] = pq_e(x, cs * CHUNK + i, invT, pr->m[cs]);
    tokens[r] = cs * CHUNK + descend(e, n_in, SUB, (t - cbase) / pr->a[cs], &ebase);
  }
  free(pr);
}

/* Row total Z of the p/q rows at temperature temp (exposed for the sum-order tests). */
float or_row_z(const float* x, int V, float temp) {
  PqRow* r = (PqRow*)malloc(sizeof(PqRow));
  pq_row(x, V, pq_inv(temp), r);
  const float z = r->Z;
  free(r);
  return z;
}

/* ---------------------------------------------------------------- shared expert (bf16 chain)
 * reference_torch.py:132-133 / model/layers.py:398-402 in bf16: g, u = bf16 projections (or_dense_rows);
 * hs = bf16(bf16(silu(g)) * u); sh = or_dense_rows(hs, Wd); gate = bf16(sigmoid(bf16 projection));
 * sh2 = bf16(gate * sh). silu(v) = v / (1 + exp(-v)); sigmoid(v) = 1 / (1 + exp(-v)). */
void or_shared_hs(const uint16_t* g, const uint16_t* u, uint16_t* hs, int n) {
  for (int i = 0; i < n; ++i) {
    const float gv = or_bf16_to_f32(g[i]), uv = or_bf16_to_f32(u[i]);
    const float sv = round_bf16(gv / (1.0f + or_expf(-gv)));
    hs[i] = or_f32_to_bf16(sv * uv);
  }
}

/* y = bf16(bf16(routed) + bf16(bf16(sigmoid(sgl)) * sh)), all [T, H] except sgl [T]. */
void or_combine_shared(const float* routed, const uint16_t* sh, const uint16_t* sgl, uint16_t* y, int T, int H) {
  for (int t = 0; t < T; ++t) {
    const float s = or_bf16_to_f32(sgl[t]);
    const float sg = round_bf16(1.0f / (1.0f + or_expf(-s)));
    for (int n = 0; n < H; ++n) {
      const float sh2 = round_bf16(sg * or_bf16_to_f32(sh[(size_t)t * H + n]));
      y[(size_t)t * H + n] = or_f32_to_bf16(round_bf16(routed[(size_t)t * H + n]) + sh2);
    }
  }
}

/* Residual add + RMSNorm (runtime/graphs.py:169 with one stream, model/reference_torch.py:30-38):
 * s = bf16(resid + y) (y NULL: s = resid), r = 1 / sqrt(sum(s^2) / H + eps) with the sum of lane l over elements
 * 512 j + 8 l .. + 7 by fmaf from 0 then the butterfly, mixed = bf16((s * r) * w) (w NULL: 1). */
void or_residual_rmsnorm(const uint16_t* resid, const uint16_t* y, const uint16_t* w, float eps, int R, int H,
                         uint16_t* stream_out, uint16_t* mixed) {
  for (int t = 0; t < R; ++t) {
    const uint16_t* xr = resid + (size_t)t * H;
    uint16_t* sr = stream_out + (size_t)t * H;
    for (int k = 0; k < H; ++k)
      sr[k] = y ? or_f32_to_bf16(or_bf16_to_f32(xr[k]) + or_bf16_to_f32(y[(size_t)t * H + k])) : xr[k];
    float lanes[64];
    for (int l = 0; l < 64; ++l) {
      float acc = 0.0f;
      for (int k8 = l; k8 < H / 8; k8 += 64)
        for (int e = 0; e < 8; ++e) {
          const float v = or_bf16_to_f32(sr[8 * k8 + e]);
          acc = fmaf(v, v, acc);
        }
      lanes[l] = acc;
    }
    const float r = 1.0f / sqrtf(butterfly_sum(lanes) / (float)H + eps);
    for (int k = 0; k < H; ++k)
      mixed[(size_t)t * H + k] = or_f32_to_bf16((or_bf16_to_f32(sr[k]) * r) * (w ? or_bf16_to_f32(w[k]) : 1.0f));
  }
}

/* Elementwise or_expf over an array (test helper). */
void or_expf_vec(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = or_expf(x[i]);
}

/* ---------------------------------------------------------------- reference sampler (engine/sampler.py:76-108)
 * Sampler.next with sanitized parameters, in the order of the reference: presence penalty on the raw logits
 * (:80-82), argmax at temperature <= 0 (:83-84), division by the temperature (:85), top-k threshold (:86-88),
 * softmax (:89, :67-69), top-p (:90-97), min-p (:98-100), inverse CDF with the uniform u (:101-108). Every float op
 * is the reference's float32 op; the order of each sum is this build's (the reference's comes from numpy: its
 * pairwise e.sum() and sequential cumsums, and its exp is numpy's):
 *   z, the top-p cumulative mass and the final total use the hierarchical order of the acceptance sums (sub-chunks
 *   of 16 summed sequentially, 64 sub-chunk totals of a 1024-entry chunk by the xor butterfly, chunk totals
 *   sequentially); exp is or_expf.
 *   top-p: entry j ranks by rho_j = key(p_j) << 20 | (2^20 - 1 - j) (probability descending, then index
 *   ascending, the stable argsort of :91); cum(rho) = hierarchical sum of p_i over rho_i > rho; j is kept iff
 *   cum(rho_j) < top_p (the reference's (cum - srt) < top_p with cum - srt = the mass ranked before j).
 *   draw: cdf_j is the hierarchical running sum (chunk base, then sub-chunk base, then the entries of the
 *   sub-chunk); the pick is the first entry with cdf_j >= u * total (u == 0: cdf_j > 0), found chunk, then
 *   sub-chunk, then entry, each level falling back to the last nonzero one; the reference counts cdf < u * total.
 * out[0] = token, out[1] = flags (1 = the total was not finite and > 0: argmax of the raw logits, :105-106). */
static int in_sorted(const int32_t* g, int n, int j) {
  int lo = 0, hi = n - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    if (g[mid] == j) return 1;
    if (g[mid] < j) lo = mid + 1;
    else hi = mid - 1;
  }
  return 0;
}

/* np.argmax: the first maximum, NaN counting as the largest (its first occurrence wins); -0 == +0. */
static int argmax_np(const float* x, int V) {
  int bi = 0;
  for (int j = 0; j < V; ++j) {
    const float v = x[j], b = x[bi];
    if (b != b) break;
    if (v != v || v > b) bi = j;
  }
  return bi;
}

/* NaN-largest order-preserving key with -0 == +0 (np.sort order of :87). */
static uint32_t nkey(float v) {
  if (v != v) return 0xFFFFFFFFu;
  return or_key(v == 0.0f ? 0.0f : v);
}

typedef struct {
  const float* w;
} ArrCtx;
static float val_arr(const void* c, int j) { return ((const ArrCtx*)c)->w[j]; }

typedef struct {
  const float* p;
  uint64_t rho;
} CumCtx;
static uint64_t rho_of(float p, int j) { return ((uint64_t)or_key(p) << 20) | (uint64_t)((1u << 20) - 1u - (uint32_t)j); }
static float val_cum(const void* c, int j) {
  const CumCtx* k = (const CumCtx*)c;
  return rho_of(k->p[j], j) > k->rho ? k->p[j] : 0.0f;
}

static float hsum(ValFn f, const void* ctx, int V) {
  const int nch = (V + CHUNK - 1) / CHUNK;
  float s = 0.0f;
  for (int c = 0; c < nch; ++c) s = s + chunk_total(f, ctx, c, V, NULL);
  return s;
}

/* The first entry whose hierarchical running sum reaches the target (ge: >=, else >), with fallbacks. */
static int hsearch(const float* w, int V, float target, int ge) {
  ArrCtx ctx = {w};
  const int nch = (V + CHUNK - 1) / CHUNK;
  float sub[64];
  int cs = -1, clast = -1;
  float base = 0.0f, run = 0.0f;
  for (int c = 0; c < nch; ++c) {
    const float t = chunk_total(val_arr, &ctx, c, V, NULL);
    const float nx = run + t;
    if (t > 0.0f) clast = c;
    if (cs < 0 && (ge ? nx >= target : nx > target)) {
      cs = c;
      base = run;
    }
    run = nx;
  }
  if (cs < 0) {
    cs = clast < 0 ? 0 : clast;
    base = 0.0f;
    for (int c = 0; c < cs; ++c) base = base + chunk_total(val_arr, &ctx, c, V, NULL);
  }
  chunk_total(val_arr, &ctx, cs, V, sub);
  int bs = -1, blast = -1;
  float sbase = base;
  run = base;
  for (int b = 0; b < 64; ++b) {
    const float nx = run + sub[b];
    if (sub[b] > 0.0f) blast = b;
    if (bs < 0 && (ge ? nx >= target : nx > target)) {
      bs = b;
      sbase = run;
    }
    run = nx;
  }
  if (bs < 0) {
    bs = blast < 0 ? 0 : blast;
    sbase = base;
    for (int b = 0; b < bs; ++b) sbase = sbase + sub[b];
  }
  int pick = -1, last = -1;
  run = sbase;
  for (int i = 0; i < SUB; ++i) {
    const int j = cs * CHUNK + bs * SUB + i;
    if (j >= V) break;
    if (w[j] > 0.0f) last = j;
    run = run + w[j];
    if (ge ? run >= target : run > target) {
      pick = j;
      break;
    }
  }
  if (pick < 0) pick = last >= 0 ? last : (cs * CHUNK + bs * SUB < V ? cs * CHUNK + bs * SUB : V - 1);
  return pick;
}

/* work: >= 2 V floats. */
void or_sample(const float* x, int V, const int32_t* gen, int n_gen, float temperature, float top_p, int top_k,
               float min_p, float presence_penalty, float u, int32_t* out, float* work) {
  float* l = work;
  float* p = work + V;
  for (int j = 0; j < V; ++j)
    l[j] = (presence_penalty != 0.0f && n_gen > 0 && in_sorted(gen, n_gen, j)) ? x[j] - presence_penalty : x[j];
  out[1] = 0;
  if (temperature <= 0.0f) {
    out[0] = argmax_np(l, V);
    return;
  }
  for (int j = 0; j < V; ++j) l[j] = l[j] / temperature;
  if (top_k > 0 && top_k < V) {
    /* the top_k-th largest key (counting multiplicity), by a bitwise search from the top */
    uint32_t kk = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = kk | (1u << bit);
      int cnt = 0;
      for (int j = 0; j < V; ++j) cnt += nkey(l[j]) >= cand;
      if (cnt >= top_k) kk = cand;
    }
    float kth = 0.0f;
    for (int j = 0; j < V; ++j)
      if (nkey(l[j]) == kk) {
        kth = l[j];
        break;
      }
    for (int j = 0; j < V; ++j) l[j] = l[j] < kth ? -INFINITY : l[j];
  }
  float m = -INFINITY;
  int nan = 0;
  for (int j = 0; j < V; ++j) {
    nan |= l[j] != l[j];
    m = fmaxf(m, l[j]);
  }
  if (nan) m = NAN;
  for (int j = 0; j < V; ++j) p[j] = or_expf(l[j] - m);
  ArrCtx pc = {p};
  const float z = hsum(val_arr, &pc, V);
  for (int j = 0; j < V; ++j) p[j] = p[j] / z;
  if (top_p < 1.0f) {
    /* the smallest rho with cum(rho) < top_p (cum falls as rho grows); bits 52..0 from the top */
    uint64_t r = 0;
    for (int bit = 51; bit >= 0; --bit) {
      const uint64_t hi = r | (((uint64_t)1 << bit) - 1) ; /* candidate: the largest value with this bit 0 */
      CumCtx cc = {p, hi};
      if (!(hsum(val_cum, &cc, V) < top_p)) r |= (uint64_t)1 << bit;
    }
    for (int j = 0; j < V; ++j) l[j] = rho_of(p[j], j) >= r ? p[j] : 0.0f;
    memcpy(p, l, sizeof(float) * (size_t)V);
  }
  if (min_p > 0.0f) {
    float pm = -INFINITY;
    for (int j = 0; j < V; ++j) pm = fmaxf(pm, p[j]);
    const float cutoff = pm * min_p;
    for (int j = 0; j < V; ++j) p[j] = p[j] < cutoff ? 0.0f : p[j];
  }
  const float total = hsum(val_arr, &pc, V);
  if (!is_finite_f(total) || !(total > 0.0f)) {
    out[0] = argmax_np(x, V);
    out[1] = 1;
    return;
  }
  out[0] = u == 0.0f ? hsearch(p, V, 0.0f, 0) : hsearch(p, V, u * total, 1);
}

/* ---------------------------------------------------------------- MTP head, dense part (no attention)
 * RMSNorm over groups (model/reference_torch.py:30-38 with `group`): per group of G elements of a row,
 * r = 1 / sqrt(sum(x^2) / G + eps) with the sum of lane l over the 8-element chunks l, l + 64, ... of the group by
 * fmaf from 0, then the butterfly; out = bf16((x r) w) (w NULL: 1). */
void or_rmsnorm_groups(const uint16_t* x, const uint16_t* w, float eps, int R, int n, int G, uint16_t* out) {
  for (int t = 0; t < R; ++t)
    for (int g = 0; g < n / G; ++g) {
      const uint16_t* xr = x + (size_t)t * n + (size_t)g * G;
      float lanes[64];
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int k8 = l; k8 < G / 8; k8 += 64)
          for (int e = 0; e < 8; ++e) {
            const float v = or_bf16_to_f32(xr[8 * k8 + e]);
            acc = fmaf(v, v, acc);
          }
        lanes[l] = acc;
      }
      const float r = 1.0f / sqrtf(butterfly_sum(lanes) / (float)G + eps);
      for (int k = 0; k < G; ++k)
        out[(size_t)t * n + (size_t)g * G + k] =
            or_f32_to_bf16((or_bf16_to_f32(xr[k]) * r) * (w ? or_bf16_to_f32(w[(size_t)g * G + k]) : 1.0f));
    }
}

static float sigmoid_f(float v) { return 1.0f / (1.0f + or_expf(-v)); }

/* lin on a bf16 weight with the op after it (model/layers.py:62-76, 192-198; engine/mtp.py:189-192): the dot of
 * or_dense_rows (any K a multiple of 8), v = bf16(dot), then epi 0: v; 1: bf16(add[r / add_div][n] + v);
 * 2: silu(bf16(v / hc)); 3: sigmoid(v); 4: 2 bf16(sigmoid(bf16(v / hc))), each rounded to bf16. */
void or_dense_epi(const uint16_t* x, int R, int K, const uint16_t* w, int N, int epi, int hc, const uint16_t* add,
                  int add_div, uint16_t* out) {
  uint16_t* dots = (uint16_t*)malloc((size_t)R * N * sizeof(uint16_t));
  or_dense_rows(x, w, dots, R, K, N);
  for (int r = 0; r < R; ++r)
    for (int n = 0; n < N; ++n) {
      const float v = or_bf16_to_f32(dots[(size_t)r * N + n]);
      float o = v;
      if (epi == 1) {
        o = or_bf16_to_f32(add[(size_t)(r / add_div) * N + n]) + v;
      } else if (epi == 2) {
        const float u = round_bf16(v / (float)hc);
        o = u / (1.0f + or_expf(-u));
      } else if (epi == 3) {
        o = sigmoid_f(v);
      } else if (epi == 4) {
        o = 2.0f * round_bf16(sigmoid_f(round_bf16(v / (float)hc)));
      }
      out[(size_t)r * N + n] = or_f32_to_bf16(o);
    }
  free(dots);
}

/* hc_mix's mean (model/layers.py:195): mixed[s][j] = bf16(sum_{c = 0..hc-1} bf16(m hn) / hc), sum in order. */
void or_hc_mean(const uint16_t* m, const uint16_t* hn, int S, int hc, int H, uint16_t* mixed) {
  for (int s = 0; s < S; ++s)
    for (int j = 0; j < H; ++j) {
      float acc = 0.0f;
      for (int c = 0; c < hc; ++c) {
        const size_t i = (size_t)s * hc * H + (size_t)c * H + j;
        acc += round_bf16(or_bf16_to_f32(m[i]) * or_bf16_to_f32(hn[i]));
      }
      mixed[(size_t)s * H + j] = or_f32_to_bf16(acc / (float)hc);
    }
}

/* HC residual (engine/mtp.py:226): out = bf16(hyp + bf16(y[s][j] inj[s][c])) (out may be hyp). */
void or_hc_inject(const uint16_t* hyp, const uint16_t* y, const uint16_t* inj, int S, int hc, int H, uint16_t* out) {
  for (int s = 0; s < S; ++s)
    for (int c = 0; c < hc; ++c)
      for (int j = 0; j < H; ++j) {
        const size_t i = (size_t)s * hc * H + (size_t)c * H + j;
        const float t = round_bf16(or_bf16_to_f32(y[(size_t)s * H + j]) * or_bf16_to_f32(inj[(size_t)s * hc + c]));
        out[i] = or_f32_to_bf16(or_bf16_to_f32(hyp[i]) + t);
      }
}
