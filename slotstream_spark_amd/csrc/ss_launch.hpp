// Host-side launchers implemented by the kernel translation units and called by the C ABI (ssmoe_capi.hip).
// Every launcher validates nothing: shapes were checked by the caller; each returns hipGetLastError().
#pragma once
#include <hip/hip_runtime.h>

#include <string>
#include <stdint.h>

#include "../../include/ssmoe.h"

namespace ss {

// Launch configuration of one kernel on the current device, worked out once per (device, kernel) and kept per
// device (ss_devcfg.hip): its dynamic LDS limit raised to max_dyn, its static LDS, the CU count, and how many
// workgroups of `threads` threads with max_dyn bytes of dynamic LDS one CU holds at once. A kernel whose workgroups
// wait on each other is launched with one workgroup per CU, and only when per_cu >= 1 at the largest dynamic LDS it
// is ever given: then every workgroup of the grid is resident at once on an otherwise idle device.
struct KernelCfg {
  int threads;
  size_t max_dyn;
  size_t lds_static;
  int cus;
  int per_cu;
};
hipError_t kernel_cfg(const void* kern, int threads, size_t max_dyn, KernelCfg* out);

// One dense bf16 row segment for launch_dense_rows: rows [0, n) of w (bf16 [n, H], row-major) against
// every token; the fp32 dot is rounded once to bf16 and stored at out[t * out_ld + row].
struct DenseSeg {
  const uint16_t* w;
  uint16_t* out;
  int n;
  int out_ld;
};

// Dot products in the defined order (lane l, chunk j: elements 512j + 8l .. +8, fmaf, then the xor butterfly).
hipError_t launch_dense_rows(const uint16_t* x, int T, int H, const DenseSeg* segs, int nseg, hipStream_t st);

// Dense bf16 GEMM c = bf16(a b^T) with MFMA fp32 accumulation (ss_gemm.hip): a [M][lda], b [N][ldb], c [M][ldc].
hipError_t launch_dense_gemm(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, uint16_t* c, int64_t ldc,
                             int M, int N, int K, hipStream_t st);

// Router tail for T tokens: scores = bf16 logits (+ bias), fp32 softmax, top-k (ties -> lower index,
// sorted by value desc), renormalised weights. probs may be null.
hipError_t launch_router_topk(const uint16_t* logits, const float* bias, float* probs, int32_t* ids, float* weights,
                              int T, int E, int K, hipStream_t st);

// Shared-expert elementwise chain (ss_router.hip): hs = bf16(bf16(silu(g)) * u) and the shared_expert_gate logit from
// one [T, ld] bf16 projection (g at columns [0, Is), u at [Is, 2 Is), the gate logit at 2 Is); and
// y = bf16(bf16(routed) + bf16(bf16(sigmoid(sgl)) * sh)).
hipError_t launch_shared_hs(const uint16_t* proj, int64_t ld, int T, int Is, uint16_t* hs, uint16_t* sgl,
                            hipStream_t st);
hipError_t launch_residual_rmsnorm(const uint16_t* resid, const uint16_t* y, const uint16_t* w, float eps, int R,
                                   int H, uint16_t* stream_out, uint16_t* mixed, hipStream_t st);
hipError_t launch_combine_shared(const float* routed, const uint16_t* sh, const uint16_t* sgl, uint16_t* y, int T,
                                 int H, hipStream_t st);

// topk_stable over fp32 rows (kernels/topk_stable.py:85-113 semantics).
hipError_t launch_topk_stable(const float* scores, const int32_t* n_valid, int32_t* idx, float* val, int R, int N,
                              int k, hipStream_t st);

// One persistent launch per block of <= 4 tokens: (verify mode) router + shared expert + routed experts +
// combine, or (decode mode) the routed experts of given ids. See ss_verify.hip.
struct VerifyArgs {
  int mode;                 // 0 = verify layer (router on device, shared expert, y); 1 = moe_decode (ids given)
  const void* x;            // [T, H] bf16, or fp32 when x_f32 (decode mode only)
  int x_f32;
  const uint16_t* router_w; // [E, H]
  const float* bias;        // [E] or null
  const uint16_t* sh_gate;  // [Is, H]
  const uint16_t* sh_up;    // [Is, H]
  const uint16_t* sh_down;  // [H, Is]
  const uint16_t* sh_g;     // [1, H]
  // Affine 4-bit (gs 64) shared expert: with sh_gs non-null, sh_gate / sh_up / sh_down hold packed words (uint32
  // [Is, H/8], [Is, H/8], [H, Is/8]) and these their bf16 scales and biases ([Is, H/64] twice, [H, Is/64]).
  const uint16_t *sh_gs, *sh_gb, *sh_us, *sh_ub, *sh_ds, *sh_db;
  const int32_t* map;
  int64_t map_len;
  const int64_t* slot_ptr;
  int64_t n_slots;
  int64_t map_base;         // layer * E
  const int32_t* ids_in;    // decode mode: [T, K]
  const float* w_in;        // decode mode: [T, K]
  int32_t* ids_out;         // verify mode: [T, K]
  float* w_out;             // verify mode: [T, K]
  uint16_t* y;              // verify mode: [T, H]
  float* out;               // [T, H] routed rank-order sum (decode: required; verify: optional)
  float* h_buf;             // [T, K, I] fp32 or null
  float* o_buf;             // [T, K, H] fp32 or null
  void* scratch;            // verify_scratch_bytes(), counters zero on entry (the kernel leaves them zero)
  int T, H, I, Is, K, E;
  int* err;
  uint64_t* trace;          // null, or [grid][16] phase timestamps (s_memrealtime, 100 MHz)
  // Chained layers (verify mode, bf16 x): with norm_in, x is the residual stream and the layer runs on
  // bf16((x * r) * norm_w), r = 1 / sqrt(sum(x^2) / H + norm_eps) (the order of ssmoe_residual_rmsnorm; norm_w null =
  // ones); with x_plus_y the combine also writes bf16(x + y) [T, H] there.
  int norm_in;
  const uint16_t* norm_w;
  float norm_eps;
  uint16_t* x_plus_y;
};
size_t verify_scratch_bytes(int T, int H, int I, int Is, int K, int E);
hipError_t launch_verify(const VerifyArgs& a, hipStream_t st);
// The affine 4-bit shared-expert instantiations (ss_verify_q4.hip); launch_verify calls it when sh_gs is set.
hipError_t launch_verify_q4(const VerifyArgs& a, hipStream_t st);
// Zeroes `bytes` (a multiple of 16) at the 16-byte aligned `p` with vector stores (a kernel, so that it can sit in a
// captured graph where a memset node could not).
hipError_t launch_zero16(void* p, size_t bytes, hipStream_t st);

// A chain of verify-mode layers in one persistent launch (ss_chain.hip). Layer 0 comes by value; layers 1 ..
// NL-1 from `more` (device memory, ssmoe_chain_layer entries).
struct ChainArgs {
  const uint16_t* stream_in;     // [T, H] bf16: layer 0's input (norm_in: its residual stream)
  int norm_in;                   // 1: layer 0 runs on bf16(rmsnorm(stream_in) * norm_w); 0: on stream_in itself
  float eps;
  ssmoe_chain_layer l0;
  const ssmoe_chain_layer* more;  // [NL - 1]
  int NL;
  const int32_t* map;
  int64_t map_len;
  const int64_t* slot_ptr;
  int64_t n_slots;
  void* scratch;                 // chain_scratch_bytes(), counters zero on entry (the kernel leaves them zero)
  int T, H, I, Is, K, E;
  int* err;
  uint64_t* trace;               // null, or [grid][16] phase timestamps of the last layer
};
size_t chain_scratch_bytes(int T, int H, int I, int Is, int K, int E);
bool chain_shape_supported(int H, int I);
const char* chain_shapes_text();  // the supported shapes, for error messages
hipError_t launch_chain(const ChainArgs& a, hipStream_t st);

// Prefill (ss_prefill.hip).
struct AlignArgs {
  const int32_t* local_expert;  // [R]: local expert of each row, outside [0, num_local) = skipped
  int64_t R;
  int num_local, block_m;
  int32_t* sorted_rows;   // [padded_rows(R, num_local, block_m)]
  int32_t* block_expert;  // [padded / block_m]
  int32_t* num_padded;    // [1]
  int32_t* scratch;       // align_scratch_ints(R, num_local) ints
};
int64_t padded_rows(int64_t R, int num_local, int block_m);
int64_t align_scratch_ints(int64_t R, int num_local);
hipError_t launch_moe_align(const AlignArgs& a, hipStream_t st);

constexpr int kPrefillBlockM = 128;  // the moe_align block the grouped GEMM consumes
struct PrefillArgs {
  const uint16_t* x;            // bf16 [T, H]
  const int32_t* row_token;     // [R]
  const float* row_weight;      // [R]
  const int32_t* sorted_rows;   // moe_align plan with block_m = kPrefillBlockM
  const int32_t* block_expert;
  const int32_t* num_padded;
  const int64_t* group_ptr;     // [num_local] record base addresses
  int num_local;
  uint16_t* h_buf;              // bf16 [R, I]
  float* out_rows;              // fp32 [R, H]
  int64_t R;
  int T, H, I;                  // T: rows of x (a row_token outside [0, T) reads zeros)
  uint64_t* trace = nullptr;    // diagnostics: per-block stamps of the two GEMMs (16384 entries), or null
};
hipError_t launch_prefill_gemm(const PrefillArgs& p, hipStream_t st);
// out[t] = sum over k (in order) of rows[t * K + k]; a row whose row_local entry is negative counts as +0.
hipError_t launch_combine(const float* rows, const int32_t* row_local, int T, int K, int H, float* out,
                          hipStream_t st);
// Resident-pool tables of a prefill: group_ptr[e] from map/slot_ptr, local[r] = ids[r] (or -1, raising a status
// bit, when the expert is out of range or not resident), row_token[r] = r / K.
hipError_t launch_prefill_tables(const int32_t* map, int64_t map_base, int64_t map_len, const int64_t* slot_ptr,
                                 int64_t n_slots, int E, int64_t* gptr, const int32_t* ids, int64_t R, int K,
                                 int32_t* local, int32_t* row_token, int* err, hipStream_t st);

// Reference sampler (ss_sampler.hip): Sampler.next over one row with sanitized parameters; u a device float.
int64_t sample_workspace_bytes(int V);
hipError_t launch_sample(const float* x, int V, const int32_t* gen, int n_gen, float temperature, float top_p,
                         int top_k, float min_p, float pp, const float* u, void* work, int32_t* out, hipStream_t st);
// The proposal draw of the p/q round (ss_accept.hip): tokens[r] ~ softmax(x[r] / temperature) with u[r], R rows in
// as few persistent launches as a resident grid allows; the workspace holds draw_work_floats(R, V) floats, zeroed
// before its first use.
int64_t draw_work_floats(int R, int V);
hipError_t launch_draw_rows(const float* x, int R, int V, float temperature, const float* u, void* work,
                            int32_t* tokens, int* err, hipStream_t st);
hipError_t launch_accept_sampled(const float* target, const int32_t* drafts, int D, int V, const int32_t* seen,
                                 int n_seen, float temperature, float top_p, int top_k, float min_p, float pp,
                                 const float* uniforms, void* work, int32_t* out, hipStream_t st);

// Achievable-peak kernels (ss_peaks.hip).
hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* out, int grid, hipStream_t st);
hipError_t launch_mfma_loop(const uint32_t* seed, int iters, float* out, int grid, hipStream_t st);
hipError_t launch_bf16_round(const float* x, uint16_t* y, int64_t n, hipStream_t st);

// Expert slot pool (ss_pool.hip).
struct Pool;
enum class PoolStatus { Ok, Invalid, Exhausted, Io };
struct EnsureTiming {
  int64_t hits, misses, bytes, total_ns, read_ns, copy_ns;
};
struct PoolStats {
  int64_t slots, chunks, pinned, owned_bytes, stride, hits, misses, bytes, lanes, direct;
};
hipError_t pool_open(const char* path, int layers, int experts, int64_t record_bytes, int max_slots,
                     int64_t chunk_bytes, int32_t* map_dev, int64_t* ptr_dev, Pool** out, std::string* err);
void pool_close(Pool* p);
hipError_t pool_set_reader(Pool* p, int lanes, bool direct, std::string* err);
hipError_t pool_resize(Pool* p, int n, std::string* err);
void pool_retire_below(Pool* p, uint64_t progress);
PoolStatus pool_ensure(Pool* p, int layer, const int32_t* experts, int n, uint64_t gen, int32_t* out,
                       EnsureTiming* t, std::string* err);
void pool_info(Pool* p, PoolStats* s);
void pool_set_progress(Pool* p, const uint64_t* progress);
hipError_t pool_copy_slot(Pool* p, int slot, void* dst, int64_t bytes, std::string* err);

// Affine 4-bit GEMV (ss_gemv.hip).
bool gemv_affine4_shape_ok(int K);
hipError_t launch_gemv_affine4(const void* x, int x_f32, int R, int K, const int32_t* q, const uint16_t* s,
                               const uint16_t* b, int N, float* y, hipStream_t st);
int64_t lm_head_greedy_workspace_bytes(int D, int N);
hipError_t launch_lm_head_greedy(const void* x, int x_f32, int D, int K, const int32_t* q, const uint16_t* s,
                                 const uint16_t* b, int N, const int32_t* drafts, void* work, float* logits,
                                 int32_t* out, hipStream_t st);
// The lm_head GEMV over the D + 1 verify rows with the p/q round behind it: the GEMV writes the logits (lin's
// values) and each row's chunk maxima, then the p/q launches (ss_accept.hip) read the logits once for the sums.
int64_t lm_head_pq_workspace_bytes(int D, int N);
hipError_t launch_lm_head_pq(const void* x, int x_f32, int D, int K, const int32_t* q, const uint16_t* s,
                             const uint16_t* b, int N, const float* draft, const int32_t* drafts, const float* uniforms,
                             float temperature, void* work, float* logits, int32_t* out, int* err, hipStream_t st);
// Argmax ids of R rows (R <= 64; workspace lm_head_greedy_workspace_bytes(R - 1, N)).
hipError_t launch_lm_head_argmax(const void* x, int x_f32, int R, int K, const int32_t* q, const uint16_t* s,
                                 const uint16_t* b, int N, int round_bf16, void* work, float* logits, int32_t* ids,
                                 hipStream_t st);

// MTP head dense ops (ss_head.hip), as ssmoe_rmsnorm / ssmoe_dense_gemv_epi / ssmoe_hc_mean / ssmoe_hc_inject /
// ssmoe_gather_rows.
hipError_t launch_rmsnorm_groups(const uint16_t* x, const uint16_t* w, float eps, int R, int n, int G, uint16_t* out,
                                 hipStream_t st);
hipError_t launch_dense_epi(const uint16_t* x, int R, int K, const uint16_t* w, int N, int epi, int hc,
                            const uint16_t* add, int add_div, uint16_t* out, hipStream_t st);
// The fused head GEMV (ss_head.hip): source rows (or table rows by device index), optional hc_inject and RMSNorm,
// then the GEMV with one or two weight ranges, or the GEMV with the branch mean fused behind it. Fields as the C
// entry point ssmoe_head_gemv; mean_H = N / 4 in mean mode.
struct HeadGemvIn {
  const uint16_t* src;
  const int32_t* src_idx;
  int64_t n_src;
  const uint16_t* inj_y;
  const uint16_t* inj;
  int inj_hc;
  const uint16_t* norm_w;
  float eps;
  int G;
  int S, n, K;
  const uint16_t* w;
  int N, epi, hc;
  const uint16_t* add;
  int add_div;
  uint16_t* out;
  const uint16_t* w2;
  int N2, epi2;
  uint16_t* out2;
  uint16_t* h_out;
  uint16_t* x_out;
  const uint16_t* mean_hn;
  uint16_t* mean_out;
  int mean_H;
  int* err;
  uint64_t* trace;
};
hipError_t launch_head_gemv(const HeadGemvIn& in, hipStream_t st);
hipError_t launch_hc_mean(const uint16_t* m, const uint16_t* hn, int S, int hc, int H, uint16_t* mixed,
                          hipStream_t st);
hipError_t launch_hc_inject(const uint16_t* hyp, const uint16_t* y, const uint16_t* inj, int S, int hc, int H,
                            uint16_t* out, hipStream_t st);
hipError_t launch_gather_rows(const void* src, int64_t n_src, int64_t row_bytes, const int32_t* idx, int n,
                              int idx_add, void* dst, int* err, hipStream_t st);

// Acceptance.
struct AcceptArgs {
  const float* target;   // [D+1, V]
  const float* draft;    // [D, V] (p/q only)
  const int32_t* drafts; // [D]
  const float* uniforms; // [D+1] (p/q only)
  int D, V;
  float temperature;
  int32_t* out;          // [D + 5]: n_accept, n_emit, n_uniform, flags, tokens[D+1]
  float* work;           // workspace floats
  int* err;
  uint64_t* trace;       // diagnostics: per-workgroup phase stamps of the one-launch p/q round, or null
};
int64_t accept_work_floats(int D, int V);
hipError_t launch_accept_greedy(const AcceptArgs& a, hipStream_t st);
hipError_t launch_accept_pq(const AcceptArgs& a, hipStream_t st);

}  // namespace ss
