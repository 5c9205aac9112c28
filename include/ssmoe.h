/* C ABI of the MI355X (gfx950) MTP-verify MoE path: libssmoe.so.
 *
 * Every pointer argument is a device pointer unless stated otherwise; `stream` is a hipStream_t (NULL = the
 * legacy default stream). No entry point allocates device memory, synchronises the host, or uses atomics in a
 * floating-point reduction; every call is capturable in a HIP graph. Each returns 0 on success or a nonzero
 * status whose text is given by ssmoe_last_error() (argument errors: SSMOE_EINVAL; launch errors: SSMOE_EHIP).
 * Reference files are cited as path:line in fortil/slotstream-spark.
 */
#ifndef SSMOE_H
#define SSMOE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SSMOE_OK 0
#define SSMOE_EINVAL 1
#define SSMOE_EHIP 2
#define SSMOE_EXHAUSTED 3 /* the pool has too few unpinned slots (slotio::Exhausted); nothing changed */
#define SSMOE_EIO 4       /* a record could not be read (slotio::IoError); nothing published */

/* Device status bits raised by kernels on bad input (the kernel skips the entry and continues). */
#define SSMOE_ERR_EXPERT_ID 1 /* expert id outside [0, E) */
#define SSMOE_ERR_SLOT 2      /* map entry outside [0, n_slots): expert not resident */
#define SSMOE_ERR_TOKEN 4     /* draft token outside [0, V) */
#define SSMOE_ERR_NONFINITE 8 /* non-finite logits reached a p/q decision */
#define SSMOE_ERR_TIMEOUT 16  /* a persistent launch's bounded wait (2^22 polls) for another workgroup ran out: its
                               * workgroups were not all resident at once, e.g. because a kernel on another stream
                               * held CUs. The launch still finishes; its outputs are not valid. */

/* Text of the last error on this host thread ("" if none). */
const char* ssmoe_last_error(void);

/* ABI version (incremented on any signature change). */
int ssmoe_version(void);

/* Reads the status word of the current device into *flags (a host pointer) and clears it when clear != 0.
 * Synchronises the device. No reference counterpart: the reference kernels do not check ids. */
int ssmoe_device_error(int* flags, int clear);

/* Diagnostics (no reference counterpart): when buf (device memory, >= 16384 uint64) is non-null, every later
 * persistent MoE launch (ssmoe_moe_decode, ssmoe_moe_verify_layer) writes per-workgroup phase timestamps
 * (s_memrealtime, 100 MHz) to buf[workgroup * 16 + phase]; a chain launch (ssmoe_moe_verify_chain) writes its last
 * layer there, the layer before at row 512 + workgroup, and a few more stamps of each at rows 256 + and 768 +
 * workgroup. The prefill grouped GEMM pair (ssmoe_fused_moe_affine, ssmoe_moe_prefill) writes four entries per
 * block: start and end stamps, expert << 32 | valid rows, XCC_ID << 32 | HW_ID; gate/up blocks at
 * buf[4 * block], down blocks at buf[8192 + 4 * block] (blocks past 2048 per kernel are not recorded). The one-launch
 * p/q round (ssmoe_accept_pq) writes 16 stamps per workgroup at buf[workgroup * 16 + k]. NULL switches
 * it off. Process-wide, not thread-safe; a launch captured in a graph keeps the setting of its capture. */
int ssmoe_set_trace(void* buf, int64_t entries);

/* Byte offsets of the nine pieces of one affine-4bit expert record (gate.w gate.s gate.b up.w up.s up.b
 * down.w down.s down.b) followed by the record size, written to off[10] (host pointer).
 * Replaces the constants of kernels/moe_gemv_affine.py:22-25 (RECORD_BYTES, O_*), parametrised by (H, I). */
int ssmoe_record_layout(int H, int I, int64_t* off);

/* Routed experts of one decode/verify step, router-free.
 * Replaces moe_decode (kernels/moe_gemv_affine.py:113-147; kernels _gate_up :56-77, _down :80-97,
 * _rank_sum :100-110). x: [R, H] bf16 (x_is_f32 = 0) or fp32 (1); expert_ids int32 [R, K]; weights fp32 [R, K];
 * the record of expert e is at slot_ptr[map[layer * E + e]] (map int32 [map_len], slot_ptr int64 [n_slots]).
 * Writes h_buf fp32 [R, K, I], o_buf fp32 [R, K, H] (o = (Wd h) * w), out fp32 [R, H] (rank-order sum).
 * Constraints: H % 128 == 0, H <= 4096, I % 128 == 0, I <= 1024, 1 <= K <= 16.
 * Takes no workspace (as the reference's): the library's static scratch has one slot per stream for the first 8
 * streams that call it on a device, so calls on different streams may overlap; a ninth stream shares a slot. */
int ssmoe_moe_decode(const void* x, int x_is_f32, const int32_t* expert_ids, const float* weights, int layer,
                     const int32_t* map, int64_t map_len, const int64_t* slot_ptr, int64_t n_slots, float* h_buf,
                     float* o_buf, float* out, int R, int H, int I, int K, int E, void* stream);

/* Stable top-k per row. Replaces topk_stable (kernels/topk_stable.py:85-113, kernel :29-82).
 * scores fp32 [R, N], N <= 65536; n_valid int32 [R] or NULL; out_idx int32 [R, k]; out_val fp32 [R, k] or NULL.
 * k <= 16: sorted by (value desc, index asc); larger k: by index asc; short rows padded with -1 / -inf. */
int ssmoe_topk_stable(const float* scores, const int32_t* n_valid, int32_t* out_idx, float* out_val, int R, int N,
                      int k, void* stream);

/* Dense bf16 projection out[t, n] = bf16(sum_k x[t, k] w[n, k]) with fp32 accumulation in a fixed order.
 * Replaces lin() on bf16 weights (model/layers.py:62-76 -> kernels/gemv_affine.py:214-262 dense path).
 * x bf16 [T, H], w bf16 [N, H], out bf16 [T, N]; H % 8 == 0, H <= 8192. */
int ssmoe_dense_gemv_bf16(const uint16_t* x, const uint16_t* w, uint16_t* out, int T, int H, int N, void* stream);

/* lin on a bf16 weight over many rows (model/layers.py:62-76 inside prefill_gemm(), the dense case of
 * kernels/gemm_affine.py:20-98): c = bf16(a w^T), a bf16 [M][lda], w bf16 [N][ldw], c bf16 [M][ldc], the dot over
 * K accumulated in fp32 by the bf16 MFMA unit and rounded once. The prefill's router logits and shared-expert
 * projections. K a multiple of 256; lda, ldw >= K and ldc >= N, all multiples of 8; a, w, c 16-byte aligned.
 * Row m of c depends on row m of a only. */
int ssmoe_dense_gemm(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, uint16_t* c, int64_t ldc, int M,
                     int N, int K, void* stream);

/* Router: logits = bf16(x router_w^T), scores = logits (+ bias), probs = softmax(scores) in fp32, top-k with
 * ties to the lower index, weights = topk / sum(topk) in rank order.
 * Replaces Segments.seg_router (model/layers.py:336-348) and reference_torch.moe_ref:121-124. bias fp32 [E] or
 * NULL (the reference has no bias); logits bf16 [T, E] (required, scratch or output); probs fp32 [T, E] or NULL;
 * ids int32 [T, K]; weights fp32 [T, K]. E <= 8192, K <= 16. */
int ssmoe_router(const uint16_t* x, const uint16_t* router_w, const float* bias, uint16_t* logits, float* probs,
                 int32_t* ids, float* weights, int T, int H, int E, int K, void* stream);

/* The routing half of ssmoe_router from given bf16 logits [T, E] (prefill computes the logits with a GEMM):
 * scores = logits (+ bias), fp32 softmax, top-k with ties to the lower index, renormalised weights.
 * Replaces the softmax / topk_stable / renorm of Segments.seg_router (model/layers.py:340-347). */
int ssmoe_router_topk(const uint16_t* logits, const float* bias, float* probs, int32_t* ids, float* weights, int T,
                      int E, int K, void* stream);

/* Bytes of the workspace ssmoe_moe_verify_layer needs for T tokens. */
int64_t ssmoe_verify_workspace_bytes(int T, int H, int I, int Is, int K, int E);

/* One MoE layer of the verify step: router (as ssmoe_router) -> routed experts (as ssmoe_moe_decode) ->
 * shared expert with its sigmoid gate -> y = bf16(routed) + shared, in bf16.
 * Replaces GraphSet._moe + Segments.seg_router (runtime/graphs.py:160-169, model/layers.py:336-402) and
 * reference_torch.moe_ref (:118-134). x bf16 [T, H]; router_w bf16 [E, H]; router_bias fp32 [E] or NULL;
 * sh_gate, sh_up bf16 [Is, H]; sh_down bf16 [H, Is]; sh_g bf16 [1, H]; workspace of
 * ssmoe_verify_workspace_bytes() bytes (256-byte aligned); outputs ids int32 [T, K], weights fp32 [T, K],
 * y bf16 [T, H], routed_out fp32 [T, H] or NULL. */
int ssmoe_moe_verify_layer(const uint16_t* x, const uint16_t* router_w, const float* router_bias,
                           const uint16_t* sh_gate, const uint16_t* sh_up, const uint16_t* sh_down,
                           const uint16_t* sh_g, int layer, const int32_t* map, int64_t map_len,
                           const int64_t* slot_ptr, int64_t n_slots, void* workspace, int64_t workspace_bytes,
                           int32_t* ids, float* weights, uint16_t* y, float* routed_out, int T, int H, int I, int Is,
                           int K, int E, void* stream);

/* One layer of a chain of MoE layers: the layer of ssmoe_moe_verify_layer run on
 * x = bf16(rmsnorm(stream_in) * norm_w) (exactly ssmoe_residual_rmsnorm with y NULL; norm_w NULL = ones), and, when
 * stream_out is non-null, stream_out = bf16(stream_in + y), the residual stream of the next layer. The norm of the next
 * seg_router and the residual add of GraphSet._moe (runtime/graphs.py:169, one stream, unit injection) folded into
 * the verify launch, so a chain needs no launch between layers. H a multiple of 512; stream_out must not alias
 * stream_in or y. */
int ssmoe_moe_verify_layer_chain(const uint16_t* stream_in, const uint16_t* norm_w, float eps,
                                 const uint16_t* router_w, const float* router_bias, const uint16_t* sh_gate,
                                 const uint16_t* sh_up, const uint16_t* sh_down, const uint16_t* sh_g, int layer,
                                 const int32_t* map, int64_t map_len, const int64_t* slot_ptr, int64_t n_slots,
                                 void* workspace, int64_t workspace_bytes, int32_t* ids, float* weights, uint16_t* y,
                                 uint16_t* stream_out, float* routed_out, int T, int H, int I, int Is, int K, int E,
                                 void* stream);

/* The scales and biases of an affine 4-bit (gs 64) shared expert (the checkpoint's quantized
 * shared_expert.{gate,up,down}_proj, AffineWeight of model/weights.py:84-92, applied by lin -> gemv,
 * model/layers.py:62-76): bf16 [Is, H/64] (gate, up) and [H, Is/64] (down), device pointers. With them the
 * entry points below take sh_gate, sh_up and sh_down as packed words, uint32 [Is, H/8], [Is, H/8] and [H, Is/8]
 * (nibble i of a word at bits 4i), and form each projection as the or_dense_rows order over weights dequantized in
 * fp32 (q * s, then + b); the shared_expert_gate row sh_g stays bf16. H and Is multiples of 64. */
typedef struct {
  const uint16_t* gate_s;
  const uint16_t* gate_b;
  const uint16_t* up_s;
  const uint16_t* up_b;
  const uint16_t* down_s;
  const uint16_t* down_b;
} ssmoe_shared_q4;

/* ssmoe_moe_verify_layer with an affine 4-bit shared expert (sh_q4 non-null, see ssmoe_shared_q4). */
int ssmoe_moe_verify_layer_q4s(const uint16_t* x, const uint16_t* router_w, const float* router_bias,
                               const uint16_t* sh_gate, const uint16_t* sh_up, const uint16_t* sh_down,
                               const uint16_t* sh_g, const ssmoe_shared_q4* sh_q4, int layer, const int32_t* map,
                               int64_t map_len, const int64_t* slot_ptr, int64_t n_slots, void* workspace,
                               int64_t workspace_bytes, int32_t* ids, float* weights, uint16_t* y, float* routed_out,
                               int T, int H, int I, int Is, int K, int E, void* stream);

/* ssmoe_moe_verify_layer_chain with an affine 4-bit shared expert (sh_q4 non-null, see ssmoe_shared_q4). */
int ssmoe_moe_verify_layer_chain_q4s(const uint16_t* stream_in, const uint16_t* norm_w, float eps,
                                     const uint16_t* router_w, const float* router_bias, const uint16_t* sh_gate,
                                     const uint16_t* sh_up, const uint16_t* sh_down, const uint16_t* sh_g,
                                     const ssmoe_shared_q4* sh_q4, int layer, const int32_t* map, int64_t map_len,
                                     const int64_t* slot_ptr, int64_t n_slots, void* workspace,
                                     int64_t workspace_bytes, int32_t* ids, float* weights, uint16_t* y,
                                     uint16_t* stream_out, float* routed_out, int T, int H, int I, int Is, int K,
                                     int E, void* stream);

/* One layer of ssmoe_moe_verify_chain: its weights, its map row and its outputs (device pointers). */
typedef struct {
  const uint16_t* router_w;  /* bf16 [E, H] */
  const float* router_bias;  /* fp32 [E] or NULL */
  const uint16_t* sh_gate;   /* bf16 [Is, H] */
  const uint16_t* sh_up;     /* bf16 [Is, H] */
  const uint16_t* sh_down;   /* bf16 [H, Is] */
  const uint16_t* sh_g;      /* bf16 [1, H] */
  const uint16_t* norm_w;    /* bf16 [H] or NULL (ones): the RMSNorm weight before the layer */
  int64_t layer;             /* the layer's experts are at slot_ptr[map[layer * E + e]] */
  int32_t* ids;              /* int32 [T, K] */
  float* weights;            /* fp32 [T, K] */
  uint16_t* y;               /* bf16 [T, H] */
  uint16_t* stream_out;      /* bf16 [T, H] or NULL: bf16(stream + y), the next layer's residual stream */
  float* routed_out;         /* fp32 [T, H] or NULL */
  /* Affine 4-bit (gs 64) shared expert (the checkpoint's quantized shared_expert.{gate,up,down}_proj, AffineWeight
   * of model/weights.py:84-92): all six NULL for bf16 weights; all six set and sh_gate / sh_up / sh_down then hold
   * packed words, uint32 [Is, H/8], [Is, H/8], [H, Is/8] (nibble i of a word at bits 4i). bf16 scales and biases: */
  const uint16_t* sh_gate_s; /* [Is, H/64] */
  const uint16_t* sh_gate_b;
  const uint16_t* sh_up_s;   /* [Is, H/64] */
  const uint16_t* sh_up_b;
  const uint16_t* sh_down_s; /* [H, Is/64] */
  const uint16_t* sh_down_b;
} ssmoe_chain_layer;

/* Bytes of the workspace ssmoe_moe_verify_chain needs (-1 on bad arguments). */
int64_t ssmoe_verify_chain_workspace_bytes(int T, int H, int I, int Is, int K, int E);

/* n_layers chained MoE layers of a verify step in one launch: layer l runs the layer of ssmoe_moe_verify_layer on
 * x_l = bf16(rmsnorm(s_l) * norm_w_l), s_0 = stream_in, s_{l+1} = bf16(s_l + y_l) (the residual add of GraphSet._moe,
 * runtime/graphs.py:160-169, with one stream and unit injection; rmsnorm as ssmoe_residual_rmsnorm). The same bits
 * as n_layers calls of ssmoe_moe_verify_layer_chain; the next layer's router, shared-expert and table reads are issued
 * during the current layer, and the stream passes between layers on the device without a launch.
 * layers_host (host memory) and layers_dev (device memory) hold the same n_layers entries: the host copy is checked
 * and supplies layer 0, the kernel reads the others from the device copy. 1 <= n_layers <= 4096; (H, I) = (2048,
 * 512), the BASELINE layer, or (2560, 640), the reference model's (other shapes: SSMOE_EINVAL; run them as
 * ssmoe_moe_verify_layer_chain launches); E + Is >= 4 * (compute units), so that every wave has a router or shared
 * row in each layer, and H / 16 < (compute units), so that some workgroups have no output rows and form the shared
 * expert's rows. The shared expert is bf16 or affine 4-bit (the sh_*_s / sh_*_b fields), the same in every layer. */
int ssmoe_moe_verify_chain(const uint16_t* stream_in, float eps, const ssmoe_chain_layer* layers_host,
                           const ssmoe_chain_layer* layers_dev, int n_layers, const int32_t* map, int64_t map_len,
                           const int64_t* slot_ptr, int64_t n_slots, void* workspace, int64_t workspace_bytes, int T,
                           int H, int I, int Is, int K, int E, void* stream);

/* ssmoe_moe_verify_layer without the workspace: the same arguments, outputs and bits, with the scratch in a static
 * device array of the library (192 KiB per GPU, held until the process ends; shapes needing more, i.e. beyond
 * I * K <= 8192, are refused with SSMOE_EINVAL). It allocates nothing. No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU race, so issue them on one stream. The
 * first call on a device clears the array with a kernel on `stream` (make that first call outside a capture). */
int ssmoe_moe_verify_layer_noalloc(const uint16_t* x, const uint16_t* router_w, const float* router_bias,
                                   const uint16_t* sh_gate, const uint16_t* sh_up, const uint16_t* sh_down,
                                   const uint16_t* sh_g, int layer, const int32_t* map, int64_t map_len,
                                   const int64_t* slot_ptr, int64_t n_slots, int32_t* ids, float* weights,
                                   uint16_t* y, float* routed_out, int T, int H, int I, int Is, int K, int E,
                                   void* stream);

/* Bytes of the workspace the acceptance entry points need (1 <= V <= 1,048,576, 0 <= D <= 60). Its first 16384
 * bytes hold cross-workgroup arrival counters: they must be zero before the first call (allocate
 * the workspace zeroed), and every call leaves them zero. Calls that share a workspace must not overlap. */
int64_t ssmoe_accept_workspace_bytes(int D, int V);

/* Greedy verify acceptance. Replaces the acceptance loop of _mtp_decode (engine/generate.py:208-229) with
 * Sampler.next at temperature 0 (engine/sampler.py:83-84, np.argmax: first maximum).
 * target fp32 [D+1, V]; drafts int32 [D]; out int32 [D+5]: n_accept, n_emit, n_uniform (0), flags
 * (1 = stopped at a non-finite row), tokens[D+1] (emitted tokens, -1 after the last). */
int ssmoe_accept_greedy(const float* target, const int32_t* drafts, int D, int V, void* workspace,
                        int64_t workspace_bytes, int32_t* out, void* stream);

/* p/q speculative acceptance (Leviathan et al. 2023, Alg. 1). No reference counterpart: the reference samples
 * each verify row with Sampler.next and compares (engine/generate.py:208-229); this entry point is the
 * rejection-sampling verify the BASELINE asks for. target fp32 [D+1, V]; draft fp32 [D, V]; drafts int32 [D];
 * uniforms fp32 [D+1] in [0, 1) (decision i uses uniforms[i], the final sample the next unused one);
 * out int32 [D+5] as for ssmoe_accept_greedy (n_uniform = uniforms consumed; flags 1 = non-finite,
 * 2 = draft token out of range, 4 = empty residual). */
int ssmoe_accept_pq(const float* target, const float* draft, const int32_t* drafts, const float* uniforms, int D,
                    int V, float temperature, void* workspace, int64_t workspace_bytes, int32_t* out,
                    void* stream);

/* ---------------------------------------------------------------- prefill */

/* Padded length of a moe_align plan: R + num_local * (block_m - 1), rounded up to a multiple of block_m.
 * Replaces padded_rows (kernels/moe_align.py:11-14). Returns -1 on bad arguments. */
int64_t ssmoe_padded_rows(int64_t R, int num_local, int block_m);

/* Bytes of the scratch ssmoe_moe_align needs. */
int64_t ssmoe_moe_align_workspace_bytes(int64_t R, int num_local);

/* Stable counting sort of rows by local expert. Replaces moe_align (kernels/moe_align.py:17-48).
 * local_expert int32 [R] (outside [0, num_local) = row skipped); outputs sorted_rows int32 [padded] (row ids,
 * sentinel R in the padding), block_expert int32 [padded / block_m] (expert of each block, -1 past num_padded),
 * num_padded int32 [1]. Deterministic: no order-dependent atomics. */
int ssmoe_moe_align(const int32_t* local_expert, int64_t R, int num_local, int block_m, void* workspace,
                    int64_t workspace_bytes, int32_t* sorted_rows, int32_t* block_expert, int32_t* num_padded,
                    void* stream);

/* Grouped affine-4bit MoE over an aligned plan (block_m = 128): h = bf16(silu(x Wg^T) * (x Wu^T)) with weights
 * dequantized to bf16(q*s + b), bf16 MFMA and fp32 accumulation, then out_rows = (h Wd^T) * row_weight in fp32.
 * Replaces fused_moe_affine's two launches (kernels/fused_moe_affine.py:136-161, kernels :39-108).
 * x bf16 [T, H]; row_token int32 [R] (a token outside [0, T) reads as a zero row); row_weight fp32 [R];
 * group_ptr int64 [num_local] record bases; h_buf bf16
 * [R, I]; out_rows fp32 [R, H] (rows outside the plan are not written). H % 256 == 0, I % 128 == 0, H, I <= 4096. */
int ssmoe_fused_moe_affine(const uint16_t* x, const int32_t* row_token, const float* row_weight,
                           const int32_t* sorted_rows, const int32_t* block_expert, const int32_t* num_padded,
                           const int64_t* group_ptr, int num_local, uint16_t* h_buf, float* out_rows, int64_t R,
                           int T, int H, int I, void* stream);

/* out[t] = ((rows[t*K] + rows[t*K+1]) + ...) + rows[t*K+K-1], fp32, sequential in router rank order.
 * Replaces combine_rank_order (kernels/fused_moe_affine.py:164-172). */
int ssmoe_combine_rank_order(const float* out_rows, int T, int K, int H, float* out, void* stream);

/* Bytes of the workspace ssmoe_moe_prefill needs. */
int64_t ssmoe_moe_prefill_workspace_bytes(int64_t T, int K, int E);

/* Routed experts of one layer over T prompt tokens with every expert resident: the sweep of SweepMoE.layer
 * (model/moe_sweep.py:80-160, plan_sweep engine/sweep.py:34-58) as one plan over all E experts (no staging
 * groups), i.e. moe_align + ssmoe_fused_moe_affine + ssmoe_combine_rank_order. expert_ids int32 [T, K];
 * weights fp32 [T, K]; records at slot_ptr[map[layer * E + e]]; h_buf bf16 [T*K, I]; out_rows fp32 [T*K, H];
 * out fp32 [T, H]. An expert id outside [0, E) or an unmapped expert raises a status bit and its row counts as 0. */
int ssmoe_moe_prefill(const uint16_t* x, const int32_t* expert_ids, const float* weights, int layer,
                      const int32_t* map, int64_t map_len, const int64_t* slot_ptr, int64_t n_slots, void* workspace,
                      int64_t workspace_bytes, uint16_t* h_buf, float* out_rows, float* out, int64_t T, int H, int I,
                      int K, int E, void* stream);

/* ---------------------------------------------------------------- reference sampler */

/* Bytes of the workspace ssmoe_sample needs for a V-token row (-1 outside 1 <= V <= 1,048,576). */
int64_t ssmoe_sample_workspace_bytes(int V);

/* One draw of the reference sampler. Replaces Sampler.next (engine/sampler.py:76-108) for one row of fp32 logits
 * [V], with the parameters already sanitized (SampleParams.sanitized, :45-64): temperature >= 0 (0: argmax of the
 * penalized logits), top_p in (0, 1], top_k >= 0 (0 or >= V: off), min_p in [0, 1], finite presence_penalty;
 * generated int32 [n_generated] the tokens generated so far, sorted ascending without repeats; u a device pointer to
 * the draw's uniform (float32((state >> 11) / 2^53) of the sampler's splitmix64 stream, :101-102). Writes out int32
 * [2]: the token and flags (1 = the kept mass was not finite and > 0: argmax of the raw logits, :105-106).
 * The reference's float32 operations in its order; the order of each sum is this library's (hierarchical, as the
 * acceptance sums), and exp is this library's. */
int ssmoe_sample(const float* logits, int V, const int32_t* generated, int n_generated, float temperature,
                 float top_p, int top_k, float min_p, float presence_penalty, const float* u, void* workspace,
                 int64_t workspace_bytes, int32_t* out, void* stream);

/* ---------------------------------------------------------------- achievable peaks (measurement only) */

/* No reference counterpart: the ceilings this build's roofline fractions are stated against beside the published
 * MI355X peaks (the method of the reference's micro-benchmarks, bench/m0/gemv_bench.py:228-268). A streaming read of
 * `bytes` (a positive multiple of 16) from src (16-byte aligned) by `grid` 256-thread workgroups with 16-byte loads,
 * folded into out uint32 [grid] (xor; zero it first). */
int ssmoe_bench_stream_read(const void* src, int64_t bytes, uint32_t* out, int grid, void* stream);

/* `grid` workgroups of 4 waves, each wave `iters` rounds of 8 independent v_mfma_f32_16x16x32_bf16 on register
 * operands from seed uint32 [8]: 2 * 16 * 16 * 32 * 8 * iters flop per wave. out fp32 [grid * 4] (the wave sums). */
int ssmoe_bench_mfma_bf16(const uint32_t* seed, int iters, float* out, int grid, void* stream);

/* No reference counterpart: the fp32 -> bf16 rounding every kernel of this library applies (round to nearest even;
 * a NaN keeps its top bits with the quiet bit set: torch's .to(torch.bfloat16) and the reference's weight and
 * activation casts), exported so that it can be checked on any bit pattern. x fp32 [n], y bf16 bits [n]. */
int ssmoe_bf16_round(const float* x, uint16_t* y, int64_t n, void* stream);

/* Bytes of the workspace ssmoe_sample_rows needs (-1 outside 1 <= R <= 64, 1 <= V <= 1,048,576); zero it before
 * its first use (it keeps a launch counter). */
int64_t ssmoe_sample_rows_workspace_bytes(int R, int V);

/* The draft tokens of a p/q round: x_r ~ softmax(logits[r] / temperature) for the R rows of logits fp32 [R, V]
 * with uniforms[r] (tokens int32 [R], on the device), with the p/q round's row statistics (ssmoe_accept_pq's sum
 * order): the chunk by its mass, then the entry inside it; one persistent launch per group of rows whose
 * (row, 1024-entry chunk) units fit a resident grid. A row with a non-finite logit yields an index in [0, V) of no
 * meaning (ssmoe_accept_pq stops at that row). Leviathan et al. 2023 Alg. 1 requires the drafts to be drawn from the
 * same q it divides by; the reference drafts greedily (engine/mtp.py:265-277, torch.argmax), which is the
 * temperature-0 limit and is not a valid proposal for p/q. No reference counterpart. temperature > 0. */
int ssmoe_sample_rows(const float* logits, int R, int V, float temperature, const float* uniforms, void* workspace,
                      int64_t workspace_bytes, int32_t* tokens, void* stream);

/* Bytes of the workspace ssmoe_accept_sampled needs (D+1 rows of ssmoe_sample's; -1 on bad arguments). */
int64_t ssmoe_accept_sampled_workspace_bytes(int D, int V);

/* The sampled verify round. Replaces the acceptance loop of _mtp_decode (engine/generate.py:208-229) at
 * temperature > 0 or with a presence penalty: for row i = 0..D of target fp32 [D+1, V], a row holding a non-finite
 * logit ends the round without a draw (flag 1, :210-212); otherwise the row draws as ssmoe_sample with uniforms[i]
 * and the penalty set seen + the tokens emitted before it (seen.add, :214), and the round goes on while the token
 * equals drafts[i] (i < D). seen int32 [n_seen] sorted ascending without repeats; workspace of
 * ssmoe_accept_sampled_workspace_bytes(D, V) bytes; out int32 [D+5] as ssmoe_accept_greedy (n_accept, n_emit,
 * n_uniform = draws at temperature > 0, flags 1 = non-finite row, 2 = draft out of range, 8 = a draw took the argmax
 * fallback, then the emitted tokens, -1 past n_emit). 0 <= D <= 60. Row i is reached only when rows 0..i-1 drew
 * their drafts, so all rows are drawn at once with penalty set seen + drafts[0..i); the launch sequence depends
 * only on the parameters and can be captured in a graph. */
int ssmoe_accept_sampled(const float* target, const int32_t* drafts, int D, int V, const int32_t* seen, int n_seen,
                         float temperature, float top_p, int top_k, float min_p, float presence_penalty,
                         const float* uniforms, void* workspace, int64_t workspace_bytes, int32_t* out, void* stream);

/* ---------------------------------------------------------------- affine 4-bit GEMV (lm_head) */

/* y = x W^T with W the MLX affine 4-bit weight (q int32 [N][K/8], nibble i of a word at bits 4i; s, b bf16
 * [N][K/64]; w = q s + b), fp32 accumulation. Replaces gemv (kernels/gemv_affine.py:214-262) for
 * AffineWeight(bits=4, gs=64), e.g. the lm_head (248,320 x 2560). x [R][K] bf16 (x_f32 = 0) or fp32 (x_f32 = 1,
 * split into bf16 high part and residual); y fp32 [R][N]. K in {1024, 2048, 2560, 4096}; x and q 16-byte aligned.
 * Row r of y depends on x row r alone: an R-row call equals R one-row calls bit for bit. */
int ssmoe_gemv_affine4(const void* x, int x_f32, int R, int K, const int32_t* q, const uint16_t* s, const uint16_t* b,
                       int N, float* y, void* stream);

/* Bytes of the workspace ssmoe_lm_head_greedy needs (-1 on bad arguments). */
int64_t ssmoe_lm_head_greedy_workspace_bytes(int D, int N);

/* The lm_head GEMV over the D+1 verify rows fused with the greedy round after it (engine/generate.py:208-229 at
 * temperature 0): each 16-row tile of the vocabulary reduces to one argmax key and a non-finite flag per row, so the
 * round reads no logits. The logits are lin's result, lin(final, lm_head).float() (runtime/graphs.py:202): for a bf16
 * x the fp32 dot rounded to bf16, for an fp32 x the dot itself. out int32 [D+5] as ssmoe_accept_greedy (n_accept,
 * n_emit, 0, flags 1 = non-finite row, 2 = draft out of range, tokens). logits fp32 [D+1][N] (those values) is
 * written too when non-null. 0 <= D <= 60. The workspace must be zero before the first call; every call leaves it
 * zero (the GEMV's last workgroup forms the round and clears the keys: one launch per 4 rows, nothing after). */
int ssmoe_lm_head_greedy(const void* x, int x_f32, int D, int K, const int32_t* q, const uint16_t* s,
                         const uint16_t* b, int N, const int32_t* drafts, void* workspace, int64_t workspace_bytes,
                         float* logits, int32_t* out, void* stream);

/* Bytes of the workspace ssmoe_lm_head_pq needs (-1 on bad arguments). */
int64_t ssmoe_lm_head_pq_workspace_bytes(int D, int N);

/* The lm_head GEMV over the D+1 verify rows with the p/q round (as ssmoe_accept_pq) behind it: the GEMV writes the
 * logits (lin's values, as ssmoe_lm_head_greedy) and, per row and 1024-entry vocabulary chunk, the maximum of
 * logit / temperature and a non-finite flag, so the round's maximum pass reads only the draft rows and the logits
 * are read once, for the sums. The same out as ssmoe_accept_pq on those logits, bit for bit. draft fp32 [D][N]
 * (the draft head's logits), drafts int32 [D], uniforms fp32 [D+1], logits fp32 [D+1][N] (written). 0 <= D <= 3;
 * the workspace's first 16 KB must be zero before the first call (every call leaves them zero). */
int ssmoe_lm_head_pq(const void* x, int x_f32, int D, int K, const int32_t* q, const uint16_t* s, const uint16_t* b,
                     int N, const float* draft, const int32_t* drafts, const float* uniforms, float temperature,
                     void* workspace, int64_t workspace_bytes, float* logits, int32_t* out, void* stream);

/* Bytes of the workspace ssmoe_lm_head_argmax needs (-1 on bad arguments). */
int64_t ssmoe_lm_head_argmax_workspace_bytes(int R, int N);

/* The draft token of each row: torch.argmax(lin(out, lm_head).float()) of MTPHead.draft (engine/mtp.py:275-276,
 * logits at engine/mtp.py:232-236). round_bf16 != 0 takes the argmax over the logits rounded to bf16 (lin returns
 * the dtype of x, bf16 for the head); ties and NaN as torch.argmax (the first maximal index; NaN counts as the
 * maximum). ids int32 [R] on the device; logits fp32 [R][N] (the values ranked) is written too when non-null.
 * 1 <= R <= 64, K as ssmoe_gemv_affine4. The workspace must be zero before the first call; every call leaves it
 * zero. */
int ssmoe_lm_head_argmax(const void* x, int x_f32, int R, int K, const int32_t* q, const uint16_t* s,
                         const uint16_t* b, int N, int round_bf16, void* workspace, int64_t workspace_bytes,
                         float* logits, int32_t* ids, void* stream);

/* ---------------------------------------------------------------- MTP draft head (dense part, no attention) */

/* RMSNorm with folded weight (model/reference_torch.py:30-38): out = bf16((x * r) * w) over each group of `group`
 * elements of a row, r = 1 / sqrt(sum(x^2) / group + eps) in fp32 (lane l of a wave sums the 8-element chunks l,
 * l + 64, ... of the group with fmaf from 0, then the xor butterfly). group = n is the plain norm (fuse's
 * pre_fc_norm_hidden over hc * H, engine/mtp.py:190); group = H is the per-branch norm of hc_mix
 * (model/layers.py:192). x, out bf16 [R][n], 16-byte aligned, not aliased; w bf16 [n] or NULL (ones); group a
 * multiple of 8 dividing n. */
int ssmoe_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int R, int n, int group, uint16_t* out,
                  void* stream);

/* Elementwise op fused behind ssmoe_dense_gemv_epi: the GEMV rounds its fp32 dot d to bf16 (v = bf16(d), the
 * result of lin) and then, with torch's bf16 rounding after each step: */
#define SSMOE_EPI_NONE 0     /* v */
#define SSMOE_EPI_ADD 1      /* bf16(add[(r / add_div)][n] + v): e.unsqueeze(-2) + h of fuse (engine/mtp.py:192) */
#define SSMOE_EPI_SILU_DIV 2 /* silu(bf16(v / hc)): hc_mix's low-rank input (model/layers.py:193) */
#define SSMOE_EPI_SIGMOID 3  /* sigmoid(v): hc_mix's mix weights (model/layers.py:194) */
#define SSMOE_EPI_INJECT 4   /* 2 * bf16(sigmoid(bf16(v / hc))): hc_mix's injection (model/layers.py:198) */

/* lin for a bf16 weight (model/layers.py:62-76, the batch-invariant dense gemv) with one SSMOE_EPI_* op fused:
 * out[r][n] = epi(bf16(sum_k x[r][k] w[n][k])), fp32 sum in the order of ssmoe_dense_gemv_bf16 (lane l of a wave sums
 * the 8-element chunks l, l + 64, ... with fmaf from 0, then the xor butterfly); silu(u) = u / (1 + exp(-u)),
 * sigmoid(u) = 1 / (1 + exp(-u)) with the fp32 exp of the router. x bf16 [R][K], w bf16 [N][K], out bf16 [R][N],
 * add bf16 [ceil(R / add_div)][N] (SSMOE_EPI_ADD only). K a multiple of 8, x and w 16-byte aligned. */
int ssmoe_dense_gemv_epi(const uint16_t* x, int R, int K, const uint16_t* w, int N, int epi, int hc,
                         const uint16_t* add, int add_div, uint16_t* out, void* stream);

/* One launch for a run of the head's dense ops, with the bits of the separate calls (ssmoe_gather_rows,
 * ssmoe_hc_inject, ssmoe_rmsnorm, ssmoe_dense_gemv_epi, ssmoe_hc_mean): the steps of engine/mtp.py:184-227 and
 * model/layers.py:190-198 between two head MoE / lm_head calls. No reference counterpart as one call.
 *   source: S rows of n (bf16 [S][n] at src), or rows src_idx[s] of the table src [n_src][n] (src_idx int32 on the
 *     device; an index outside [0, n_src) reads zeros and raises SSMOE_ERR_TOKEN);
 *   inject (inj non-null): h = bf16(src + bf16(inj_y[s][j % (n / inj_hc)] * inj[s][j / (n / inj_hc)]));
 *   norm (group > 0): x = ssmoe_rmsnorm(h, norm_w, eps, group) (norm_w NULL: 1);
 *   the GEMV of ssmoe_dense_gemv_epi over x viewed as S n / K rows of K: weight rows w [N][K] with epi, hc, add,
 *     add_div into out, and rows w2 [N2][K] with epi2 into out2 (N2 may be 0);
 *   or, with mean_out non-null (hc == 4, N = 4 H, no w2, n == K <= 512): also mean_out [S][H] =
 *     ssmoe_hc_mean(out, mean_hn, 4).
 *   h_out / x_out (bf16 [S][n], or NULL) receive h and x.
 * n a multiple of K and of group, K and n multiples of 8, n <= 32768, n / K <= 4, n / group <= 64; pointers
 * 16-byte aligned. */
typedef struct {
  const uint16_t* src;
  const int32_t* src_idx;
  int64_t n_src;
  const uint16_t* inj_y;
  const uint16_t* inj;
  int inj_hc;
  const uint16_t* norm_w;
  float eps;
  int group;
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
} ssmoe_head_gemv_args;
int ssmoe_head_gemv(const ssmoe_head_gemv_args* a, void* stream);

/* The weighted mean of hc_mix (model/layers.py:195): mixed[s][j] = bf16(sum_c bf16(m[s][c H + j] hn[s][c H + j]) /
 * hc), the sum over c = 0 .. hc-1 in order. m, hn bf16 [S][hc H]; mixed bf16 [S][H]. */
int ssmoe_hc_mean(const uint16_t* m, const uint16_t* hn, int S, int hc, int H, uint16_t* mixed, void* stream);

/* The hyper-connection residual (engine/mtp.py:226, h + (m.unsqueeze(-2) * inj.unsqueeze(-1)).flatten(-2)):
 * out[s][c H + j] = bf16(hyp[s][c H + j] + bf16(y[s][j] inj[s][c])). hyp, out bf16 [S][hc H] (out may be hyp),
 * y bf16 [S][H], inj bf16 [S][hc]. */
int ssmoe_hc_inject(const uint16_t* hyp, const uint16_t* y, const uint16_t* inj, int S, int hc, int H, uint16_t* out,
                    void* stream);

/* dst row i = src row idx[i] + idx_add for i < n, read on the device: the embedding lookup of a drafted token
 * (embed([tok]) of engine/mtp.py:274) and the pick of a kept row after a verify round (StepRecord.restore,
 * kernels/gdn_step_record.py:48-56), or the last token a round emitted. row_bytes a multiple of 4, src and dst 4-byte
 * aligned (16-byte pieces when row_bytes and both addresses allow). A row index outside [0, n_src) writes a zero row
 * and raises SSMOE_ERR_TOKEN in the device status. */
int ssmoe_gather_rows(const void* src, int64_t n_src, int64_t row_bytes, const int32_t* idx, int n, int idx_add,
                      void* dst, void* stream);

/* ---------------------------------------------------------------- expert slot pool */

/* An expert slot pool in HBM fed from experts.bin (layout slotstream-pool-layer-expert-piece-v1: the record of
 * layer L, expert e at (L * experts + e) * record_bytes, docs/model-and-repack.md:37-57). Replaces slotio::Pool +
 * Ensurer (slotio/include/slotio/pool.hpp:39-165, slotio/src/ensure.cpp) behind runtime/pool.py's ExpertPool.
 * map int32 [layers * experts] and slot_ptr int64 [max_slots] are the caller's device tables (the ones the kernels
 * read); the pool keeps them current. Slots are device chunks of chunk_bytes; a slot is record_bytes rounded up
 * to 256. Returns SSMOE_EIO if the file cannot be opened. */
int ssmoe_pool_open(const char* experts_path, int layers, int experts, int64_t record_bytes, int max_slots,
                    int64_t chunk_bytes, int32_t* map, int64_t* slot_ptr, void** pool);
int ssmoe_pool_close(void* pool);

/* Reader set-up (slotio Reader::Config lanes, reader.hpp:1; File::open_direct): the misses of an ensure are spread
 * over `lanes` (1..12) reader threads, each with two pinned staging buffers and its own stream, so reads and
 * host-to-device copies overlap. direct != 0 reads with O_DIRECT (record_bytes must be a multiple of 4096;
 * SSMOE_EIO if the file system refuses it). A new pool has 1 lane, buffered. */
int ssmoe_pool_set_reader(void* pool, int lanes, int direct);

/* Grow or shrink to `slots` slots (Pool::resize_slots): shrinking unmaps every slot >= slots and drops its pin. */
int ssmoe_pool_resize(void* pool, int slots);

/* The slot of every requested expert of `layer` (host arrays, input order, duplicates allowed), reading the missing
 * ones from the file into CLOCK victims (Ensurer::ensure). Every returned slot is pinned with generation `gen` until
 * ssmoe_pool_retire_below passes it. Transactional: SSMOE_EXHAUSTED when the unpinned slots cannot hold the misses
 * (nothing changes), SSMOE_EIO when a read fails (pins restored, victims left unmapped, nothing published).
 * timing int64 [6] (may be NULL): hits, misses, bytes read, total ns, read ns, copy ns. */
int ssmoe_pool_ensure(void* pool, int layer, const int32_t* experts, int n, uint64_t gen, int32_t* slots,
                      int64_t* timing);

/* Unpin every slot pinned with a generation below `progress` (Pins::retire_below). */
int ssmoe_pool_retire_below(void* pool, uint64_t progress);

/* Progress word (host memory, e.g. pinned and advanced by a kernel at the end of a step): every ensure first
 * retires the pins below its value (Ensurer::set_progress_ptr). NULL detaches it. */
int ssmoe_pool_set_progress(void* pool, const uint64_t* progress);

/* Copy `bytes` of slot `slot` to dst (host or device memory), the reference's slot_view. */
int ssmoe_pool_copy_slot(void* pool, int slot, void* dst, int64_t bytes);

/* stats int64 [10]: slots, chunks, pinned slots, owned bytes, slot stride, hits, misses, bytes read, lanes,
 * direct. */
int ssmoe_pool_stats(void* pool, int64_t* stats);

/* ---------------------------------------------------------------- shared expert (prefill) */

/* hs[t, i] = bf16(bf16(silu(g)) * u), g = proj[t, i], u = proj[t, Is + i], and sgl[t] = proj[t, 2 Is]: the F.silu and
 * bf16 product of the shared expert (model/layers.py:398-402, reference_torch.py:132-133) applied to one bf16
 * projection [T, ld] that holds the shared gate, up and shared_expert_gate outputs side by side.
 * hs bf16 [T, Is]; sgl bf16 [T]. */
int ssmoe_shared_hs(const uint16_t* proj, int64_t ld, int T, int Is, uint16_t* hs, uint16_t* sgl, void* stream);

/* Residual stream and RMSNorm between chained layers: s = bf16(resid + y) stored to stream_out (skipped when y is
 * NULL: s = resid), mixed = bf16((s * r) * w), r = 1 / sqrt(sum(s^2) / H + eps), weight NULL = ones. Follows the
 * residual add of GraphSet._moe (runtime/graphs.py:169) with one stream and unit injection, and rmsnorm
 * (model/reference_torch.py:30-38) with a fixed reduction order. bf16 [R, H] rows; stream_out may equal resid. */
int ssmoe_residual_rmsnorm(const uint16_t* resid, const uint16_t* y, const uint16_t* weight, float eps, int R, int H,
                           uint16_t* stream_out, uint16_t* mixed, void* stream);

/* y = bf16(bf16(routed) + bf16(bf16(sigmoid(sgl)) * sh)): routed.to(bf16) + sigmoid(x w_sg) * sh with the reference's
 * bf16 rounding of each op (model/layers.py:398-402, reference_torch.py:132-134). routed fp32 [T, H] (16-byte
 * aligned); sh bf16 [T, H]; sgl bf16 [T]; y bf16 [T, H]; H % 4 == 0. */
int ssmoe_combine_shared(const float* routed, const uint16_t* sh, const uint16_t* sgl, uint16_t* y, int T, int H,
                         void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SSMOE_H */
