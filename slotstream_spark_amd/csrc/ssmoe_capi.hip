// extern "C" entry points of libssmoe.so (declared in include/ssmoe.h): argument checks, workspace carving and
// launches. No entry point allocates device memory or synchronises, except ssmoe_device_error.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/ssmoe.h"
#include "ss_common.hpp"
#include "ss_launch.hpp"

// Per-device status word raised by kernels on bad input.
__device__ int ss_status_storage;

// Scratch of ssmoe_moe_decode, which (like the reference's moe_decode) takes no workspace argument: h fragments,
// h partial sums and the persistent kernel's counters for one block of <= 4 rows. Zero at load; every launch leaves
// its counters zero. One slot per stream for the first kDecodeSlots streams that call it on a device (a host table
// assigns them), so calls on different streams do not share a slot; calls on one stream run in order. A stream past
// the first kDecodeSlots shares a slot with an earlier one.
constexpr size_t kDecodeScratch = 320 * 1024;
constexpr int kDecodeSlots = 8;
__device__ __align__(256) unsigned char ss_decode_scratch[kDecodeSlots][kDecodeScratch];

// Scratch of ssmoe_moe_verify_layer_noalloc, the verify layer for callers that cannot allocate: the counters, tagged
// router logits, shared-expert rows and h fragments that ssmoe_moe_verify_layer keeps in the caller's workspace.
// 192 KiB holds every (H, I, Is, K, E) the verify kernel takes with I * K <= 8192 (the BASELINE layer, H 2048 / I 512
// / K 10, needs 127 KiB; the reference model's H 2560 / I 640 / K 10, 150 KiB). Host code never names this array
// in a launch: it uses the address hipGetSymbolAddress returns for the current device (g_noalloc_scratch).
constexpr size_t kNoAllocScratch = 192 * 1024;
__device__ __align__(256) unsigned char ss_noalloc_scratch[kNoAllocScratch];

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return SSMOE_OK;
}

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(SSMOE_EHIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

constexpr int kMaxDevices = 64;
int* g_status[kMaxDevices] = {nullptr};
void* g_decode_scratch[kMaxDevices] = {nullptr};
void* g_noalloc_scratch[kMaxDevices] = {nullptr};
std::mutex g_noalloc_mu;

int current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return hip_check(e, "hipGetDevice");
  if (*dev < 0 || *dev >= kMaxDevices) return fail(SSMOE_EHIP, "device %d out of range", *dev);
  return ok();
}

// Device addresses of the status word and the decode scratch on the current device (looked up once per device).
int status_ptr(int** out) {
  int dev = 0;
  if (int rc = current_device(&dev)) return rc;
  if (!g_status[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(ss_status_storage));
    if (e != hipSuccess) return hip_check(e, "hipGetSymbolAddress(status)");
    g_status[dev] = static_cast<int*>(p);
  }
  *out = g_status[dev];
  return ok();
}

// The decode scratch slot of `stream` on the current device: the stream's own slot once it has one, else the next
// free one, else (more streams than slots) the slot its handle hashes to.
hipStream_t g_decode_streams[kMaxDevices][kDecodeSlots];
int g_decode_used[kMaxDevices] = {0};
std::mutex g_decode_mu;

int decode_scratch_ptr(hipStream_t stream, void** out) {
  int dev = 0;
  if (int rc = current_device(&dev)) return rc;
  std::lock_guard<std::mutex> lock(g_decode_mu);
  if (!g_decode_scratch[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(ss_decode_scratch));
    if (e != hipSuccess) return hip_check(e, "hipGetSymbolAddress(decode scratch)");
    g_decode_scratch[dev] = p;
  }
  int slot = -1;
  for (int i = 0; i < g_decode_used[dev] && slot < 0; ++i)
    if (g_decode_streams[dev][i] == stream) slot = i;
  if (slot < 0 && g_decode_used[dev] < kDecodeSlots) {
    slot = g_decode_used[dev]++;
    g_decode_streams[dev][slot] = stream;
  }
  if (slot < 0) slot = (int)((reinterpret_cast<uintptr_t>(stream) >> 4) % kDecodeSlots);
  *out = static_cast<unsigned char*>(g_decode_scratch[dev]) + (size_t)slot * kDecodeScratch;
  return ok();
}

// Device address of ss_noalloc_scratch on the current device. The first call on a device looks it up and clears it
// with a fill kernel on `st` (ordered before the launch that follows on the same stream): the kernel needs its
// counters at zero and no tagged logit word of an earlier launch left behind.
int noalloc_scratch_ptr(void** out, hipStream_t st) {
  int dev = 0;
  if (int rc = current_device(&dev)) return rc;
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_scratch[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(ss_noalloc_scratch));
    if (e != hipSuccess) return hip_check(e, "hipGetSymbolAddress(no-alloc scratch)");
    e = ss::launch_zero16(p, kNoAllocScratch, st);
    if (e != hipSuccess) return hip_check(e, "no-alloc scratch clear");
    g_noalloc_scratch[dev] = p;
  }
  *out = g_noalloc_scratch[dev];
  return ok();
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_moe_shape(int R, int H, int I, int K, int E) {
  if (R < 1) return fail(SSMOE_EINVAL, "R must be >= 1, got %d", R);
  if (H < 128 || H % 128 || H > 4096) return fail(SSMOE_EINVAL, "H must be a multiple of 128 in [128, 4096], got %d", H);
  if (I < 128 || I % 128 || I > 1024) return fail(SSMOE_EINVAL, "I must be a multiple of 128 in [128, 1024], got %d", I);
  if (K < 1 || K > 16) return fail(SSMOE_EINVAL, "K must be in [1, 16], got %d", K);
  if (E < 1) return fail(SSMOE_EINVAL, "E must be >= 1, got %d", E);
  return ok();
}

constexpr int kBlock = 4;  // rows per persistent launch
uint64_t* g_trace = nullptr;  // diagnostics: phase timestamps of the persistent kernel (ssmoe_set_trace)

}  // namespace

extern "C" {

const char* ssmoe_last_error(void) { return g_err.c_str(); }

int ssmoe_version(void) { return 1; }

int ssmoe_device_error(int* flags, int clear) {
  if (!flags) return fail(SSMOE_EINVAL, "flags must be a host pointer");
  int* p = nullptr;
  if (int rc = status_ptr(&p)) return rc;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_check(e, "hipDeviceSynchronize");
  e = hipMemcpy(flags, p, sizeof(int), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_check(e, "hipMemcpy(status)");
  if (clear) {
    const int zero = 0;
    e = hipMemcpy(p, &zero, sizeof(int), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_check(e, "hipMemcpy(status clear)");
  }
  return ok();
}

int ssmoe_set_trace(void* buf, int64_t entries) {
  if (buf && entries < 1024 * 16) return fail(SSMOE_EINVAL, "trace buffer needs >= %d entries", 1024 * 16);
  g_trace = static_cast<uint64_t*>(buf);
  return ok();
}

int ssmoe_record_layout(int H, int I, int64_t* off) {
  if (!off) return fail(SSMOE_EINVAL, "off must be a host pointer to 10 int64");
  if (H < 64 || H % 64 || I < 64 || I % 64) return fail(SSMOE_EINVAL, "H and I must be positive multiples of 64");
  const SsRecord r = ss_record_layout(H, I);
  const int64_t v[10] = {r.gw, r.gs, r.gb, r.uw, r.us, r.ub, r.dw, r.ds, r.db, r.bytes};
  for (int i = 0; i < 10; ++i) off[i] = v[i];
  return ok();
}

int ssmoe_moe_decode(const void* x, int x_is_f32, const int32_t* expert_ids, const float* weights, int layer,
                     const int32_t* map, int64_t map_len, const int64_t* slot_ptr, int64_t n_slots, float* h_buf,
                     float* o_buf, float* out, int R, int H, int I, int K, int E, void* stream) {
  if (int rc = check_moe_shape(R, H, I, K, E)) return rc;
  if (!x || !expert_ids || !weights || !map || !slot_ptr || !h_buf || !out)
    return fail(SSMOE_EINVAL, "x, expert_ids, weights, map, slot_ptr, h_buf and out must be non-null");
  if (layer < 0) return fail(SSMOE_EINVAL, "layer must be >= 0, got %d", layer);
  if (!aligned(x, 16) || !aligned(h_buf, 16)) return fail(SSMOE_EINVAL, "x and h_buf must be 16-byte aligned");
  if ((int64_t)(layer + 1) * E > map_len)
    return fail(SSMOE_EINVAL, "map holds %lld entries, layer %d needs %lld", (long long)map_len, layer,
                (long long)(layer + 1) * E);
  if (ss::verify_scratch_bytes(kBlock, H, I, 0, K, 0) > kDecodeScratch)
    return fail(SSMOE_EINVAL, "shape needs more decode scratch than the library holds");
  int* err = nullptr;
  void* scratch = nullptr;
  if (int rc = status_ptr(&err)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (int rc = decode_scratch_ptr(st, &scratch)) return rc;
  const size_t xsz = x_is_f32 ? 4 : 2;
  for (int r0 = 0; r0 < R; r0 += kBlock) {
    ss::VerifyArgs a{};
    a.mode = 1;
    a.x = static_cast<const char*>(x) + (size_t)r0 * H * xsz;
    a.x_f32 = x_is_f32 ? 1 : 0;
    a.map = map;
    a.map_len = map_len;
    a.slot_ptr = slot_ptr;
    a.n_slots = n_slots;
    a.map_base = (int64_t)layer * E;
    a.ids_in = expert_ids + (size_t)r0 * K;
    a.w_in = weights + (size_t)r0 * K;
    a.out = out + (size_t)r0 * H;
    a.h_buf = h_buf + (size_t)r0 * K * I;
    a.o_buf = o_buf ? o_buf + (size_t)r0 * K * H : nullptr;
    a.scratch = scratch;
    a.T = R - r0 < kBlock ? R - r0 : kBlock;
    a.H = H;
    a.I = I;
    a.Is = 0;
    a.K = K;
    a.E = E;
    a.err = err;
    a.trace = g_trace;
    if (int rc = hip_check(ss::launch_verify(a, st), "moe_decode launch")) return rc;
  }
  return ok();
}

int ssmoe_topk_stable(const float* scores, const int32_t* n_valid, int32_t* out_idx, float* out_val, int R, int N,
                      int k, void* stream) {
  if (R < 1 || N < 1 || N > 65536) return fail(SSMOE_EINVAL, "need R >= 1 and 1 <= N <= 65536 (R=%d N=%d)", R, N);
  if (k < 1 || k > N) return fail(SSMOE_EINVAL, "need 1 <= k <= N, got k=%d N=%d", k, N);
  if (!scores || !out_idx) return fail(SSMOE_EINVAL, "scores and out_idx must be non-null");
  return hip_check(ss::launch_topk_stable(scores, n_valid, out_idx, out_val, R, N, k, static_cast<hipStream_t>(stream)),
                   "topk_stable launch");
}

int ssmoe_dense_gemv_bf16(const uint16_t* x, const uint16_t* w, uint16_t* out, int T, int H, int N, void* stream) {
  if (T < 1 || N < 1 || H < 8 || H % 8 || H > 8192)
    return fail(SSMOE_EINVAL, "need T, N >= 1 and H a multiple of 8 in [8, 8192] (T=%d H=%d N=%d)", T, H, N);
  if (!x || !w || !out) return fail(SSMOE_EINVAL, "x, w and out must be non-null");
  if (!aligned(x, 16) || !aligned(w, 16)) return fail(SSMOE_EINVAL, "x and w must be 16-byte aligned");
  ss::DenseSeg s{w, out, N, N};
  return hip_check(ss::launch_dense_rows(x, T, H, &s, 1, static_cast<hipStream_t>(stream)), "dense gemv launch");
}

int ssmoe_dense_gemm(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, uint16_t* c, int64_t ldc, int M,
                     int N, int K, void* stream) {
  if (M < 0 || N < 0 || K < 256 || K % 256) return fail(SSMOE_EINVAL, "need M, N >= 0 and K a positive multiple of 256");
  if (lda < K || ldw < K || ldc < N || lda % 8 || ldw % 8 || ldc % 8)
    return fail(SSMOE_EINVAL, "need lda, ldw >= K, ldc >= N, all multiples of 8");
  if (!a || !w || !c) return fail(SSMOE_EINVAL, "a, w and c must be non-null");
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(c, 16)) return fail(SSMOE_EINVAL, "a, w and c must be 16-byte aligned");
  return hip_check(ss::launch_dense_gemm(a, lda, w, ldw, c, ldc, M, N, K, static_cast<hipStream_t>(stream)),
                   "dense gemm launch");
}

int ssmoe_router(const uint16_t* x, const uint16_t* router_w, const float* bias, uint16_t* logits, float* probs,
                 int32_t* ids, float* weights, int T, int H, int E, int K, void* stream) {
  if (T < 1 || H < 8 || H % 8 || H > 8192) return fail(SSMOE_EINVAL, "need T >= 1, H a multiple of 8 <= 8192");
  if (E < 1 || E > 8192 || K < 1 || K > 16 || K > E) return fail(SSMOE_EINVAL, "need 1 <= K <= min(16, E), E <= 8192");
  if (!x || !router_w || !logits || !ids || !weights)
    return fail(SSMOE_EINVAL, "x, router_w, logits, ids and weights must be non-null");
  if (!aligned(x, 16) || !aligned(router_w, 16)) return fail(SSMOE_EINVAL, "x and router_w must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  ss::DenseSeg s{router_w, logits, E, E};
  if (int rc = hip_check(ss::launch_dense_rows(x, T, H, &s, 1, st), "router gemv launch")) return rc;
  return hip_check(ss::launch_router_topk(logits, bias, probs, ids, weights, T, E, K, st), "router topk launch");
}

int ssmoe_router_topk(const uint16_t* logits, const float* bias, float* probs, int32_t* ids, float* weights, int T,
                      int E, int K, void* stream) {
  if (T < 1 || E < 1 || E > 8192 || K < 1 || K > 16 || K > E)
    return fail(SSMOE_EINVAL, "need T >= 1 and 1 <= K <= min(16, E), E <= 8192 (T=%d E=%d K=%d)", T, E, K);
  if (!logits || !ids || !weights) return fail(SSMOE_EINVAL, "logits, ids and weights must be non-null");
  return hip_check(ss::launch_router_topk(logits, bias, probs, ids, weights, T, E, K, static_cast<hipStream_t>(stream)),
                   "router top-k launch");
}

int64_t ssmoe_verify_workspace_bytes(int T, int H, int I, int Is, int K, int E) {
  if (T < 1 || Is < 1 || I < 1 || K < 1 || E < 1) return -1;
  (void)T;
  return (int64_t)ss::verify_scratch_bytes(kBlock, H, I, Is, K, E);
}

// The affine 4-bit shared expert's scales and biases: all six or none; with them the weights hold packed words.
static int check_shared_q4(const ssmoe_shared_q4* q4, int H, int Is) {
  if (!q4) return ok();
  if (!q4->gate_s || !q4->gate_b || !q4->up_s || !q4->up_b || !q4->down_s || !q4->down_b)
    return fail(SSMOE_EINVAL, "an affine 4-bit shared expert needs all six scale and bias pointers");
  if (H % 64 || Is % 64) return fail(SSMOE_EINVAL, "an affine 4-bit (gs 64) shared expert needs H and Is multiples of 64");
  if (!aligned(q4->gate_s, 2) || !aligned(q4->gate_b, 2) || !aligned(q4->up_s, 2) || !aligned(q4->up_b, 2) ||
      !aligned(q4->down_s, 2) || !aligned(q4->down_b, 2))
    return fail(SSMOE_EINVAL, "scales and biases must be 2-byte aligned");
  return ok();
}

static int verify_layer_impl(const uint16_t* x, const uint16_t* router_w, const float* router_bias,
                             const uint16_t* sh_gate, const uint16_t* sh_up, const uint16_t* sh_down,
                             const uint16_t* sh_g, int layer, const int32_t* map, int64_t map_len,
                             const int64_t* slot_ptr, int64_t n_slots, void* workspace, int64_t workspace_bytes,
                             int32_t* ids, float* weights, uint16_t* y, float* routed_out, int T, int H, int I, int Is,
                             int K, int E, void* stream, int norm_in, const uint16_t* norm_w, float norm_eps,
                             uint16_t* x_plus_y, const ssmoe_shared_q4* q4 = nullptr) {
  if (int rc = check_moe_shape(T, H, I, K, E)) return rc;
  if (E > 512 || K > E) return fail(SSMOE_EINVAL, "need K <= E <= 512, got K=%d E=%d", K, E);
  if (Is < 8 || Is % 8 || Is > (I > 512 ? 1024 : 512))
    return fail(SSMOE_EINVAL, "Is must be a multiple of 8 in [8, %d] (I = %d), got %d", I > 512 ? 1024 : 512, I, Is);
  if (int rc = check_shared_q4(q4, H, Is)) return rc;
  if (!x || !router_w || !sh_gate || !sh_up || !sh_down || !sh_g || !map || !slot_ptr || !workspace || !ids ||
      !weights || !y)
    return fail(SSMOE_EINVAL, "every pointer except router_bias and routed_out must be non-null");
  if (!aligned(x, 16) || !aligned(router_w, 16) || !aligned(sh_gate, 16) || !aligned(sh_up, 16) ||
      !aligned(sh_down, 16) || !aligned(sh_g, 16) || !aligned(workspace, 256))
    return fail(SSMOE_EINVAL, "x and weights must be 16-byte aligned, workspace 256-byte aligned");
  if (layer < 0 || (int64_t)(layer + 1) * E > map_len)
    return fail(SSMOE_EINVAL, "map holds %lld entries, layer %d needs %lld", (long long)map_len, layer,
                (long long)(layer + 1) * E);
  const size_t need = ss::verify_scratch_bytes(kBlock, H, I, Is, K, E);
  if (workspace_bytes < (int64_t)need)
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes, (long long)need);
  int* err = nullptr;
  if (int rc = status_ptr(&err)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int r0 = 0; r0 < T; r0 += kBlock) {
    ss::VerifyArgs a{};
    a.mode = 0;
    a.x = x + (size_t)r0 * H;
    a.router_w = router_w;
    a.bias = router_bias;
    a.sh_gate = sh_gate;
    a.sh_up = sh_up;
    a.sh_down = sh_down;
    a.sh_g = sh_g;
    if (q4) {
      a.sh_gs = q4->gate_s;
      a.sh_gb = q4->gate_b;
      a.sh_us = q4->up_s;
      a.sh_ub = q4->up_b;
      a.sh_ds = q4->down_s;
      a.sh_db = q4->down_b;
    }
    a.map = map;
    a.map_len = map_len;
    a.slot_ptr = slot_ptr;
    a.n_slots = n_slots;
    a.map_base = (int64_t)layer * E;
    a.ids_out = ids + (size_t)r0 * K;
    a.w_out = weights + (size_t)r0 * K;
    a.y = y + (size_t)r0 * H;
    a.out = routed_out ? routed_out + (size_t)r0 * H : nullptr;
    a.scratch = workspace;
    a.T = T - r0 < kBlock ? T - r0 : kBlock;
    a.H = H;
    a.I = I;
    a.Is = Is;
    a.K = K;
    a.E = E;
    a.err = err;
    a.trace = g_trace;
    a.norm_in = norm_in;
    a.norm_w = norm_w;
    a.norm_eps = norm_eps;
    a.x_plus_y = x_plus_y ? x_plus_y + (size_t)r0 * H : nullptr;
    if (int rc = hip_check(ss::launch_verify(a, st), "verify layer launch")) return rc;
  }
  return ok();
}

int ssmoe_moe_verify_layer(const uint16_t* x, const uint16_t* router_w, const float* router_bias,
                           const uint16_t* sh_gate, const uint16_t* sh_up, const uint16_t* sh_down,
                           const uint16_t* sh_g, int layer, const int32_t* map, int64_t map_len,
                           const int64_t* slot_ptr, int64_t n_slots, void* workspace, int64_t workspace_bytes,
                           int32_t* ids, float* weights, uint16_t* y, float* routed_out, int T, int H, int I, int Is,
                           int K, int E, void* stream) {
  return verify_layer_impl(x, router_w, router_bias, sh_gate, sh_up, sh_down, sh_g, layer, map, map_len, slot_ptr,
                           n_slots, workspace, workspace_bytes, ids, weights, y, routed_out, T, H, I, Is, K, E, stream,
                           0, nullptr, 0.f, nullptr);
}

int ssmoe_moe_verify_layer_chain(const uint16_t* stream_in, const uint16_t* norm_w, float eps,
                                 const uint16_t* router_w, const float* router_bias, const uint16_t* sh_gate,
                                 const uint16_t* sh_up, const uint16_t* sh_down, const uint16_t* sh_g, int layer,
                                 const int32_t* map, int64_t map_len, const int64_t* slot_ptr, int64_t n_slots,
                                 void* workspace, int64_t workspace_bytes, int32_t* ids, float* weights, uint16_t* y,
                                 uint16_t* stream_out, float* routed_out, int T, int H, int I, int Is, int K, int E,
                                 void* stream) {
  if (H % 512 != 0) return fail(SSMOE_EINVAL, "chained layers need H a multiple of 512, got %d", H);
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(SSMOE_EINVAL, "eps must be finite and >= 0");
  if (norm_w && !aligned(norm_w, 16)) return fail(SSMOE_EINVAL, "norm_w must be 16-byte aligned");
  if (stream_out && (stream_out == stream_in || stream_out == y))
    return fail(SSMOE_EINVAL, "stream_out must not alias stream_in or y (other workgroups still read stream_in)");
  if (stream_out && !aligned(stream_out, 16)) return fail(SSMOE_EINVAL, "stream_out must be 16-byte aligned");
  return verify_layer_impl(stream_in, router_w, router_bias, sh_gate, sh_up, sh_down, sh_g, layer, map, map_len,
                           slot_ptr, n_slots, workspace, workspace_bytes, ids, weights, y, routed_out, T, H, I, Is, K,
                           E, stream, 1, norm_w, eps, stream_out);
}

int ssmoe_moe_verify_layer_q4s(const uint16_t* x, const uint16_t* router_w, const float* router_bias,
                               const uint16_t* sh_gate, const uint16_t* sh_up, const uint16_t* sh_down,
                               const uint16_t* sh_g, const ssmoe_shared_q4* sh_q4, int layer, const int32_t* map,
                               int64_t map_len, const int64_t* slot_ptr, int64_t n_slots, void* workspace,
                               int64_t workspace_bytes, int32_t* ids, float* weights, uint16_t* y, float* routed_out,
                               int T, int H, int I, int Is, int K, int E, void* stream) {
  if (!sh_q4) return fail(SSMOE_EINVAL, "sh_q4 must be non-null (bf16 shared weights: ssmoe_moe_verify_layer)");
  return verify_layer_impl(x, router_w, router_bias, sh_gate, sh_up, sh_down, sh_g, layer, map, map_len, slot_ptr,
                           n_slots, workspace, workspace_bytes, ids, weights, y, routed_out, T, H, I, Is, K, E, stream,
                           0, nullptr, 0.f, nullptr, sh_q4);
}

int ssmoe_moe_verify_layer_chain_q4s(const uint16_t* stream_in, const uint16_t* norm_w, float eps,
                                     const uint16_t* router_w, const float* router_bias, const uint16_t* sh_gate,
                                     const uint16_t* sh_up, const uint16_t* sh_down, const uint16_t* sh_g,
                                     const ssmoe_shared_q4* sh_q4, int layer, const int32_t* map, int64_t map_len,
                                     const int64_t* slot_ptr, int64_t n_slots, void* workspace,
                                     int64_t workspace_bytes, int32_t* ids, float* weights, uint16_t* y,
                                     uint16_t* stream_out, float* routed_out, int T, int H, int I, int Is, int K,
                                     int E, void* stream) {
  if (!sh_q4) return fail(SSMOE_EINVAL, "sh_q4 must be non-null (bf16 shared weights: ssmoe_moe_verify_layer_chain)");
  if (H % 512 != 0) return fail(SSMOE_EINVAL, "chained layers need H a multiple of 512, got %d", H);
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(SSMOE_EINVAL, "eps must be finite and >= 0");
  if (norm_w && !aligned(norm_w, 16)) return fail(SSMOE_EINVAL, "norm_w must be 16-byte aligned");
  if (stream_out && (stream_out == stream_in || stream_out == y))
    return fail(SSMOE_EINVAL, "stream_out must not alias stream_in or y (other workgroups still read stream_in)");
  if (stream_out && !aligned(stream_out, 16)) return fail(SSMOE_EINVAL, "stream_out must be 16-byte aligned");
  return verify_layer_impl(stream_in, router_w, router_bias, sh_gate, sh_up, sh_down, sh_g, layer, map, map_len,
                           slot_ptr, n_slots, workspace, workspace_bytes, ids, weights, y, routed_out, T, H, I, Is, K,
                           E, stream, 1, norm_w, eps, stream_out, sh_q4);
}

int64_t ssmoe_verify_chain_workspace_bytes(int T, int H, int I, int Is, int K, int E) {
  if (T < 1 || T > kBlock || !ss::chain_shape_supported(H, I) || Is < 8 || Is % 8 || Is > (I > 512 ? 1024 : 512) ||
      K < 1 || K > 16 ||
      E < K || E > 512)
    return -1;
  return (int64_t)ss::chain_scratch_bytes(kBlock, H, I, Is, K, E);
}

int ssmoe_moe_verify_chain(const uint16_t* stream_in, float eps, const ssmoe_chain_layer* layers_host,
                           const ssmoe_chain_layer* layers_dev, int n_layers, const int32_t* map, int64_t map_len,
                           const int64_t* slot_ptr, int64_t n_slots, void* workspace, int64_t workspace_bytes, int T,
                           int H, int I, int Is, int K, int E, void* stream) {
  if (int rc = check_moe_shape(T, H, I, K, E)) return rc;
  if (T > kBlock) return fail(SSMOE_EINVAL, "a chain takes at most %d tokens, got %d", kBlock, T);
  if (!ss::chain_shape_supported(H, I))
    return fail(SSMOE_EINVAL, "no chain kernel for H=%d, I=%d (%s); launch the layers one by one "
                "(ssmoe_moe_verify_layer_chain)", H, I, ss::chain_shapes_text());
  if (E > 512 || K > E) return fail(SSMOE_EINVAL, "need K <= E <= 512, got K=%d E=%d", K, E);
  if (Is < 8 || Is % 8 || Is > (I > 512 ? 1024 : 512))
    return fail(SSMOE_EINVAL, "Is must be a multiple of 8 in [8, %d] (I = %d), got %d", I > 512 ? 1024 : 512, I, Is);
  if (n_layers < 1 || n_layers > 4096) return fail(SSMOE_EINVAL, "n_layers must be in [1, 4096], got %d", n_layers);
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(SSMOE_EINVAL, "eps must be finite and >= 0");
  if (!stream_in || !aligned(stream_in, 16)) return fail(SSMOE_EINVAL, "stream_in must be a 16-byte aligned pointer");
  if (!layers_host || (n_layers > 1 && !layers_dev))
    return fail(SSMOE_EINVAL, "layers_host (and, for more than one layer, layers_dev) must be non-null");
  if (!map || !slot_ptr || !workspace || !aligned(workspace, 256))
    return fail(SSMOE_EINVAL, "map, slot_ptr and a 256-byte aligned workspace are required");
  for (int l = 0; l < n_layers; ++l) {
    const ssmoe_chain_layer& q = layers_host[l];
    if (!q.router_w || !q.sh_gate || !q.sh_up || !q.sh_down || !q.sh_g || !q.ids || !q.weights || !q.y)
      return fail(SSMOE_EINVAL, "layer %d: weights, ids, weights and y must be non-null", l);
    if (!aligned(q.router_w, 16) || !aligned(q.sh_gate, 16) || !aligned(q.sh_up, 16) || !aligned(q.sh_down, 16) ||
        !aligned(q.sh_g, 16) || (q.norm_w && !aligned(q.norm_w, 16)))
      return fail(SSMOE_EINVAL, "layer %d: weights must be 16-byte aligned", l);
    if (q.layer < 0 || (q.layer + 1) * E > map_len)
      return fail(SSMOE_EINVAL, "layer %d: map holds %lld entries, map row %lld needs %lld", l, (long long)map_len,
                  (long long)q.layer, (long long)(q.layer + 1) * E);
    if (q.stream_out && (q.stream_out == q.y || (l == 0 && q.stream_out == stream_in)))
      return fail(SSMOE_EINVAL, "layer %d: stream_out must not alias y or stream_in", l);
    const bool any_q4 = q.sh_gate_s || q.sh_gate_b || q.sh_up_s || q.sh_up_b || q.sh_down_s || q.sh_down_b;
    if (any_q4 != (layers_host[0].sh_gate_s != nullptr))
      return fail(SSMOE_EINVAL, "layer %d: every layer of a chain has an affine 4-bit shared expert, or none", l);
    if (any_q4) {
      const ssmoe_shared_q4 q4{q.sh_gate_s, q.sh_gate_b, q.sh_up_s, q.sh_up_b, q.sh_down_s, q.sh_down_b};
      if (check_shared_q4(&q4, H, Is)) {
        const std::string m = ssmoe_last_error();
        return fail(SSMOE_EINVAL, "layer %d: %s", l, m.c_str());
      }
    }
  }
  const size_t need = ss::chain_scratch_bytes(kBlock, H, I, Is, K, E);
  if (workspace_bytes < (int64_t)need)
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes, (long long)need);
  int dev = 0, cus = 0;
  if (int rc = current_device(&dev)) return rc;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return fail(SSMOE_EHIP, "hipDeviceGetAttribute(multiprocessor count) failed");
  if (E + Is < 4 * cus || H / 16 >= cus)
    return fail(SSMOE_EINVAL, "a chain needs E + Is >= 4 * CUs (one router or shared row per wave) and H / 16 < CUs "
                "(workgroups without output rows for the shared expert's rows; %d CUs; E + Is = %d, H = %d); launch "
                "the layers one by one", cus, E + Is, H);
  int* err = nullptr;
  if (int rc = status_ptr(&err)) return rc;
  ss::ChainArgs a{};
  a.stream_in = stream_in;
  a.norm_in = 1;
  a.eps = eps;
  a.l0 = layers_host[0];
  a.more = n_layers > 1 ? layers_dev + 1 : nullptr;
  a.NL = n_layers;
  a.map = map;
  a.map_len = map_len;
  a.slot_ptr = slot_ptr;
  a.n_slots = n_slots;
  a.scratch = workspace;
  a.T = T;
  a.H = H;
  a.I = I;
  a.Is = Is;
  a.K = K;
  a.E = E;
  a.err = err;
  a.trace = g_trace;
  return hip_check(ss::launch_chain(a, static_cast<hipStream_t>(stream)), "verify chain launch");
}

int ssmoe_moe_verify_layer_noalloc(const uint16_t* x, const uint16_t* router_w, const float* router_bias,
                                   const uint16_t* sh_gate, const uint16_t* sh_up, const uint16_t* sh_down,
                                   const uint16_t* sh_g, int layer, const int32_t* map, int64_t map_len,
                                   const int64_t* slot_ptr, int64_t n_slots, int32_t* ids, float* weights,
                                   uint16_t* y, float* routed_out, int T, int H, int I, int Is, int K, int E,
                                   void* stream) {
  if (int rc = check_moe_shape(T, H, I, K, E)) return rc;
  if (Is < 8 || Is % 8 || Is > (I > 512 ? 1024 : 512))
    return fail(SSMOE_EINVAL, "Is must be a multiple of 8 in [8, %d] (I = %d), got %d", I > 512 ? 1024 : 512, I, Is);
  if (E > 512) return fail(SSMOE_EINVAL, "need E <= 512, got %d", E);
  const size_t need = ss::verify_scratch_bytes(kBlock, H, I, Is, K, E);
  if (need > kNoAllocScratch)
    return fail(SSMOE_EINVAL, "shape needs %zu bytes of scratch; the no-alloc entry point holds %zu (I * K <= 8192 "
                "fits); use ssmoe_moe_verify_layer with a workspace", need, kNoAllocScratch);
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* scratch = nullptr;
  if (int rc = noalloc_scratch_ptr(&scratch, st)) return rc;
  return verify_layer_impl(x, router_w, router_bias, sh_gate, sh_up, sh_down, sh_g, layer, map, map_len, slot_ptr,
                           n_slots, scratch, (int64_t)kNoAllocScratch, ids, weights, y, routed_out, T, H, I, Is, K, E,
                           stream, 0, nullptr, 0.f, nullptr);
}

int64_t ssmoe_accept_workspace_bytes(int D, int V) {
  if (D < 0 || V < 1) return -1;
  return ss::accept_work_floats(D, V) * 4;
}

static int check_accept(int D, int V, void* workspace, int64_t workspace_bytes, int32_t* out) {
  if (D < 0 || D > 60) return fail(SSMOE_EINVAL, "D must be in [0, 60], got %d", D);
  if (V < 1 || V > (1 << 20)) return fail(SSMOE_EINVAL, "V must be in [1, 1048576], got %d", V);
  if (!workspace || !out) return fail(SSMOE_EINVAL, "workspace and out must be non-null");
  if (workspace_bytes < ss::accept_work_floats(D, V) * 4)
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)(ss::accept_work_floats(D, V) * 4));
  return ok();
}

int ssmoe_accept_greedy(const float* target, const int32_t* drafts, int D, int V, void* workspace,
                        int64_t workspace_bytes, int32_t* out, void* stream) {
  if (int rc = check_accept(D, V, workspace, workspace_bytes, out)) return rc;
  if (!target || (D > 0 && !drafts)) return fail(SSMOE_EINVAL, "target and drafts must be non-null");
  ss::AcceptArgs a{};
  a.target = target;
  a.drafts = drafts;
  a.D = D;
  a.V = V;
  a.out = out;
  a.work = static_cast<float*>(workspace);
  return hip_check(ss::launch_accept_greedy(a, static_cast<hipStream_t>(stream)), "accept greedy launch");
}

int ssmoe_accept_pq(const float* target, const float* draft, const int32_t* drafts, const float* uniforms, int D,
                    int V, float temperature, void* workspace, int64_t workspace_bytes, int32_t* out,
                    void* stream) {
  if (int rc = check_accept(D, V, workspace, workspace_bytes, out)) return rc;
  if (!target || !uniforms || (D > 0 && (!draft || !drafts)))
    return fail(SSMOE_EINVAL, "target, draft, drafts and uniforms must be non-null");
  if (!(temperature > 0.f) || temperature != temperature)
    return fail(SSMOE_EINVAL, "temperature must be > 0, got %g", (double)temperature);
  int* err = nullptr;
  if (int rc = status_ptr(&err)) return rc;
  ss::AcceptArgs a{};
  a.target = target;
  a.draft = draft;
  a.drafts = drafts;
  a.uniforms = uniforms;
  a.D = D;
  a.V = V;
  a.temperature = temperature;
  a.out = out;
  a.work = static_cast<float*>(workspace);
  a.err = err;
  a.trace = g_trace;
  return hip_check(ss::launch_accept_pq(a, static_cast<hipStream_t>(stream)), "accept pq launch");
}

// ---------------------------------------------------------------- prefill
int64_t ssmoe_padded_rows(int64_t R, int num_local, int block_m) {
  if (R < 0 || num_local < 1 || block_m < 1) return -1;
  return ss::padded_rows(R, num_local, block_m);
}

int64_t ssmoe_moe_align_workspace_bytes(int64_t R, int num_local) {
  if (R < 0 || num_local < 1) return -1;
  return ss::align_scratch_ints(R, num_local) * 4;
}

static int check_align(int64_t R, int num_local, int block_m) {
  if (R < 0 || R > (1ll << 30)) return fail(SSMOE_EINVAL, "R must be in [0, 2^30], got %lld", (long long)R);
  if (num_local < 1 || num_local > 4096) return fail(SSMOE_EINVAL, "num_local must be in [1, 4096], got %d", num_local);
  if (block_m < 1 || block_m > 1024) return fail(SSMOE_EINVAL, "block_m must be in [1, 1024], got %d", block_m);
  return ok();
}

int ssmoe_moe_align(const int32_t* local_expert, int64_t R, int num_local, int block_m, void* workspace,
                    int64_t workspace_bytes, int32_t* sorted_rows, int32_t* block_expert, int32_t* num_padded,
                    void* stream) {
  if (int rc = check_align(R, num_local, block_m)) return rc;
  if ((R > 0 && !local_expert) || !workspace || !sorted_rows || !block_expert || !num_padded)
    return fail(SSMOE_EINVAL, "local_expert, workspace and the three outputs must be non-null");
  if (workspace_bytes < ss::align_scratch_ints(R, num_local) * 4)
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)(ss::align_scratch_ints(R, num_local) * 4));
  ss::AlignArgs a{};
  a.local_expert = local_expert;
  a.R = R;
  a.num_local = num_local;
  a.block_m = block_m;
  a.sorted_rows = sorted_rows;
  a.block_expert = block_expert;
  a.num_padded = num_padded;
  a.scratch = static_cast<int32_t*>(workspace);
  return hip_check(ss::launch_moe_align(a, static_cast<hipStream_t>(stream)), "moe_align launch");
}

static int check_prefill_shape(int64_t R, int H, int I) {
  if (R < 0 || R > (1ll << 30)) return fail(SSMOE_EINVAL, "R must be in [0, 2^30], got %lld", (long long)R);
  if (H < 256 || H % 256 || H > 4096) return fail(SSMOE_EINVAL, "H must be a multiple of 256 in [256, 4096], got %d", H);
  if (I < 128 || I % 128 || I > 4096) return fail(SSMOE_EINVAL, "I must be a multiple of 128 in [128, 4096], got %d", I);
  return ok();
}

int ssmoe_fused_moe_affine(const uint16_t* x, const int32_t* row_token, const float* row_weight,
                           const int32_t* sorted_rows, const int32_t* block_expert, const int32_t* num_padded,
                           const int64_t* group_ptr, int num_local, uint16_t* h_buf, float* out_rows, int64_t R,
                           int T, int H, int I, void* stream) {
  if (int rc = check_prefill_shape(R, H, I)) return rc;
  if (T < 0) return fail(SSMOE_EINVAL, "T must be >= 0, got %d", T);
  if (num_local < 1) return fail(SSMOE_EINVAL, "num_local must be >= 1, got %d", num_local);
  if (R == 0) return ok();
  if (!x || !row_token || !row_weight || !sorted_rows || !block_expert || !num_padded || !group_ptr || !h_buf ||
      !out_rows)
    return fail(SSMOE_EINVAL, "every pointer must be non-null");
  if (!aligned(x, 16) || !aligned(h_buf, 16)) return fail(SSMOE_EINVAL, "x and h_buf must be 16-byte aligned");
  ss::PrefillArgs p{};
  p.x = x;
  p.row_token = row_token;
  p.row_weight = row_weight;
  p.sorted_rows = sorted_rows;
  p.block_expert = block_expert;
  p.num_padded = num_padded;
  p.group_ptr = group_ptr;
  p.num_local = num_local;
  p.h_buf = h_buf;
  p.out_rows = out_rows;
  p.R = R;
  p.T = T;
  p.H = H;
  p.I = I;
  p.trace = g_trace;
  return hip_check(ss::launch_prefill_gemm(p, static_cast<hipStream_t>(stream)), "fused_moe_affine launch");
}

int ssmoe_combine_rank_order(const float* out_rows, int T, int K, int H, float* out, void* stream) {
  if (T < 0 || K < 1 || H < 4 || H % 4) return fail(SSMOE_EINVAL, "need T >= 0, K >= 1, H a multiple of 4");
  if (T > 0 && (!out_rows || !out)) return fail(SSMOE_EINVAL, "out_rows and out must be non-null");
  if (!aligned(out_rows, 16) || !aligned(out, 16)) return fail(SSMOE_EINVAL, "out_rows and out must be 16-byte aligned");
  return hip_check(ss::launch_combine(out_rows, nullptr, T, K, H, out, static_cast<hipStream_t>(stream)),
                   "combine launch");
}

// Workspace of ssmoe_moe_prefill: local [R], row_token [R], group_ptr [E] (8-byte), sorted_rows [P],
// block_expert [P / kPrefillBlockM], num_padded, then the moe_align scratch.
struct PrefillWs {
  int64_t local, row_token, gptr, sorted, bexp, npad, scratch, total;
};
static PrefillWs prefill_ws(int64_t T, int K, int E) {
  const int64_t R = T * K;
  const int64_t P = ss::padded_rows(R, E, ss::kPrefillBlockM);
  auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
  PrefillWs w{};
  int64_t o = 0;
  w.local = o;
  o = up(o + R * 4);
  w.row_token = o;
  o = up(o + R * 4);
  w.gptr = o;
  o = up(o + (int64_t)E * 8);
  w.sorted = o;
  o = up(o + P * 4);
  w.bexp = o;
  o = up(o + P / ss::kPrefillBlockM * 4);
  w.npad = o;
  o = up(o + 4);
  w.scratch = o;
  o = up(o + ss::align_scratch_ints(R, E) * 4);
  w.total = o;
  return w;
}

int64_t ssmoe_moe_prefill_workspace_bytes(int64_t T, int K, int E) {
  if (T < 0 || K < 1 || E < 1) return -1;
  return prefill_ws(T, K, E).total;
}

int ssmoe_moe_prefill(const uint16_t* x, const int32_t* expert_ids, const float* weights, int layer,
                      const int32_t* map, int64_t map_len, const int64_t* slot_ptr, int64_t n_slots, void* workspace,
                      int64_t workspace_bytes, uint16_t* h_buf, float* out_rows, float* out, int64_t T, int H, int I,
                      int K, int E, void* stream) {
  if (T < 0 || K < 1 || K > 64 || E < 1 || E > 4096) return fail(SSMOE_EINVAL, "need T >= 0, 1 <= K <= 64, 1 <= E <= 4096");
  if (int rc = check_prefill_shape(T * K, H, I)) return rc;
  if (layer < 0) return fail(SSMOE_EINVAL, "layer must be >= 0, got %d", layer);
  if ((int64_t)(layer + 1) * E > map_len)
    return fail(SSMOE_EINVAL, "map holds %lld entries, layer %d needs %lld", (long long)map_len, layer,
                (long long)(layer + 1) * E);
  if (T == 0) return ok();
  if (!x || !expert_ids || !weights || !map || !slot_ptr || !workspace || !h_buf || !out_rows || !out)
    return fail(SSMOE_EINVAL, "every pointer must be non-null");
  if (!aligned(x, 16) || !aligned(h_buf, 16) || !aligned(out_rows, 16) || !aligned(out, 16) ||
      !aligned(workspace, 256))
    return fail(SSMOE_EINVAL, "x, h_buf, out_rows, out 16-byte and workspace 256-byte aligned");
  const PrefillWs w = prefill_ws(T, K, E);
  if (workspace_bytes < w.total)
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes, (long long)w.total);
  int* err = nullptr;
  if (int rc = status_ptr(&err)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int32_t* local = reinterpret_cast<int32_t*>(ws + w.local);
  int32_t* row_token = reinterpret_cast<int32_t*>(ws + w.row_token);
  int64_t* gptr = reinterpret_cast<int64_t*>(ws + w.gptr);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + w.sorted);
  int32_t* bexp = reinterpret_cast<int32_t*>(ws + w.bexp);
  int32_t* npad = reinterpret_cast<int32_t*>(ws + w.npad);
  const int64_t R = T * K;
  if (int rc = hip_check(ss::launch_prefill_tables(map, (int64_t)layer * E, map_len, slot_ptr, n_slots, E, gptr,
                                                   expert_ids, R, K, local, row_token, err, st),
                         "prefill tables launch"))
    return rc;
  ss::AlignArgs al{};
  al.local_expert = local;
  al.R = R;
  al.num_local = E;
  al.block_m = ss::kPrefillBlockM;
  al.sorted_rows = sorted;
  al.block_expert = bexp;
  al.num_padded = npad;
  al.scratch = reinterpret_cast<int32_t*>(ws + w.scratch);
  if (int rc = hip_check(ss::launch_moe_align(al, st), "moe_align launch")) return rc;
  ss::PrefillArgs p{};
  p.x = x;
  p.row_token = row_token;
  p.row_weight = weights;
  p.sorted_rows = sorted;
  p.block_expert = bexp;
  p.num_padded = npad;
  p.group_ptr = gptr;
  p.num_local = E;
  p.h_buf = h_buf;
  p.out_rows = out_rows;
  p.R = R;
  p.T = (int)T;
  p.H = H;
  p.I = I;
  p.trace = g_trace;
  if (int rc = hip_check(ss::launch_prefill_gemm(p, st), "prefill gemm launch")) return rc;
  return hip_check(ss::launch_combine(out_rows, local, (int)T, K, H, out, st), "combine launch");
}

// ---------------------------------------------------------------- shared expert (prefill)
int ssmoe_shared_hs(const uint16_t* proj, int64_t ld, int T, int Is, uint16_t* hs, uint16_t* sgl, void* stream) {
  if (T < 0 || Is < 1 || ld < 2 * (int64_t)Is + 1)
    return fail(SSMOE_EINVAL, "need T >= 0, Is >= 1, ld >= 2 Is + 1 (T=%d Is=%d ld=%lld)", T, Is, (long long)ld);
  if (T > 0 && (!proj || !hs || !sgl)) return fail(SSMOE_EINVAL, "proj, hs and sgl must be non-null");
  return hip_check(ss::launch_shared_hs(proj, ld, T, Is, hs, sgl, static_cast<hipStream_t>(stream)),
                   "shared_hs launch");
}

int ssmoe_residual_rmsnorm(const uint16_t* resid, const uint16_t* y, const uint16_t* weight, float eps, int R, int H,
                           uint16_t* stream_out, uint16_t* mixed, void* stream) {
  if (!resid || !mixed || (y && !stream_out)) return fail(SSMOE_EINVAL, "resid and mixed (and stream_out with y) must be non-null");
  if (R < 0 || R > 65536 || H < 8 || H > 65536 || H % 8 != 0)
    return fail(SSMOE_EINVAL, "need 0 <= R <= 65536 and H a multiple of 8 in [8, 65536] (got R=%d H=%d)", R, H);
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(SSMOE_EINVAL, "eps must be finite and >= 0");
  if (!aligned(resid, 16) || !aligned(mixed, 16) || (y && !aligned(y, 16)) || (weight && !aligned(weight, 16)) ||
      (stream_out && !aligned(stream_out, 16)))
    return fail(SSMOE_EINVAL, "all rows must be 16-byte aligned");
  if (mixed == resid || mixed == y || mixed == stream_out || (y && (y == stream_out)))
    return fail(SSMOE_EINVAL, "mixed must not alias the stream, and y must not alias stream_out");
  return hip_check(ss::launch_residual_rmsnorm(resid, y, weight, eps, R, H, stream_out, mixed,
                                               static_cast<hipStream_t>(stream)),
                   "residual_rmsnorm launch");
}

int ssmoe_combine_shared(const float* routed, const uint16_t* sh, const uint16_t* sgl, uint16_t* y, int T, int H,
                         void* stream) {
  if (T < 0 || H < 4 || H % 4) return fail(SSMOE_EINVAL, "need T >= 0 and H a positive multiple of 4");
  if (T > 0 && (!routed || !sh || !sgl || !y)) return fail(SSMOE_EINVAL, "every pointer must be non-null");
  if (!aligned(routed, 16) || !aligned(sh, 8) || !aligned(y, 8))
    return fail(SSMOE_EINVAL, "routed must be 16-byte aligned, sh and y 8-byte aligned");
  return hip_check(ss::launch_combine_shared(routed, sh, sgl, y, T, H, static_cast<hipStream_t>(stream)),
                   "combine_shared launch");
}

// ---------------------------------------------------------------- reference sampler
int64_t ssmoe_sample_workspace_bytes(int V) {
  if (V < 1 || V > (1 << 20)) return -1;
  return ss::sample_workspace_bytes(V);
}

static int check_sample(int V, float temperature, float top_p, int top_k, float min_p, float presence_penalty,
                        const int32_t* generated, int n_generated, void* workspace, int64_t workspace_bytes,
                        int64_t rows) {
  if (V < 1 || V > (1 << 20)) return fail(SSMOE_EINVAL, "V must be in [1, 1048576], got %d", V);
  if (!(temperature >= 0.f) || temperature > 3.4e38f) return fail(SSMOE_EINVAL, "temperature must be finite and >= 0");
  if (!(top_p > 0.f && top_p <= 1.f)) return fail(SSMOE_EINVAL, "top_p must be in (0, 1], got %g", (double)top_p);
  if (!(min_p >= 0.f && min_p <= 1.f)) return fail(SSMOE_EINVAL, "min_p must be in [0, 1], got %g", (double)min_p);
  if (top_k < 0) return fail(SSMOE_EINVAL, "top_k must be >= 0, got %d", top_k);
  if (!(presence_penalty == presence_penalty) || presence_penalty > 3.4e38f || presence_penalty < -3.4e38f)
    return fail(SSMOE_EINVAL, "presence_penalty must be finite");
  if (n_generated < 0 || (n_generated > 0 && !generated))
    return fail(SSMOE_EINVAL, "generated must hold n_generated >= 0 token ids");
  if (!workspace) return fail(SSMOE_EINVAL, "workspace must be non-null");
  if (!aligned(workspace, 256)) return fail(SSMOE_EINVAL, "workspace must be 256-byte aligned");
  if (workspace_bytes < rows * ss::sample_workspace_bytes(V))
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)(rows * ss::sample_workspace_bytes(V)));
  return ok();
}

int ssmoe_sample(const float* logits, int V, const int32_t* generated, int n_generated, float temperature,
                 float top_p, int top_k, float min_p, float presence_penalty, const float* u, void* workspace,
                 int64_t workspace_bytes, int32_t* out, void* stream) {
  if (int rc = check_sample(V, temperature, top_p, top_k, min_p, presence_penalty, generated, n_generated, workspace,
                            workspace_bytes, 1))
    return rc;
  if (!logits || !u || !out) return fail(SSMOE_EINVAL, "logits, u and out must be non-null");
  return hip_check(ss::launch_sample(logits, V, generated, n_generated, temperature, top_p, top_k, min_p,
                                     presence_penalty, u, workspace, out, static_cast<hipStream_t>(stream)),
                   "sample launch");
}

int ssmoe_bench_stream_read(const void* src, int64_t bytes, uint32_t* out, int grid, void* stream) {
  if (!src || !out) return fail(SSMOE_EINVAL, "src and out must be non-null");
  if (!aligned(src, 16) || bytes < 16 || bytes % 16) return fail(SSMOE_EINVAL, "src must be 16-byte aligned and bytes a positive multiple of 16");
  if (grid < 1 || grid > (1 << 20)) return fail(SSMOE_EINVAL, "grid must be in [1, 1048576], got %d", grid);
  return hip_check(ss::launch_stream_read(src, (size_t)bytes, out, grid, static_cast<hipStream_t>(stream)),
                   "stream read launch");
}

int ssmoe_bench_mfma_bf16(const uint32_t* seed, int iters, float* out, int grid, void* stream) {
  if (!seed || !out) return fail(SSMOE_EINVAL, "seed and out must be non-null");
  if (iters < 1 || grid < 1 || grid > (1 << 20)) return fail(SSMOE_EINVAL, "iters >= 1 and grid in [1, 1048576]");
  return hip_check(ss::launch_mfma_loop(seed, iters, out, grid, static_cast<hipStream_t>(stream)), "mfma loop launch");
}

int ssmoe_bf16_round(const float* x, uint16_t* y, int64_t n, void* stream) {
  if (n < 0) return fail(SSMOE_EINVAL, "n must be >= 0, got %lld", (long long)n);
  if (n == 0) return SSMOE_OK;
  if (!x || !y) return fail(SSMOE_EINVAL, "x and y must be non-null");
  return hip_check(ss::launch_bf16_round(x, y, n, static_cast<hipStream_t>(stream)), "bf16 round launch");
}

int64_t ssmoe_sample_rows_workspace_bytes(int R, int V) {
  if (R < 1 || R > 64 || V < 1 || V > (1 << 20)) return -1;
  return ss::draw_work_floats(R, V) * 4;
}

int ssmoe_sample_rows(const float* logits, int R, int V, float temperature, const float* uniforms, void* workspace,
                      int64_t workspace_bytes, int32_t* tokens, void* stream) {
  if (R < 1 || R > 64) return fail(SSMOE_EINVAL, "R must be in [1, 64], got %d", R);
  if (V < 1 || V > (1 << 20)) return fail(SSMOE_EINVAL, "V must be in [1, 1048576], got %d", V);
  if (!(temperature > 0.f) || temperature > 3.4e38f)
    return fail(SSMOE_EINVAL, "temperature must be finite and > 0 (a proposal is drawn, not taken as the argmax)");
  if (!logits || !uniforms || !tokens || !workspace)
    return fail(SSMOE_EINVAL, "logits, uniforms, tokens and workspace must be non-null");
  if (!aligned(workspace, 256)) return fail(SSMOE_EINVAL, "workspace must be 256-byte aligned");
  if (workspace_bytes < ss::draw_work_floats(R, V) * 4)
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)(ss::draw_work_floats(R, V) * 4));
  int* err = nullptr;
  if (int rc = status_ptr(&err)) return rc;
  return hip_check(ss::launch_draw_rows(logits, R, V, temperature, uniforms, workspace, tokens, err,
                                        static_cast<hipStream_t>(stream)),
                   "sample rows launch");
}

int64_t ssmoe_accept_sampled_workspace_bytes(int D, int V) {
  if (D < 0 || D > 60 || V < 1 || V > (1 << 20)) return -1;
  return (int64_t)(D + 1) * ss::sample_workspace_bytes(V);
}

int ssmoe_accept_sampled(const float* target, const int32_t* drafts, int D, int V, const int32_t* seen, int n_seen,
                         float temperature, float top_p, int top_k, float min_p, float presence_penalty,
                         const float* uniforms, void* workspace, int64_t workspace_bytes, int32_t* out,
                         void* stream) {
  if (D < 0 || D > 60) return fail(SSMOE_EINVAL, "D must be in [0, 60], got %d", D);
  if (int rc = check_sample(V, temperature, top_p, top_k, min_p, presence_penalty, seen, n_seen, workspace,
                            workspace_bytes, D + 1))
    return rc;
  if (!target || !uniforms || !out || (D > 0 && !drafts))
    return fail(SSMOE_EINVAL, "target, drafts, uniforms and out must be non-null");
  return hip_check(ss::launch_accept_sampled(target, drafts, D, V, seen, n_seen, temperature, top_p, top_k, min_p,
                                             presence_penalty, uniforms, workspace, out,
                                             static_cast<hipStream_t>(stream)),
                   "accept sampled launch");
}

static int check_gemv(const void* x, int K, const int32_t* q, const uint16_t* s, const uint16_t* b, int N) {
  if (!ss::gemv_affine4_shape_ok(K)) return fail(SSMOE_EINVAL, "K must be 1024, 2048, 2560 or 4096, got %d", K);
  if (N < 1) return fail(SSMOE_EINVAL, "N must be >= 1, got %d", N);
  if (!x || !q || !s || !b) return fail(SSMOE_EINVAL, "x, q, s and b must be non-null");
  if (!aligned(x, 16) || !aligned(q, 16)) return fail(SSMOE_EINVAL, "x and q must be 16-byte aligned");
  if (!aligned(s, 4) || !aligned(b, 4)) return fail(SSMOE_EINVAL, "s and b must be 4-byte aligned");
  return ok();
}

int ssmoe_gemv_affine4(const void* x, int x_f32, int R, int K, const int32_t* q, const uint16_t* s, const uint16_t* b,
                       int N, float* y, void* stream) {
  if (R < 0) return fail(SSMOE_EINVAL, "R must be >= 0, got %d", R);
  if (int rc = check_gemv(x, K, q, s, b, N)) return rc;
  if (!y) return fail(SSMOE_EINVAL, "y must be non-null");
  if (R == 0) return ok();
  return hip_check(ss::launch_gemv_affine4(x, x_f32 ? 1 : 0, R, K, q, s, b, N, y, static_cast<hipStream_t>(stream)),
                   "gemv launch");
}

int64_t ssmoe_lm_head_greedy_workspace_bytes(int D, int N) {
  if (D < 0 || D > 60 || N < 1) return -1;
  return ss::lm_head_greedy_workspace_bytes(D, N);
}

int ssmoe_lm_head_greedy(const void* x, int x_f32, int D, int K, const int32_t* q, const uint16_t* s,
                         const uint16_t* b, int N, const int32_t* drafts, void* workspace, int64_t workspace_bytes,
                         float* logits, int32_t* out, void* stream) {
  if (D < 0 || D > 60) return fail(SSMOE_EINVAL, "D must be in [0, 60], got %d", D);
  if (int rc = check_gemv(x, K, q, s, b, N)) return rc;
  if (!out || (D > 0 && !drafts)) return fail(SSMOE_EINVAL, "drafts and out must be non-null");
  if (!workspace || !aligned(workspace, 256)) return fail(SSMOE_EINVAL, "workspace must be non-null and 256-byte aligned");
  if (workspace_bytes < ss::lm_head_greedy_workspace_bytes(D, N))
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)ss::lm_head_greedy_workspace_bytes(D, N));
  return hip_check(ss::launch_lm_head_greedy(x, x_f32 ? 1 : 0, D, K, q, s, b, N, drafts, workspace, logits, out,
                                             static_cast<hipStream_t>(stream)),
                   "lm_head greedy launch");
}

int64_t ssmoe_lm_head_pq_workspace_bytes(int D, int N) {
  if (D < 0 || D > 3 || N < 1 || N > (1 << 20)) return -1;
  return ss::lm_head_pq_workspace_bytes(D, N);
}

int ssmoe_lm_head_pq(const void* x, int x_f32, int D, int K, const int32_t* q, const uint16_t* s, const uint16_t* b,
                     int N, const float* draft, const int32_t* drafts, const float* uniforms, float temperature,
                     void* workspace, int64_t workspace_bytes, float* logits, int32_t* out, void* stream) {
  if (D < 0 || D > 3) return fail(SSMOE_EINVAL, "D must be in [0, 3], got %d", D);
  if (N > (1 << 20)) return fail(SSMOE_EINVAL, "N must be <= 1048576, got %d", N);
  if (int rc = check_gemv(x, K, q, s, b, N)) return rc;
  if (!logits || !out || !uniforms || (D > 0 && (!draft || !drafts)))
    return fail(SSMOE_EINVAL, "logits, out, uniforms, draft and drafts must be non-null");
  if (!(temperature > 0.f) || temperature != temperature)
    return fail(SSMOE_EINVAL, "temperature must be > 0, got %g", (double)temperature);
  if (!workspace || !aligned(workspace, 256)) return fail(SSMOE_EINVAL, "workspace must be non-null and 256-byte aligned");
  if (workspace_bytes < ss::lm_head_pq_workspace_bytes(D, N))
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)ss::lm_head_pq_workspace_bytes(D, N));
  int* err = nullptr;
  if (int rc = status_ptr(&err)) return rc;
  return hip_check(ss::launch_lm_head_pq(x, x_f32 ? 1 : 0, D, K, q, s, b, N, draft, drafts, uniforms, temperature,
                                         workspace, logits, out, err, static_cast<hipStream_t>(stream)),
                   "lm_head p/q launch");
}

int64_t ssmoe_lm_head_argmax_workspace_bytes(int R, int N) {
  if (R < 1 || R > 64 || N < 1) return -1;
  return ss::lm_head_greedy_workspace_bytes(R - 1, N);
}

int ssmoe_lm_head_argmax(const void* x, int x_f32, int R, int K, const int32_t* q, const uint16_t* s,
                         const uint16_t* b, int N, int round_bf16, void* workspace, int64_t workspace_bytes,
                         float* logits, int32_t* ids, void* stream) {
  if (R < 1 || R > 64) return fail(SSMOE_EINVAL, "R must be in [1, 64], got %d", R);
  if (int rc = check_gemv(x, K, q, s, b, N)) return rc;
  if (!ids) return fail(SSMOE_EINVAL, "ids must be non-null");
  if (!workspace || !aligned(workspace, 256)) return fail(SSMOE_EINVAL, "workspace must be non-null and 256-byte aligned");
  if (workspace_bytes < ss::lm_head_greedy_workspace_bytes(R - 1, N))
    return fail(SSMOE_EINVAL, "workspace holds %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)ss::lm_head_greedy_workspace_bytes(R - 1, N));
  return hip_check(ss::launch_lm_head_argmax(x, x_f32 ? 1 : 0, R, K, q, s, b, N, round_bf16, workspace, logits, ids,
                                             static_cast<hipStream_t>(stream)),
                   "lm_head argmax launch");
}

int ssmoe_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int R, int n, int group, uint16_t* out,
                  void* stream) {
  if (R < 0 || n < 8 || group < 8 || group % 8 || n % group)
    return fail(SSMOE_EINVAL, "need R >= 0 and group a multiple of 8 dividing n (R %d, n %d, group %d)", R, n, group);
  if (!x || !out) return fail(SSMOE_EINVAL, "x and out must be non-null");
  if (!aligned(x, 16) || !aligned(out, 16) || (w && !aligned(w, 16)))
    return fail(SSMOE_EINVAL, "x, w and out must be 16-byte aligned");
  if (x == out) return fail(SSMOE_EINVAL, "out must not alias x");
  if (!(eps >= 0.f)) return fail(SSMOE_EINVAL, "eps must be >= 0");
  return hip_check(ss::launch_rmsnorm_groups(x, w, eps, R, n, group, out, static_cast<hipStream_t>(stream)),
                   "rmsnorm launch");
}

int ssmoe_dense_gemv_epi(const uint16_t* x, int R, int K, const uint16_t* w, int N, int epi, int hc,
                         const uint16_t* add, int add_div, uint16_t* out, void* stream) {
  if (R < 0 || K < 8 || K % 8 || N < 1) return fail(SSMOE_EINVAL, "need R >= 0, K a multiple of 8, N >= 1");
  if (epi < SSMOE_EPI_NONE || epi > SSMOE_EPI_INJECT) return fail(SSMOE_EINVAL, "unknown epilogue %d", epi);
  if ((epi == SSMOE_EPI_SILU_DIV || epi == SSMOE_EPI_INJECT) && hc < 1) return fail(SSMOE_EINVAL, "hc must be >= 1");
  if (epi == SSMOE_EPI_ADD && (!add || add_div < 1)) return fail(SSMOE_EINVAL, "EPI_ADD needs add and add_div >= 1");
  if (!x || !w || !out) return fail(SSMOE_EINVAL, "x, w and out must be non-null");
  if (!aligned(x, 16) || !aligned(w, 16)) return fail(SSMOE_EINVAL, "x and w must be 16-byte aligned");
  return hip_check(ss::launch_dense_epi(x, R, K, w, N, epi, hc, add, add_div, out, static_cast<hipStream_t>(stream)),
                   "dense gemv launch");
}

int ssmoe_head_gemv(const ssmoe_head_gemv_args* p, void* stream) {
  if (!p) return fail(SSMOE_EINVAL, "args must be non-null");
  const ssmoe_head_gemv_args& a = *p;
  if (a.S < 0 || a.n < 8 || a.K < 8 || a.n % 8 || a.K % 8 || a.n % a.K)
    return fail(SSMOE_EINVAL, "need S >= 0, n and K multiples of 8, n a multiple of K (n=%d K=%d)", a.n, a.K);
  if (a.n > 32768 || (a.n / a.K) > 4) return fail(SSMOE_EINVAL, "need n <= 32768 and n / K <= 4");
  if (a.group < 0 || (a.group > 0 && (a.n % a.group || a.group % 8)))
    return fail(SSMOE_EINVAL, "group must be 0 (no norm) or a multiple of 8 dividing n, got %d", a.group);
  if (a.group > 0 && a.n / a.group > 64)
    return fail(SSMOE_EINVAL, "at most 64 norm groups per row, got n %d, group %d", a.n, a.group);
  if (a.N < 1 || a.N2 < 0) return fail(SSMOE_EINVAL, "need N >= 1 and N2 >= 0");
  for (int e : {a.epi, a.epi2})
    if (e < SSMOE_EPI_NONE || e > SSMOE_EPI_INJECT) return fail(SSMOE_EINVAL, "unknown epilogue %d", e);
  if ((a.epi == SSMOE_EPI_SILU_DIV || a.epi == SSMOE_EPI_INJECT || a.epi2 == SSMOE_EPI_SILU_DIV ||
       a.epi2 == SSMOE_EPI_INJECT) && a.hc < 1)
    return fail(SSMOE_EINVAL, "hc must be >= 1");
  if (a.epi == SSMOE_EPI_ADD && (!a.add || a.add_div < 1)) return fail(SSMOE_EINVAL, "EPI_ADD needs add, add_div >= 1");
  if (a.epi2 == SSMOE_EPI_ADD) return fail(SSMOE_EINVAL, "the second weight range takes no EPI_ADD");
  if (!a.src || !a.w || !a.out || (a.N2 > 0 && (!a.w2 || !a.out2)))
    return fail(SSMOE_EINVAL, "src, w and out (and w2, out2 with N2 > 0) must be non-null");
  if (a.inj && (!a.inj_y || a.inj_hc < 1 || a.n % a.inj_hc || (a.n / a.inj_hc) % 8))
    return fail(SSMOE_EINVAL, "the injection needs inj_y and inj_hc dividing n into multiples of 8");
  if (a.mean_out && (!a.mean_hn || a.hc != 4 || a.N % 4 || a.N2 > 0 || a.n != a.K || a.K > 512))
    return fail(SSMOE_EINVAL, "the fused mean needs mean_hn, hc == 4, N a multiple of 4, no w2 and n == K <= 512");
  if (a.src_idx && a.n_src < 1) return fail(SSMOE_EINVAL, "a table source needs n_src >= 1");
  if (!aligned(a.src, 16) || !aligned(a.w, 16) || (a.w2 && !aligned(a.w2, 16)) || (a.norm_w && !aligned(a.norm_w, 16)) ||
      (a.inj_y && !aligned(a.inj_y, 16)) || (a.h_out && !aligned(a.h_out, 16)) || (a.x_out && !aligned(a.x_out, 16)))
    return fail(SSMOE_EINVAL, "src, w, w2, norm_w, inj_y, h_out and x_out must be 16-byte aligned");
  if (a.S == 0) return ok();
  int* err = nullptr;
  if (int rc = status_ptr(&err)) return rc;
  ss::HeadGemvIn in{};
  in.src = a.src;
  in.src_idx = a.src_idx;
  in.n_src = a.n_src;
  in.inj_y = a.inj ? a.inj_y : nullptr;
  in.inj = a.inj;
  in.inj_hc = a.inj ? a.inj_hc : 1;
  in.norm_w = a.norm_w;
  in.eps = a.eps;
  in.G = a.group;
  in.S = a.S;
  in.n = a.n;
  in.K = a.K;
  in.w = a.w;
  in.N = a.N;
  in.epi = a.epi;
  in.hc = a.hc;
  in.add = a.add;
  in.add_div = a.add_div;
  in.out = a.out;
  in.w2 = a.w2;
  in.N2 = a.N2;
  in.epi2 = a.epi2;
  in.out2 = a.out2;
  in.h_out = a.h_out;
  in.x_out = a.x_out;
  in.mean_hn = a.mean_hn;
  in.mean_out = a.mean_out;
  in.mean_H = a.N / 4;
  in.err = err;
  in.trace = g_trace;
  return hip_check(ss::launch_head_gemv(in, static_cast<hipStream_t>(stream)), "head gemv launch");
}

int ssmoe_hc_mean(const uint16_t* m, const uint16_t* hn, int S, int hc, int H, uint16_t* mixed, void* stream) {
  if (S < 0 || hc < 1 || H < 1) return fail(SSMOE_EINVAL, "need S >= 0, hc >= 1, H >= 1");
  if (!m || !hn || !mixed) return fail(SSMOE_EINVAL, "m, hn and mixed must be non-null");
  return hip_check(ss::launch_hc_mean(m, hn, S, hc, H, mixed, static_cast<hipStream_t>(stream)), "hc_mean launch");
}

int ssmoe_hc_inject(const uint16_t* hyp, const uint16_t* y, const uint16_t* inj, int S, int hc, int H, uint16_t* out,
                    void* stream) {
  if (S < 0 || hc < 1 || H < 1) return fail(SSMOE_EINVAL, "need S >= 0, hc >= 1, H >= 1");
  if (!hyp || !y || !inj || !out) return fail(SSMOE_EINVAL, "hyp, y, inj and out must be non-null");
  return hip_check(ss::launch_hc_inject(hyp, y, inj, S, hc, H, out, static_cast<hipStream_t>(stream)),
                   "hc_inject launch");
}

int ssmoe_gather_rows(const void* src, int64_t n_src, int64_t row_bytes, const int32_t* idx, int n, int idx_add,
                      void* dst, void* stream) {
  if (n < 0 || n_src < 1 || row_bytes < 4 || row_bytes % 4)
    return fail(SSMOE_EINVAL, "need n >= 0, n_src >= 1 and row_bytes a positive multiple of 4");
  if (!src || !idx || !dst) return fail(SSMOE_EINVAL, "src, idx and dst must be non-null");
  if (!aligned(src, 4) || !aligned(dst, 4)) return fail(SSMOE_EINVAL, "src and dst must be 4-byte aligned");
  int* st = nullptr;
  if (int rc = status_ptr(&st)) return rc;
  return hip_check(ss::launch_gather_rows(src, n_src, row_bytes, idx, n, idx_add, dst, st,
                                          static_cast<hipStream_t>(stream)),
                   "gather launch");
}

int ssmoe_pool_open(const char* experts_path, int layers, int experts, int64_t record_bytes, int max_slots,
                    int64_t chunk_bytes, int32_t* map, int64_t* slot_ptr, void** pool) {
  if (!experts_path || !map || !slot_ptr || !pool) return fail(SSMOE_EINVAL, "path, map, slot_ptr and pool must be non-null");
  if (layers < 1 || experts < 1 || (int64_t)layers * experts > (1LL << 30))
    return fail(SSMOE_EINVAL, "need layers >= 1, experts >= 1, layers * experts <= 2^30 (got %d x %d)", layers, experts);
  if (record_bytes < 1 || max_slots < 0 || chunk_bytes < record_bytes)
    return fail(SSMOE_EINVAL, "need record_bytes >= 1, max_slots >= 0, chunk_bytes >= record_bytes");
  if (!aligned(slot_ptr, 8) || !aligned(map, 4)) return fail(SSMOE_EINVAL, "map / slot_ptr misaligned");
  ss::Pool* p = nullptr;
  std::string err;
  hipError_t e = ss::pool_open(experts_path, layers, experts, record_bytes, max_slots, chunk_bytes, map, slot_ptr, &p, &err);
  if (e == hipErrorFileNotFound) return fail(SSMOE_EIO, "%s", err.c_str());
  if (e != hipSuccess) return fail(SSMOE_EHIP, "%s: %s", err.c_str(), hipGetErrorString(e));
  *pool = p;
  return ok();
}

int ssmoe_pool_close(void* pool) {
  ss::pool_close(static_cast<ss::Pool*>(pool));
  return ok();
}

int ssmoe_pool_set_reader(void* pool, int lanes, int direct) {
  if (!pool) return fail(SSMOE_EINVAL, "pool must be non-null");
  std::string err;
  hipError_t e = ss::pool_set_reader(static_cast<ss::Pool*>(pool), lanes, direct != 0, &err);
  if (e == hipErrorInvalidValue) return fail(SSMOE_EINVAL, "%s", err.c_str());
  if (e == hipErrorFileNotFound) return fail(SSMOE_EIO, "%s", err.c_str());
  return hip_check(e, "pool reader set-up");
}

int ssmoe_pool_resize(void* pool, int slots) {
  if (!pool) return fail(SSMOE_EINVAL, "pool must be non-null");
  std::string err;
  hipError_t e = ss::pool_resize(static_cast<ss::Pool*>(pool), slots, &err);
  if (e == hipErrorInvalidValue) return fail(SSMOE_EINVAL, "%s", err.c_str());
  if (e != hipSuccess) return fail(SSMOE_EHIP, "pool resize: %s %s", err.c_str(), hipGetErrorString(e));
  return ok();
}

int ssmoe_pool_ensure(void* pool, int layer, const int32_t* experts, int n, uint64_t gen, int32_t* slots,
                      int64_t* timing) {
  if (!pool || n < 0 || (n > 0 && (!experts || !slots)))
    return fail(SSMOE_EINVAL, "pool, experts and slots must be non-null, n >= 0");
  std::string err;
  ss::EnsureTiming t{};
  const ss::PoolStatus st = ss::pool_ensure(static_cast<ss::Pool*>(pool), layer, experts, n, gen, slots, &t, &err);
  if (timing) {
    const int64_t v[6] = {t.hits, t.misses, t.bytes, t.total_ns, t.read_ns, t.copy_ns};
    for (int k = 0; k < 6; ++k) timing[k] = v[k];
  }
  switch (st) {
    case ss::PoolStatus::Ok: return ok();
    case ss::PoolStatus::Invalid: return fail(SSMOE_EINVAL, "%s", err.c_str());
    case ss::PoolStatus::Exhausted: return fail(SSMOE_EXHAUSTED, "%s", err.c_str());
    default: return fail(SSMOE_EIO, "%s", err.c_str());
  }
}

int ssmoe_pool_retire_below(void* pool, uint64_t progress) {
  if (!pool) return fail(SSMOE_EINVAL, "pool must be non-null");
  ss::pool_retire_below(static_cast<ss::Pool*>(pool), progress);
  return ok();
}

int ssmoe_pool_set_progress(void* pool, const uint64_t* progress) {
  if (!pool) return fail(SSMOE_EINVAL, "pool must be non-null");
  ss::pool_set_progress(static_cast<ss::Pool*>(pool), progress);
  return ok();
}

int ssmoe_pool_copy_slot(void* pool, int slot, void* dst, int64_t bytes) {
  if (!pool || !dst) return fail(SSMOE_EINVAL, "pool and dst must be non-null");
  std::string err;
  hipError_t e = ss::pool_copy_slot(static_cast<ss::Pool*>(pool), slot, dst, bytes, &err);
  if (e == hipErrorInvalidValue) return fail(SSMOE_EINVAL, "%s", err.c_str());
  return hip_check(e, "pool slot copy");
}

int ssmoe_pool_stats(void* pool, int64_t* stats) {
  if (!pool || !stats) return fail(SSMOE_EINVAL, "pool and stats must be non-null");
  ss::PoolStats s{};
  ss::pool_info(static_cast<ss::Pool*>(pool), &s);
  const int64_t v[10] = {s.slots, s.chunks, s.pinned, s.owned_bytes, s.stride, s.hits, s.misses, s.bytes,
                         s.lanes, s.direct};
  for (int k = 0; k < 10; ++k) stats[k] = v[k];
  return ok();
}

}  // extern "C"

