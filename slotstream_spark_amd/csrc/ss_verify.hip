// The verify kernel's instantiations with a bf16 shared expert, the launch dispatch, and the scratch layout size.
// The kernel itself and its phases are described in ss_verify_kernel.hpp; the affine 4-bit shared-expert
// instantiations are compiled in ss_verify_q4.hip (a translation unit of their own, so the two build in parallel).
#include "ss_verify_kernel.hpp"

namespace ss {

size_t verify_scratch_bytes(int T, int H, int I, int Is, int K, int E) {
  return vlayout(T, H, I, Is, K, E).total;
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
  return a.x_f32 ? launch_nj<NJG, NJD, true, false>(a, st) : launch_nj<NJG, NJD, false, false>(a, st);
}

hipError_t launch_verify(const VerifyArgs& a, hipStream_t st) {
  // Shapes with instantiated kernels: H in {1024, 2048, 2560, 4096} x I in {128, 256, 512, 640, 1024}.
  if (a.mode == 0 && a.sh_gs) return launch_verify_q4(a, st);
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
