// Achievable-peak kernels of this build, the ceilings the roofline fractions are also stated against (beside the
// published MI355X peaks): a streaming read of a large buffer (HBM read bandwidth with this library's load forms)
// and a loop of independent bf16 MFMAs (the dense bf16 matrix-core rate with this library's MFMA form). Method of the
// reference's achievable-peak micro-benchmarks (bench/m0/gemv_bench.py:228-268): time a kernel that does nothing but
// the bound operation.
#include "ss_common.hpp"
#include "ss_launch.hpp"

namespace ss {

namespace {

// Every thread reads 16-byte words in a grid-stride loop, 8 loads in flight per round, and folds them with xor into
// one word per workgroup (so that no load can be dropped).
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ src, size_t n16, uint32_t* out) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 7 * stride < n16; i += 8 * stride) {
    uint4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = ldg16(src + i + k * stride);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = ldg16(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  acc = ss_wave_or(acc);
  if ((threadIdx.x & 63) == 0) atomicXor(out + blockIdx.x, acc);
}

// Each wave runs `iters` rounds of 8 independent v_mfma_f32_16x16x32_bf16 on register operands (the verify and
// prefill kernels' MFMA form); the accumulators are summed into one word per wave at the end.
__global__ __launch_bounds__(256) void mfma_loop_kernel(const uint32_t* __restrict__ seed, int iters, float* out) {
  const int lane = threadIdx.x & 63;
  ss_u32x4 a, b;
  a.x = seed[lane & 7];
  a.y = seed[(lane + 1) & 7];
  a.z = seed[(lane + 2) & 7];
  a.w = seed[(lane + 3) & 7];
  b.x = seed[(lane + 4) & 7];
  b.y = seed[(lane + 5) & 7];
  b.z = seed[(lane + 6) & 7];
  b.w = seed[(lane + 7) & 7];
  ss_f32x4 acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = ss_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = ss_mfma(a, b, acc[k]);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += acc[k].x + acc[k].y + acc[k].z + acc[k].w;
  s = ss_wave_sum(s);
  if (lane == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = s;
}

// y[i] = ss_f32_to_bf16(x[i]): the rounding every kernel of the library applies, exported so that tests can hold it
// to the reference's rule (round to nearest even; NaN: the top bits with the quiet bit set) on any bit pattern.
__global__ __launch_bounds__(256) void bf16_round_kernel(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                         int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) y[i] = (uint16_t)ss_f32_to_bf16(x[i]);
}

}  // namespace

hipError_t launch_bf16_round(const float* x, uint16_t* y, int64_t n, hipStream_t st) {
  const int64_t blocks = (n + 255) / 256;
  const int grid = (int)(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
  hipLaunchKernelGGL(bf16_round_kernel, dim3(grid), dim3(256), 0, st, x, y, n);
  return hipGetLastError();
}

hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* out, int grid, hipStream_t st) {
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(256), 0, st, static_cast<const uint4*>(src), bytes / 16, out);
  return hipGetLastError();
}

hipError_t launch_mfma_loop(const uint32_t* seed, int iters, float* out, int grid, hipStream_t st) {
  hipLaunchKernelGGL(mfma_loop_kernel, dim3(grid), dim3(256), 0, st, seed, iters, out);
  return hipGetLastError();
}

}  // namespace ss
