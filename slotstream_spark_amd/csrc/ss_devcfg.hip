// Per-device launch configuration of the library's kernels (declared in ss_launch.hpp).
#include <mutex>
#include <map>
#include <utility>

#include "ss_launch.hpp"

namespace ss {

hipError_t kernel_cfg(const void* kern, int threads, size_t max_dyn, KernelCfg* out) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, KernelCfg> cache;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find({dev, kern});
  if (it != cache.end() && it->second.max_dyn >= max_dyn && it->second.threads == threads) {
    *out = it->second;
    return hipSuccess;
  }
  KernelCfg c{};
  c.threads = threads;
  c.max_dyn = max_dyn;
  hipFuncAttributes attr;
  e = hipFuncGetAttributes(&attr, kern);
  if (e != hipSuccess) return e;
  c.lds_static = attr.sharedSizeBytes;
  if (max_dyn > 0) {
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_dyn);
    if (e != hipSuccess) return e;
  }
  e = hipDeviceGetAttribute(&c.cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&c.per_cu, kern, threads, max_dyn);
  if (e != hipSuccess) return e;
  cache[{dev, kern}] = c;
  *out = c;
  return hipSuccess;
}

}  // namespace ss
