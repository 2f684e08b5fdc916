// Library-wide C ABI helpers: per-thread error message, version, device properties.
#include <stdarg.h>
#include <atomic>
#include <mutex>
#include <set>
#include <stdio.h>
#include <tuple>

#include "mfd_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

int mfd_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int mfd_set_hip_error(hipError_t e) {
  return mfd_set_error(MFD_ERR_HIP, "HIP error %d: %s", (int)e, hipGetErrorString(e));
}

extern "C" const char* mfd_last_error(void) { return g_last_error; }

extern "C" int mfd_version(void) { return 1; }

int mfd_num_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int mfd_set_max_lds(const void* fn, int bytes) {
  static std::mutex mu;
  static std::set<std::tuple<int, const void*, int>> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(dev, fn, bytes);
  if (done.count(key)) return MFD_OK;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return mfd_set_hip_error(e);
  done.insert(key);
  return MFD_OK;
}
