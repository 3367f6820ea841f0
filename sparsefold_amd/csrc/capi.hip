// C-ABI plumbing: version, thread-local error messages, launch checks, occupancy queries.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "sf_common.h"

namespace {
thread_local char g_err[1024] = {0};
}

void sf_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int sf_check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    sf_set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return 2;
  }
  return 0;
}

int sf_resident_workgroups(const void* kernel, int threads) {
  static std::mutex mu;
  static std::map<std::tuple<int, const void*, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  const auto key = std::make_tuple(dev, kernel, threads);
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess) per_cu = 1;
  const int n = (cus > 0 ? cus : 1) * (per_cu > 0 ? per_cu : 1);
  std::lock_guard<std::mutex> lock(mu);
  cache[key] = n;
  return n;
}

extern "C" int sf_hip_abi_version(void) { return SF_HIP_ABI_VERSION; }

extern "C" size_t sf_hip_last_error(char* buf, size_t n) {
  const size_t len = strlen(g_err);
  if (buf != nullptr && n > 0) {
    const size_t c = len < n - 1 ? len : n - 1;
    memcpy(buf, g_err, c);
    buf[c] = 0;
  }
  return len;
}
