// C-ABI plumbing: version, thread-local error messages, launch checks.
#include <cstdarg>
#include <cstdio>
#include <cstring>

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
