// Error state and small C-ABI entry points of libnanopd_hip.so.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <string>

#include "common.h"

namespace {
thread_local std::string g_last_error;
}

namespace npd {

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error.assign(buf);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NPD_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return NPD_OK;
}

int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];   // 0: not queried yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < kMaxDevices) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  if (dev < kMaxDevices) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace npd

extern "C" const char* npd_last_error(void) { return g_last_error.c_str(); }

extern "C" int npd_version(void) { return 100; }
