// Error state and small host utilities behind the C ABI.
#include <atomic>
#include <cstdarg>
#include <cstdio>

#include "dmla_host.h"

namespace dmla {

namespace {
thread_local char g_msg[512] = {0};
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_msg[0] = 0; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DMLA_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return DMLA_OK;
}

int device_cu_count() {
  // Per device, filled on first use; threads that race there store the same value.
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace dmla

extern "C" int dmla_version(void) { return 100; /* 0.1.0 */ }

extern "C" const char* dmla_last_error(void) { return dmla::g_msg; }
