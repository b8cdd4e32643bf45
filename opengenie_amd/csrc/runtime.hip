// Library identification, argument-error reporting and device queries.
#include <stdarg.h>
#include <atomic>
#include <stdio.h>

#include "host.h"

namespace oga {

static thread_local char g_err[512] = "";

static int vfail(int code, const char* fmt, va_list ap) {
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  return code;
}

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  int r = vfail(OGA_EINVAL, fmt, ap);
  va_end(ap);
  return r;
}

int unsupported(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  int r = vfail(OGA_EUNSUPPORTED, fmt, ap);
  va_end(ap);
  return r;
}

// Per-device cache; callers on several threads may fill an entry at once
// (with the same value), hence the relaxed atomics.
int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace oga

extern "C" int oga_abi_version(void) { return 1; }

extern "C" const char* oga_last_error(void) { return oga::g_err; }
