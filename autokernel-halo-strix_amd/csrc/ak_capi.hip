// C-ABI plumbing: per-thread error message, launch checking, version query.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "mfma_ring.h"

namespace {
thread_local char g_last_error[512] = "";
}

int ak_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int ak_check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return ak_set_error(AK_ERR_LAUNCH, "%s: kernel launch failed: %s", what,
                        hipGetErrorString(err));
  }
  return AK_OK;
}

extern "C" const char* ak_last_error(void) { return g_last_error; }

extern "C" int ak_abi_version(void) { return AK_ABI_VERSION; }

extern "C" const char* ak_target_arch(void) { return "gfx950"; }

namespace ak {

// The cache entries are atomics: concurrent first calls may both query the
// attribute, but they store the same value and no caller reads a torn entry.
int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace ak
