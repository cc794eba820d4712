// Error channel and version query of the C ABI.
#include <stdarg.h>
#include <atomic>
#include <stdio.h>

#include "common.h"

namespace va {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return VA_ERR_LAUNCH;
  }
  return VA_OK;
}

// Compute units of the current device (cached per device; 256, the MI355X
// count, when no device is visible, e.g. when only the workspace size is
// queried on a host without a GPU).
int current_device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return 256;
  }
  if (dev < 64) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n <= 0) {
    (void)hipGetLastError();
    n = 256;
  }
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace va

extern "C" const char* va_last_error(void) { return va::g_last_error; }

extern "C" int va_abi_version(void) { return VA_ATTN_ABI_VERSION; }
