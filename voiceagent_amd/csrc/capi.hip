// Error channel and version query of the C ABI.
#include <stdarg.h>
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

}  // namespace va

extern "C" const char* va_last_error(void) { return va::g_last_error; }

extern "C" int va_abi_version(void) { return VA_ATTN_ABI_VERSION; }
