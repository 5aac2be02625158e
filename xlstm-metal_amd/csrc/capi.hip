// Library-wide C-ABI entry points: version and per-thread error message.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace xl {

static thread_local char g_last_error[512] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(XL_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return XL_OK;
}

}  // namespace xl

extern "C" int xl_abi_version(void) { return XL_ABI_VERSION; }

extern "C" const char* xl_last_error(void) { return xl::g_last_error; }
