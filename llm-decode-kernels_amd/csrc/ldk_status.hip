// Thread-local error reporting and version query of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "ldk_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace ldk {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LDK_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return LDK_OK;
}

}  // namespace ldk

extern "C" int ldk_abi_version(void) { return LDK_ABI_VERSION; }

extern "C" const char* ldk_last_error(void) { return g_last_error; }
