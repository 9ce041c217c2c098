// Thread-local error message and the two trivial exports.
#include <stdarg.h>
#include <stdio.h>

#include "flw_common.h"

namespace flw {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FLW_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return FLW_OK;
}

}  // namespace flw

extern "C" const char* flw_last_error(void) { return flw::g_last_error; }
extern "C" int flw_abi_version(void) { return FLW_ABI_VERSION; }
