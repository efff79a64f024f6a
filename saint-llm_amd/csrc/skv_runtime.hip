// Error state and version query of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "skv_common.h"

namespace skv {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(SKV_EHIP, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
  }
  return SKV_OK;
}

}  // namespace skv

extern "C" int skv_abi_version(void) { return SKV_ABI_VERSION; }

extern "C" const char* skv_last_error(void) { return skv::g_last_error; }
