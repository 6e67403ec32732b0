// capi.hip -- error reporting shared by the libtpo_hip entry points.
#include <stdarg.h>
#include <stdio.h>

#include "tpo_common.hpp"

namespace tpo {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(TPO_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return TPO_OK;
}

}  // namespace tpo

extern "C" const char* tpo_last_error(void) { return tpo::g_err; }

extern "C" int tpo_abi_version(void) { return (2 << 16) | 4; }
