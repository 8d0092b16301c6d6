// Library-wide C ABI pieces: thread-local error reporting and the version.
#include <stdarg.h>
#include <stdio.h>

#include "skv_common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace skv {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// Reports a failed launch (bad configuration, missing code object) as
// SKV_E_HIP. Kernel faults surface asynchronously at the next synchronising
// call, as for any HIP launch.
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SKV_E_HIP, "%s: %s", what, hipGetErrorString(e));
  return SKV_OK;
}

}  // namespace skv

extern "C" const char* skv_last_error(void) { return g_err; }

extern "C" int skv_version(void) { return 100; }
