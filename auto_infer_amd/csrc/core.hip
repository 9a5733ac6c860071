// Error reporting and version of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace aia {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return AIA_OK;
  return fail(AIA_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

}  // namespace aia

extern "C" int aia_version(void) { return 100; }

extern "C" const char* aia_last_error(void) { return aia::g_last_error; }
