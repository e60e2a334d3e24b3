// Library-wide state of the C ABI: the thread-local error string and the version.
#include <stdarg.h>
#include <stdio.h>

#include "i8l_common.h"

namespace i8l {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return I8L_OK;
  set_error("%s: %s (%s)", where, hipGetErrorString(e), hipGetErrorName(e));
  return I8L_HIP_ERROR;
}

}  // namespace i8l

extern "C" const char* i8l_last_error(void) { return i8l::g_err; }

extern "C" const char* i8l_version(void) { return "int8_linear_amd 0.1.0 gfx950"; }
