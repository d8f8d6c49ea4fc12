// Host-side status plumbing shared by every entry point.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/qstore_hip.h"

namespace qs {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return QS_OK;
  snprintf(g_last_error, sizeof(g_last_error), "%s: %s", what, hipGetErrorString(e));
  return QS_ERR_HIP;
}

}  // namespace qs

extern "C" int qs_version(void) { return 100; }

extern "C" const char* qs_last_error(void) { return qs::g_last_error; }
