// Error state and version of the C ABI (include/trnsparse_hip.h).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace tsp {

static thread_local char g_err[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return TSP_OK;
  return fail(TSP_EHIP, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

}  // namespace tsp

extern "C" int tsp_version(void) { return 100; }

extern "C" const char* tsp_last_error(void) { return tsp::g_err; }
