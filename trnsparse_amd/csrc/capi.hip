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

__global__ __launch_bounds__(256) void zero_fill_kernel(uint8_t* __restrict__ p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0;
}

int zero_fill(void* p, int64_t bytes, hipStream_t st) {
  if (bytes <= 0) return TSP_OK;
  int64_t grid = ceil_div(bytes, 256);
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)grid), dim3(256), 0, st, (uint8_t*)p, bytes);
  return check_launch("zero_fill launch");
}

}  // namespace tsp

extern "C" int tsp_version(void) { return 100; }

extern "C" const char* tsp_last_error(void) { return tsp::g_err; }
