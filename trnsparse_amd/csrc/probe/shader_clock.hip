// Shader-clock probe for the benchmark (not part of the C ABI of
// include/trnsparse_hip.h; built as its own libtrnsparse_clock.so).
//
// One wave spins for a fixed span of the 100 MHz real-time counter
// (s_memrealtime) and records how many shader-clock cycles (s_memtime)
// passed meanwhile. Launched on a side stream while a train of kernels runs
// on the main stream, the ratio is the shader clock those kernels ran at.
// GRBM_GUI_ACTIVE cannot show this: it ticks at a fixed rate (measured
// ~2.4 GHz per XCD) whatever the power manager does to the shader clock.
//
// The loop ends when the real-time counter has advanced `ticks`, which it
// always does, so every launch terminates.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ __launch_bounds__(64) void shader_clock_spin(uint64_t ticks, uint64_t* out) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  uint64_t r = r0;
  while (r - r0 < ticks) {
    __builtin_amdgcn_s_sleep(8);
    r = __builtin_amdgcn_s_memrealtime();
  }
  const uint64_t c1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) {
    out[0] = c1 - c0;
    out[1] = r - r0;
  }
}

}  // namespace

// out: two uint64 on the device, written with (shader cycles, real-time
// ticks). ticks: span to measure, in 10 ns units (capped at one second).
extern "C" int tsp_probe_shader_clock(uint64_t ticks, uint64_t* out, void* stream) {
  if (out == nullptr || ticks == 0 || ticks > 100000000ull) return -1;
  hipLaunchKernelGGL(shader_clock_spin, dim3(1), dim3(64), 0, (hipStream_t)stream, ticks, out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
