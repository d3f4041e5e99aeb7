// Helpers for kernels that issue MFMAs and VALU work in a fixed slot order.
#pragma once

#include <utility>

#include "common.h"

namespace tsp {

// f(integral_constant<int, k>) for k = 0 .. N-1 in order, fully unrolled at
// compile time (slot loops are too long for the loop unroller).
template <typename F, int... Ks>
__device__ __attribute__((always_inline)) inline void static_for_impl(F&& f, std::integer_sequence<int, Ks...>) {
  (f(std::integral_constant<int, Ks>{}), ...);
}
template <int N, typename F>
__device__ __attribute__((always_inline)) inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Keep a register operand that only MFMAs read in AGPRs (MFMA takes its A
// and B operands from either file), leaving the VGPRs to values the VALU uses.
__device__ inline void pin_agpr(bf16x8& v) {
  u32x4 t = __builtin_bit_cast(u32x4, v);
  asm volatile("" : "+a"(t));
  v = __builtin_bit_cast(bf16x8, t);
}

}  // namespace tsp
