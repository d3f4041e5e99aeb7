// Shared device/host helpers for the trnsparse MI355X (gfx950) kernels.
//
// Everything in this library is written for CDNA4: 64-lane wavefronts,
// MFMA matrix cores, 160 KiB of LDS per CU, 8 XCDs with private L2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/trnsparse_hip.h"

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace tsp {

// ---------------------------------------------------------------- errors
// Thread-local message behind tsp_last_error(); set by every failing entry.
int fail(int code, const char* fmt, ...);
// Map a HIP status from a launch / API call to TSP_EHIP with a message.
int check_hip(hipError_t e, const char* what);
// Check the most recent launch on this thread.
int check_launch(const char* what);
// Zero `bytes` bytes at device pointer p with a fill kernel on `st` (used
// instead of hipMemsetAsync so callers may capture the work in a HIP graph).
int zero_fill(void* p, int64_t bytes, hipStream_t st);

// dB = A^T X of bsr_spmm's backward at block sizes 8, 16, 32, 64 (fp32 or
// bf16 in and out), defined with the small-block forward kernel.
int launch_bsr_small_t(int dtype, int64_t bs, const void* blocks, const int64_t* col_ptrs,
                       const int64_t* col_block_rows, const int64_t* col_block_ids, int64_t n_block_cols, int64_t m,
                       int64_t n, const void* X, int64_t ldx, int64_t ncols, void* out, int64_t ldo, hipStream_t st);

// ---------------------------------------------------------------- bf16
// Round-to-nearest-even fp32 -> bf16 bit pattern (NaN kept quiet), the same
// rounding torch applies in `tensor.to(torch.bfloat16)`.
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__host__ __device__ inline float bf16_bits_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, ((uint32_t)h) << 16);
}

// Value-type traits used by the generic (any block size / any dtype) kernels.
template <typename T> struct Acc { typedef float type; };
template <> struct Acc<double> { typedef double type; };

template <typename T> __device__ inline typename Acc<T>::type to_acc(T v) { return (typename Acc<T>::type)v; }
template <> __device__ inline float to_acc<uint16_t>(uint16_t v) { return bf16_bits_to_f32(v); }

template <typename T> __device__ inline T from_acc(typename Acc<T>::type v) { return (T)v; }
template <> __device__ inline uint16_t from_acc<uint16_t>(float v) { return f32_to_bf16_bits(v); }

// Non-temporal (streaming) global loads: data read once should not evict
// the re-used operands (x of SpMV, B panels of SpMM) from L2.
template <typename T> __device__ inline T ld_stream(const T* p) { return __builtin_nontemporal_load(p); }

__device__ inline int lane_id() { return threadIdx.x & 63; }

// Sum over the 64 lanes of a wavefront (xor butterfly; every lane gets the total).
template <typename T> __device__ inline T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Sum within aligned groups of G lanes (G a power of two <= 64).
template <typename T> __device__ inline T group_sum(T v, int G) {
  for (int o = G >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace tsp
