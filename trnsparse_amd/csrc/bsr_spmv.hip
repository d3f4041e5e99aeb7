// BSR times one vector, fused with the vector update of a fixed-step solver.
//
//   out[r] = alpha * (A x)[r] + beta * u[r] + gamma * v[r] + delta * w[r]
//
// for r < m (u, v, w optional). With alpha = 1 and no u, v, w it is the
// N = 1 case of bsr_spmm (reference ops.py:162-192; the reference's
// iterative solvers call bsr_spmm(A, x[:, None]), iterative.py:44-50); with
// alpha = -omega, u = x, v = b it is one Richardson step
// (iterative.py:256-295), and with w = x_prev one Chebyshev step
// (iterative.py:200-253) — A is read once per step and the update needs no
// second pass.
//
// N = 1 is HBM-bound (2 flops per 4-byte block element): no MFMA. The fast
// kernel (block size 128) gives one workgroup a 4-row slice of a block
// row and its 4 wavefronts every 4th stored block of the row each: per
// block a wavefront reads the slice's 4 x 128 elements as one contiguous
// run (2 KiB in fp32) with 16-byte loads (lane l always covers the same 16 bytes of a
// block row, so its x piece is one 16-byte load per block), accumulates a
// partial per row and reduces each row over the lanes that share it; the
// 4 wavefronts' row sums are then added in wavefront order through LDS.
// Splitting a block row's blocks over 4 wavefronts keeps the longest rows
// from setting the kernel's length (cfg3's rows hold 8 to 20 blocks).
// Slices of heavy block rows are dispatched first (on a matrix with a few
// full block rows among light ones this order is worth a fifth of the
// time). 4-row slices against 8: the same time on cfg3, 7 % less on such a
// skewed matrix. Other block sizes use a thread-per-row kernel.
#include "common.h"

namespace {

template <typename T> struct SAcc { typedef float type; };
template <> struct SAcc<double> { typedef double type; };
template <typename T> __device__ inline typename SAcc<T>::type to_a(T v) { return (typename SAcc<T>::type)v; }
template <> __device__ inline float to_a<uint16_t>(uint16_t v) { return tsp::bf16_bits_to_f32(v); }
template <typename T> __device__ inline T from_a(typename SAcc<T>::type v) { return (T)v; }
template <> __device__ inline uint16_t from_a<uint16_t>(float v) { return tsp::f32_to_bf16_bits(v); }

constexpr int SB = 128;    // block size of the fast kernel
constexpr int SLICE = 4;   // rows per workgroup

template <typename T, int V> struct alignas(sizeof(T) * V) Vec { T e[V]; };

// out[r] for one row from the accumulated product
template <typename T>
__device__ inline void finish(int64_t r, typename SAcc<T>::type ax, typename SAcc<T>::type alpha, const T* u,
                              typename SAcc<T>::type beta, const T* v, typename SAcc<T>::type gamma, const T* w,
                              typename SAcc<T>::type delta, T* out) {
  typename SAcc<T>::type y = alpha * ax;
  if (u) y += beta * to_a(u[r]);
  if (v) y += gamma * to_a(v[r]);
  if (w) y += delta * to_a(w[r]);
  out[r] = from_a<T>(y);
}

// Fast kernel: workgroup per (block row, 4-row slice), wavefront w takes the
// row's stored blocks w, w + 4, ... V elements per 16-byte load; LPR = SB / V
// lanes share a row, RPI = 64 / LPR rows per load instruction, NI = SLICE /
// RPI loads per block.
template <typename T>
__global__ __launch_bounds__(256) void bsr_spmv_b128(const T* __restrict__ blocks, const int64_t* __restrict__ rp,
                                                     const int64_t* __restrict__ ci, int64_t mb, int64_t m, int64_t n,
                                                     const T* __restrict__ x, typename SAcc<T>::type alpha,
                                                     const T* __restrict__ u, typename SAcc<T>::type beta,
                                                     const T* __restrict__ v, typename SAcc<T>::type gamma,
                                                     const T* __restrict__ w_vec, typename SAcc<T>::type delta,
                                                     T* __restrict__ out, const int32_t* __restrict__ order) {
  typedef typename SAcc<T>::type AccT;
  constexpr int V = 16 / sizeof(T);
  constexpr int LPR = SB / V;
  constexpr int RPI = 64 / LPR;
  constexpr int NI = SLICE / RPI;
  constexpr int NSL = SB / SLICE;  // slices per block row
  __shared__ typename SAcc<T>::type part[4][SLICE];
  const int64_t unit = blockIdx.x;
  if (unit >= mb * NSL) return;
  const int w = threadIdx.x >> 6;
  const int64_t i = order ? order[unit / NSL] : unit / NSL;
  const int sl = (int)(unit % NSL);
  const int lane = threadIdx.x & 63;
  const int cl = lane % LPR;           // 16-byte piece of a block row
  const int rl = lane / LPR;           // row within a load instruction
  const int64_t r0 = sl * SLICE;       // first row of the slice within the block
  AccT acc[NI];
#pragma unroll
  for (int q = 0; q < NI; ++q) acc[q] = 0;
  const int64_t s = rp[i], e = rp[i + 1];
  // the row's block columns, 64 at a time, one per lane (read with
  // readlane), and UNR blocks' loads in flight before their products
  constexpr int UNR = 4;
  for (int64_t base = s; base < e; base += 64) {
    const int cnt = (int)(e - base < 64 ? e - base : 64);
    const int myc = lane < cnt ? (int)ci[base + lane] : 0;
    for (int k0 = w; k0 < cnt; k0 += 4 * UNR) {
      Vec<T, V> xv[UNR], a[UNR][NI];
#pragma unroll
      for (int j = 0; j < UNR; ++j) {
        const int kk = k0 + 4 * j;
        if (kk < cnt) {
          const int64_t c0 = (int64_t)__builtin_amdgcn_readlane(myc, kk) * SB + cl * V;
          // x piece (zero past n: the reference pads B's rows)
          if (c0 + V <= n) {
            xv[j] = *(const Vec<T, V>*)(x + c0);
          } else {
#pragma unroll
            for (int t = 0; t < V; ++t) xv[j].e[t] = c0 + t < n ? x[c0 + t] : T(0);
          }
          const T* blk = blocks + (base + kk) * SB * SB + r0 * SB;
#pragma unroll
          for (int q = 0; q < NI; ++q) a[j][q] = *(const Vec<T, V>*)(blk + (q * 64 + lane) * V);
        }
      }
#pragma unroll
      for (int j = 0; j < UNR; ++j) {
        if (k0 + 4 * j < cnt) {
#pragma unroll
          for (int q = 0; q < NI; ++q)
#pragma unroll
            for (int t = 0; t < V; ++t) acc[q] += to_a(a[j][q].e[t]) * to_a(xv[j].e[t]);
        }
      }
    }
  }
  // row (r0 + q * RPI + rl): sum over its LPR lanes, then over the 4
  // wavefronts in wavefront order
#pragma unroll
  for (int q = 0; q < NI; ++q) {
    AccT t = acc[q];
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
    if (cl == 0) part[w][q * RPI + rl] = t;
  }
  __syncthreads();
  if (threadIdx.x < SLICE) {
    const int rr = threadIdx.x;
    const AccT t = ((part[0][rr] + part[1][rr]) + part[2][rr]) + part[3][rr];
    const int64_t r = i * SB + r0 + rr;
    if (r < m) finish<T>(r, t, alpha, u, beta, v, gamma, w_vec, delta, out);
  }
}

// Any block size: thread per row.
template <typename T>
__global__ __launch_bounds__(256) void bsr_spmv_generic(const T* __restrict__ blocks, const int64_t* __restrict__ rp,
                                                        const int64_t* __restrict__ ci, int64_t b, int64_t m,
                                                        int64_t n, const T* __restrict__ x,
                                                        typename SAcc<T>::type alpha, const T* __restrict__ u,
                                                        typename SAcc<T>::type beta, const T* __restrict__ v,
                                                        typename SAcc<T>::type gamma, const T* __restrict__ w,
                                                        typename SAcc<T>::type delta, T* __restrict__ out) {
  typedef typename SAcc<T>::type AccT;
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= m) return;
  const int64_t i = r / b, rr = r % b;
  AccT acc = 0;
  for (int64_t k = rp[i]; k < rp[i + 1]; ++k) {
    const int64_t c0 = ci[k] * b;
    const T* row = blocks + (k * b + rr) * b;
    for (int64_t c = 0; c < b && c0 + c < n; ++c) acc += to_a(row[c]) * to_a(x[c0 + c]);
  }
  finish<T>(r, acc, alpha, u, beta, v, gamma, w, delta, out);
}

template <typename T>
int launch(const void* blocks, const int64_t* rp, const int64_t* ci, int64_t b, int64_t m, int64_t n, const void* x,
           double alpha, const void* u, double beta, const void* v, double gamma, const void* w, double delta,
           void* out, const int32_t* order, hipStream_t st) {
  typedef typename SAcc<T>::type AccT;
  const int64_t mb = tsp::ceil_div(m, b);
  const bool aligned = ((uintptr_t)blocks % 16) == 0 && ((uintptr_t)x % 16) == 0;
  if (b == SB && aligned) {
    const int64_t g = mb * (SB / SLICE);  // one workgroup per (block row, slice)
    if (g > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmv: too many block rows");
    hipLaunchKernelGGL(bsr_spmv_b128<T>, dim3((unsigned)g), dim3(256), 0, st, (const T*)blocks, rp, ci, mb, m, n,
                       (const T*)x, (AccT)alpha, (const T*)u, (AccT)beta, (const T*)v, (AccT)gamma, (const T*)w,
                       (AccT)delta, (T*)out, order);
    return tsp::check_launch("bsr_spmv_b128 launch");
  }
  const int64_t g = tsp::ceil_div(m, 256);
  if (g > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmv: too many rows");
  hipLaunchKernelGGL(bsr_spmv_generic<T>, dim3((unsigned)g), dim3(256), 0, st, (const T*)blocks, rp, ci, b, m, n,
                     (const T*)x, (AccT)alpha, (const T*)u, (AccT)beta, (const T*)v, (AccT)gamma, (const T*)w,
                     (AccT)delta, (T*)out);
  return tsp::check_launch("bsr_spmv_generic launch");
}

}  // namespace

extern "C" int tsp_bsr_spmv(const void* blocks, int dtype, const int64_t* block_row_ptrs,
                            const int64_t* block_col_indices, int64_t n_blocks, int64_t block_size, int64_t m,
                            int64_t n, const void* x, double alpha, const void* u, double beta, const void* v,
                            double gamma, const void* w, double delta, void* out, const int32_t* row_order,
                            void* stream) {
  if (dtype != TSP_F32 && dtype != TSP_F64 && dtype != TSP_BF16)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmv: dtype %d not supported", dtype);
  if (m < 0 || n < 0 || block_size <= 0 || n_blocks < 0) return tsp::fail(TSP_EINVAL, "tsp_bsr_spmv: bad size");
  if (m == 0) return TSP_OK;
  if (!block_row_ptrs || !out || (n_blocks > 0 && (!blocks || !block_col_indices || !x)))
    return tsp::fail(TSP_EINVAL, "tsp_bsr_spmv: null pointer");
  if (x && x == out) return tsp::fail(TSP_EINVAL, "tsp_bsr_spmv: out must not alias x");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TSP_F32)
    return launch<float>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, x, alpha, u, beta, v, gamma, w,
                         delta, out, row_order, st);
  if (dtype == TSP_F64)
    return launch<double>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, x, alpha, u, beta, v, gamma, w,
                          delta, out, row_order, st);
  return launch<uint16_t>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, x, alpha, u, beta, v, gamma, w,
                          delta, out, row_order, st);
}
