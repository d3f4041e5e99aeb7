// CSR SpMV with rows bucketed by length, for gfx950 (bandwidth-bound; no MFMA).
//
// Semantics of the reference spmv (trnsparse/ops.py:30-48):
//   out = alpha * (A @ x)            then  + beta * y   only if y and beta != 0
//
// Row-per-wavefront kernels with an nnz-bucketed split for skewed rows:
//   short rows  (nnz <= 32):        8 lanes per row, 8 rows per wavefront, in
//                                   natural row order (longer rows are
//                                   skipped there);
//   medium rows (32 < nnz <= 2048): one wavefront per row, from a list;
//   long rows   (nnz > 2048):       one 512-thread workgroup per row, from a
//                                   list (wavefront sums meet in LDS).
// The lanes of a row take every G-th entry (coalesced value and index loads,
// several in flight), multiply by the gathered x, and reduce with xor
// shuffles inside the wavefront. Each row is summed by one group in a fixed
// order: deterministic. The plan (the medium and long row lists and their
// counts) depends only on the pattern; callers build it once per matrix.
#include "common.h"

namespace {

constexpr int SHORT_MAX = 32;
constexpr int MEDIUM_MAX = 2048;
constexpr int SHORT_LANES = 8;
constexpr int LONG_THREADS = 512;

template <typename T> struct BAcc { typedef float type; };
template <> struct BAcc<double> { typedef double type; };

// plan (int32): [0] medium count, [1] long count, [2..3] unused, then the
// medium rows at [4, 4 + m) and the long rows at [4 + m, 4 + 2m)
__global__ __launch_bounds__(64) void bucket_zero_kernel(int32_t* __restrict__ plan) {
  if (threadIdx.x < 4) plan[threadIdx.x] = 0;
}

template <typename IdxT>
__global__ __launch_bounds__(256) void bucket_plan_kernel(const IdxT* __restrict__ ptr, int64_t m,
                                                          int32_t* __restrict__ plan) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= m) return;
  const int64_t len = (int64_t)ptr[r + 1] - (int64_t)ptr[r];
  if (len <= SHORT_MAX) return;
  if (len <= MEDIUM_MAX) {
    const int slot = atomicAdd(&plan[0], 1);
    plan[4 + slot] = (int32_t)r;
  } else {
    const int slot = atomicAdd(&plan[1], 1);
    plan[4 + m + slot] = (int32_t)r;
  }
}

template <typename T>
__device__ inline T finish(typename BAcc<T>::type acc, double alpha, const T* __restrict__ y, double beta, int64_t r) {
  typedef typename BAcc<T>::type A;
  A v = (A)alpha * acc;
  if (y) v += (A)beta * (A)y[r];
  return (T)v;
}

template <typename A>
__device__ inline A xor_sum(A v, int width) {
  for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename IdxT, typename T>
__global__ __launch_bounds__(256) void spmv_short_kernel(const T* __restrict__ vals, const IdxT* __restrict__ cols,
                                                         const IdxT* __restrict__ ptr, int64_t m,
                                                         const T* __restrict__ x, double alpha,
                                                         const T* __restrict__ y, double beta, T* __restrict__ out) {
  typedef typename BAcc<T>::type A;
  const int64_t r = ((int64_t)blockIdx.x * 256 + threadIdx.x) / SHORT_LANES;
  const int j = threadIdx.x % SHORT_LANES;
  // the 8 lanes of a row take the same branches, so the shuffles below only
  // ever read lanes of the same row
  if (r >= m) return;
  const int64_t b = (int64_t)ptr[r], e = (int64_t)ptr[r + 1];
  if (e - b > SHORT_MAX) return;  // a medium or long row: its own kernel writes it
  A acc = 0;
#pragma unroll
  for (int i = 0; i < SHORT_MAX / SHORT_LANES; ++i) {
    const int64_t k = b + j + SHORT_LANES * i;
    if (k < e) acc += (A)__builtin_nontemporal_load(&vals[k]) * (A)x[(int64_t)__builtin_nontemporal_load(&cols[k])];
  }
  acc = xor_sum(acc, SHORT_LANES);
  if (j == 0) out[r] = finish<T>(acc, alpha, y, beta, r);
}

template <typename IdxT, typename T>
__global__ __launch_bounds__(256) void spmv_medium_kernel(const T* __restrict__ vals, const IdxT* __restrict__ cols,
                                                          const IdxT* __restrict__ ptr,
                                                          const int32_t* __restrict__ rows, int64_t nrows,
                                                          const T* __restrict__ x, double alpha,
                                                          const T* __restrict__ y, double beta,
                                                          T* __restrict__ out) {
  typedef typename BAcc<T>::type A;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (i >= nrows) return;
  const int64_t r = rows[i];
  const int64_t b = (int64_t)ptr[r], e = (int64_t)ptr[r + 1];
  A acc[4] = {0, 0, 0, 0};
  int64_t k = b + lane;
  for (; k + 192 < e; k += 256) {  // four loads in flight per lane
#pragma unroll
    for (int u = 0; u < 4; ++u)
      acc[u] += (A)__builtin_nontemporal_load(&vals[k + 64 * u]) *
                (A)x[(int64_t)__builtin_nontemporal_load(&cols[k + 64 * u])];
  }
  for (; k < e; k += 64)
    acc[0] += (A)__builtin_nontemporal_load(&vals[k]) * (A)x[(int64_t)__builtin_nontemporal_load(&cols[k])];
  A s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  s = xor_sum(s, 64);
  if (lane == 0) out[r] = finish<T>(s, alpha, y, beta, r);
}

template <typename IdxT, typename T>
__global__ __launch_bounds__(LONG_THREADS) void spmv_long_kernel(const T* __restrict__ vals,
                                                                 const IdxT* __restrict__ cols,
                                                                 const IdxT* __restrict__ ptr,
                                                                 const int32_t* __restrict__ rows,
                                                                 const T* __restrict__ x, double alpha,
                                                                 const T* __restrict__ y, double beta,
                                                                 T* __restrict__ out) {
  typedef typename BAcc<T>::type A;
  __shared__ A part[LONG_THREADS / 64];
  const int64_t r = rows[blockIdx.x];
  const int tid = threadIdx.x;
  const int64_t b = (int64_t)ptr[r], e = (int64_t)ptr[r + 1];
  A acc[4] = {0, 0, 0, 0};
  int64_t k = b + tid;
  for (; k + 3 * LONG_THREADS < e; k += 4 * LONG_THREADS) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
      acc[u] += (A)__builtin_nontemporal_load(&vals[k + LONG_THREADS * u]) *
                (A)x[(int64_t)__builtin_nontemporal_load(&cols[k + LONG_THREADS * u])];
  }
  for (; k < e; k += LONG_THREADS)
    acc[0] += (A)__builtin_nontemporal_load(&vals[k]) * (A)x[(int64_t)__builtin_nontemporal_load(&cols[k])];
  A s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  s = xor_sum(s, 64);
  if ((tid & 63) == 0) part[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) {
    A t = 0;
    for (int w = 0; w < LONG_THREADS / 64; ++w) t += part[w];
    out[r] = finish<T>(t, alpha, y, beta, r);
  }
}

template <typename IdxT, typename T>
int launch(const void* values, const void* cols, const void* ptrs, int64_t m, const int32_t* plan, int64_t n_medium,
           int64_t n_long, const void* x, double alpha, const void* y, double beta, void* out, hipStream_t st) {
  const int64_t gs = tsp::ceil_div(m * SHORT_LANES, 256);
  const int64_t gm = tsp::ceil_div(n_medium * 64, 256);
  if (gs > INT32_MAX || gm > INT32_MAX || n_long > INT32_MAX)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_bucketed_spmv: too many rows");
  if (gs > 0)
    hipLaunchKernelGGL((spmv_short_kernel<IdxT, T>), dim3((unsigned)gs), dim3(256), 0, st, (const T*)values,
                       (const IdxT*)cols, (const IdxT*)ptrs, m, (const T*)x, alpha, (const T*)y, beta, (T*)out);
  int rc = tsp::check_launch("spmv_short_kernel launch");
  if (rc) return rc;
  if (gm > 0) {
    hipLaunchKernelGGL((spmv_medium_kernel<IdxT, T>), dim3((unsigned)gm), dim3(256), 0, st, (const T*)values,
                       (const IdxT*)cols, (const IdxT*)ptrs, plan + 4, n_medium, (const T*)x, alpha, (const T*)y, beta,
                       (T*)out);
    rc = tsp::check_launch("spmv_medium_kernel launch");
    if (rc) return rc;
  }
  if (n_long > 0) {
    hipLaunchKernelGGL((spmv_long_kernel<IdxT, T>), dim3((unsigned)n_long), dim3(LONG_THREADS), 0, st,
                       (const T*)values, (const IdxT*)cols, (const IdxT*)ptrs, plan + 4 + m, (const T*)x, alpha,
                       (const T*)y, beta, (T*)out);
    rc = tsp::check_launch("spmv_long_kernel launch");
    if (rc) return rc;
  }
  return TSP_OK;
}

}  // namespace

extern "C" int64_t tsp_csr_bucket_plan_size(int64_t m) {
  if (m < 0 || m > INT32_MAX) return -1;
  return (4 + 2 * m) * 4;
}

extern "C" int tsp_csr_bucket_plan(const void* row_ptrs, int index_type, int64_t m, void* plan, void* stream) {
  if (index_type != TSP_I32 && index_type != TSP_I64)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_bucket_plan: index type %d not supported", index_type);
  if (m < 0 || m > INT32_MAX) return tsp::fail(TSP_EINVAL, "tsp_csr_bucket_plan: bad row count");
  if (!plan || (m > 0 && !row_ptrs)) return tsp::fail(TSP_EINVAL, "tsp_csr_bucket_plan: null pointer");
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(bucket_zero_kernel, dim3(1), dim3(64), 0, st, (int32_t*)plan);
  int rc = tsp::check_launch("bucket_zero_kernel launch");
  if (rc || m == 0) return rc;
  const int64_t grid = tsp::ceil_div(m, 256);
  if (index_type == TSP_I32)
    hipLaunchKernelGGL((bucket_plan_kernel<int32_t>), dim3((unsigned)grid), dim3(256), 0, st, (const int32_t*)row_ptrs,
                       m, (int32_t*)plan);
  else
    hipLaunchKernelGGL((bucket_plan_kernel<int64_t>), dim3((unsigned)grid), dim3(256), 0, st, (const int64_t*)row_ptrs,
                       m, (int32_t*)plan);
  return tsp::check_launch("bucket_plan_kernel launch");
}

extern "C" int tsp_csr_bucketed_spmv(const void* values, int dtype, const void* col_indices, const void* row_ptrs,
                                     int index_type, int64_t m, int64_t n, int64_t nnz, const void* plan,
                                     int64_t n_medium, int64_t n_long, const void* x, double alpha, const void* y,
                                     double beta, void* out, void* stream) {
  if (dtype != TSP_F32 && dtype != TSP_F64)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_bucketed_spmv: dtype %d not supported", dtype);
  if (index_type != TSP_I32 && index_type != TSP_I64)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_bucketed_spmv: index type %d not supported", index_type);
  if (m < 0 || n < 0 || nnz < 0 || n_medium < 0 || n_long < 0 || n_medium + n_long > m)
    return tsp::fail(TSP_EINVAL, "tsp_csr_bucketed_spmv: bad size");
  if (m == 0) return TSP_OK;
  if (!row_ptrs || !plan || !out || (nnz > 0 && (!values || !col_indices || !x)))
    return tsp::fail(TSP_EINVAL, "tsp_csr_bucketed_spmv: null pointer");
  const void* yy = (y && beta != 0.0) ? y : nullptr;
  hipStream_t st = (hipStream_t)stream;
  const int32_t* p = (const int32_t*)plan;
  if (dtype == TSP_F32)
    return index_type == TSP_I32
               ? launch<int32_t, float>(values, col_indices, row_ptrs, m, p, n_medium, n_long, x, alpha, yy, beta, out,
                                        st)
               : launch<int64_t, float>(values, col_indices, row_ptrs, m, p, n_medium, n_long, x, alpha, yy, beta, out,
                                        st);
  return index_type == TSP_I32
             ? launch<int32_t, double>(values, col_indices, row_ptrs, m, p, n_medium, n_long, x, alpha, yy, beta, out,
                                       st)
             : launch<int64_t, double>(values, col_indices, row_ptrs, m, p, n_medium, n_long, x, alpha, yy, beta, out,
                                       st);
}
