// CSR SpMV and SpMM for gfx950 (bandwidth-bound; no MFMA).
//
// Semantics follow the reference (trnsparse/ops.py:30-48 spmv, :51-78 spmm):
//   out = alpha * (A @ x)            then  + beta * y   only if y and beta != 0
// alpha multiplies the finished row sum; y is read, never written.
//
// SpMV: work partition ("windows")
//   A row r sits at position pos(r) = (row_ptrs[r] - row_ptrs[0]) + r on the
//   merged rows+nonzeros axis, which is strictly increasing. Window k holds
//   the rows with pos(r) in [k*CAP, (k+1)*CAP): at most CAP rows, and all but
//   its last row end inside the window (fewer than CAP nonzeros before the
//   last row starts). The table windows[k] = first row of window k is built
//   in one pass on the device (each row writes the windows that begin at it)
//   and depends only on the pattern, so callers cache it with the matrix.
//
// SpMV kernel: one 256-thread workgroup per window.
//   1. stream the window's values and column indices with coalesced,
//      non-temporal loads (8 per thread in flight), gather x (kept in L2 by
//      the streaming hint), and stage the products plus the row offsets in
//      LDS;
//   2. reduce rows with G lanes per row (G = power of two filling the
//      workgroup, up to a wavefront), xor-shuffle reduction inside the group;
//   3. a last row longer than the LDS capacity is reduced by the whole
//      workgroup (skewed / Zipf rows), wavefront shuffles + LDS across waves.
//
// SDDMM (values gradient of A X, tsp_csr_sddmm): per nonzero the dot product
// of G's row and X's row over the dense columns, lanes as in the narrow SpMM.
//
// SpMM: one wavefront per row, lanes across the columns of B (coalesced B
// row reads), the row's (col, value) pairs loaded 64 at a time and broadcast
// with shuffles. fp32 B with a multiple of 4 columns takes the narrow
// variant: several rows per wavefront, each row's nonzeros split over lane
// groups, 16-byte B loads, 128-column passes.
#include "common.h"

namespace {

constexpr int SPMV_THREADS = 256;
constexpr int CAP = 2048;       // rows + nonzeros per window
constexpr int LDS_CAP = 4096;   // staged products per window
constexpr int UNROLL = 8;

template <typename IdxT>
__global__ __launch_bounds__(256) void csr_plan_kernel(const IdxT* __restrict__ ptr, int64_t m, int64_t nwin,
                                                       int64_t* __restrict__ win) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r > m) return;
  const int64_t base = (int64_t)ptr[0];
  const int64_t pos = (int64_t)ptr[r] - base + r;
  const int64_t prev = r == 0 ? -1 : (int64_t)ptr[r - 1] - base + (r - 1);
  // windows k with prev < k*CAP <= pos start at row r
  int64_t k = prev < 0 ? 0 : prev / CAP + 1;
  const int64_t kend = pos / CAP;
  for (; k <= kend && k < nwin; ++k) win[k] = r;
  if (r == m) win[nwin] = m;
}

template <typename T> struct SpmvAcc { typedef float type; };
template <> struct SpmvAcc<double> { typedef double type; };

template <typename IdxT, typename T>
__global__ __launch_bounds__(SPMV_THREADS) void csr_spmv_kernel(
    const T* __restrict__ vals, const IdxT* __restrict__ cols, const IdxT* __restrict__ ptr,
    const int64_t* __restrict__ win, const T* __restrict__ x, T alpha, const T* __restrict__ y, T beta,
    T* __restrict__ out) {
  typedef typename SpmvAcc<T>::type AccT;
  __shared__ AccT prod[LDS_CAP];
  __shared__ int offs[CAP + 1];
  __shared__ AccT wsum[SPMV_THREADS / 64];

  const int tid = threadIdx.x;
  const int64_t r0 = win[blockIdx.x], r1 = win[blockIdx.x + 1];
  if (r0 >= r1) return;
  const int64_t p0 = (int64_t)ptr[r0];
  const int64_t pend = (int64_t)ptr[r1];
  const bool long_tail = pend - p0 > LDS_CAP;
  const int64_t rs = long_tail ? r1 - 1 : r1;  // rows [r0, rs) go through LDS
  const int nr = (int)(rs - r0);
  const int n = (int)((int64_t)ptr[rs] - p0);  // < LDS_CAP by construction

  // row offsets (relative to p0) for the staged rows
  for (int i = tid; i <= nr; i += SPMV_THREADS) offs[i] = (int)((int64_t)ptr[r0 + i] - p0);

  // products of the staged nonzeros
  for (int base = 0; base < n; base += SPMV_THREADS * UNROLL) {
    IdxT c[UNROLL];
    T v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int i = base + u * SPMV_THREADS + tid;
      if (i < n) {
        c[u] = tsp::ld_stream(cols + p0 + i);
        v[u] = tsp::ld_stream(vals + p0 + i);
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int i = base + u * SPMV_THREADS + tid;
      if (i < n) prod[i] = (AccT)v[u] * (AccT)x[c[u]];
    }
  }
  __syncthreads();

  if (nr > 0) {
    int G = 64;
    while (G > 1 && G * nr > SPMV_THREADS) G >>= 1;
    const int q = tid & (G - 1);
    const int rows_per_pass = SPMV_THREADS / G;
    const int npass = (nr + rows_per_pass - 1) / rows_per_pass;
    // every lane runs every pass: the group reduction shuffles need the full wavefront
    for (int pass = 0; pass < npass; ++pass) {
      const int rr = pass * rows_per_pass + tid / G;
      AccT s = 0;
      if (rr < nr) {
        const int a = offs[rr], e = offs[rr + 1];
        for (int j = a + q; j < e; j += G) s += prod[j];
      }
      s = tsp::group_sum(s, G);
      if (rr < nr && q == 0) {
        const int64_t r = r0 + rr;
        T res = alpha * (T)s;
        if (y) res = res + beta * y[r];
        out[r] = res;
      }
    }
  }

  if (long_tail) {
    // whole-workgroup reduction of the last row
    const int64_t r = r1 - 1;
    const int64_t a = (int64_t)ptr[r], e = (int64_t)ptr[r + 1];
    AccT s = 0;
    for (int64_t j0 = a; j0 < e; j0 += SPMV_THREADS * UNROLL) {
      IdxT c[UNROLL];
      T v[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t j = j0 + u * SPMV_THREADS + tid;
        if (j < e) {
          c[u] = tsp::ld_stream(cols + j);
          v[u] = tsp::ld_stream(vals + j);
        }
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t j = j0 + u * SPMV_THREADS + tid;
        if (j < e) s += (AccT)v[u] * (AccT)x[c[u]];
      }
    }
    s = tsp::wave_sum(s);
    if ((tid & 63) == 0) wsum[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
      AccT t = 0;
      for (int w = 0; w < SPMV_THREADS / 64; ++w) t += wsum[w];
      T res = alpha * (T)t;
      if (y) res = res + beta * y[r];
      out[r] = res;
    }
  }
}

// SpMM: wavefront per row, NC column chunks of 64 per pass.
template <typename IdxT, typename T, int NC>
__global__ __launch_bounds__(256) void csr_spmm_kernel(
    const T* __restrict__ vals, const IdxT* __restrict__ cols, const IdxT* __restrict__ ptr, int64_t m,
    const T* __restrict__ B, int64_t ldb, int64_t ncols, T alpha, const T* __restrict__ Cin, int64_t ldci, T beta,
    T* __restrict__ out, int64_t ldo) {
  typedef typename SpmvAcc<T>::type AccT;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x / 64);
  for (int64_t r = wave; r < m; r += nwaves) {
    const int64_t a = (int64_t)ptr[r], e = (int64_t)ptr[r + 1];
    for (int64_t c0 = 0; c0 < ncols; c0 += 64 * NC) {
      AccT acc[NC];
#pragma unroll
      for (int u = 0; u < NC; ++u) acc[u] = 0;
      for (int64_t e0 = a; e0 < e; e0 += 64) {
        const int64_t my = e0 + lane;
        int64_t cl = 0;
        T vl = 0;
        if (my < e) {
          cl = (int64_t)cols[my];
          vl = vals[my];
        }
        const int cnt = (int)((e - e0) < 64 ? (e - e0) : 64);
#pragma unroll 4
        for (int j = 0; j < cnt; ++j) {
          const int64_t cj = __shfl(cl, j, 64);
          const AccT vj = (AccT)__shfl(vl, j, 64);
          const T* brow = B + cj * ldb + c0 + lane;
#pragma unroll
          for (int u = 0; u < NC; ++u)
            if (c0 + 64 * u + lane < ncols) acc[u] += vj * (AccT)brow[64 * u];
        }
      }
#pragma unroll
      for (int u = 0; u < NC; ++u) {
        const int64_t c = c0 + 64 * u + lane;
        if (c < ncols) {
          T res = alpha * (T)acc[u];
          if (Cin) res = res + beta * Cin[r * ldci + c];
          out[r * ldo + c] = res;
        }
      }
    }
  }
}

// SpMM for fp32 B with ncols % 4 == 0 and 16-byte aligned rows: lanes =
// (row slot, nonzero group, column quad). P lanes cover up to 128 columns
// of a row as column quads (P a power of two; wider B takes several column
// passes, each a work item of its own), G lane groups
// take every G-th nonzero of the row, and R = 64 / (P G) rows run side by
// side in a wavefront, so narrow B still fills the wavefront and every B
// access is a 16-byte load. U nonzeros per group are fetched before their B
// rows are loaded (U independent gathers in flight per lane). The groups'
// float4 partial sums are added with xor shuffles at the end of the rows.
template <typename IdxT, int P, int G>
__global__ __launch_bounds__(256) void csr_spmm_narrow_kernel(
    const float* __restrict__ vals, const IdxT* __restrict__ cols, const IdxT* __restrict__ ptr, int64_t m,
    const float* __restrict__ B, int64_t ldb, int64_t ncols, float alpha, const float* __restrict__ Cin,
    int64_t ldci, float beta, float* __restrict__ out, int64_t ldo) {
  constexpr int R = 64 / (P * G);
  constexpr int U = 4;
  const int lane = threadIdx.x & 63;
  const int cq = lane % P, gi = (lane / P) % G, rs = lane / (P * G);
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x / 64);
  for (int64_t rc = wave; rc < tsp::ceil_div(m, R) * tsp::ceil_div(ncols, 4 * P); rc += nwaves) {
    // item rc: rows r0 .. r0 + R, columns c0 .. c0 + 4P (wider B takes several column passes)
    const int64_t npass = tsp::ceil_div(ncols, 4 * P);
    const int64_t r0 = (rc / npass) * R, c0 = (rc % npass) * 4 * P + 4 * cq;
    const bool cvalid = c0 < ncols;
    const int64_t r = r0 + rs;
    int64_t a = 0, e = 0;
    if (r < m) {
      a = (int64_t)ptr[r];
      e = (int64_t)ptr[r + 1];
    }
    f32x4 acc = f32x4{};
    for (int64_t j0 = a + gi; j0 < e; j0 += (int64_t)G * U) {
      int64_t cj[U];
      float vj[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t j = j0 + (int64_t)u * G;
        cj[u] = j < e ? (int64_t)cols[j] : -1;
        vj[u] = j < e ? vals[j] : 0.f;
      }
      f32x4 bv[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        bv[u] = (cj[u] >= 0 && cvalid) ? *(const f32x4*)(B + cj[u] * ldb + c0) : f32x4{};
#pragma unroll
      for (int u = 0; u < U; ++u) acc += vj[u] * bv[u];
    }
#pragma unroll
    for (int o = P; o < P * G; o <<= 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += __shfl_xor(acc[i], o, 64);
    }
    if (gi == 0 && r < m && cvalid) {
      f32x4 res = alpha * acc;
      if (Cin) res = res + beta * *(const f32x4*)(Cin + r * ldci + c0);
      *(f32x4*)(out + r * ldo + c0) = res;
    }
  }
}

template <typename IdxT>
int spmm_narrow_launch(const void* values, const void* col, const void* rp, int64_t m, const void* B, int64_t ldb,
                       int64_t ncols, double alpha, const void* C, int64_t ldc, double beta, void* out, int64_t ldo,
                       hipStream_t st) {
  const float* cc = (C && beta != 0.0) ? (const float*)C : nullptr;
  const int64_t quads = ncols / 4;
  int P = 1;
  while (P < quads && P < 32) P <<= 1;
  const int G = P >= 16 ? 64 / P : 8;
  const int64_t R = 64 / (P * G);
  int64_t grid = tsp::ceil_div(tsp::ceil_div(m, R) * tsp::ceil_div(ncols, 4 * P), 4);
  if (grid > 65536) grid = 65536;
#define TSP_NARROW(PP, GG)                                                                                          \
  hipLaunchKernelGGL((csr_spmm_narrow_kernel<IdxT, PP, GG>), dim3((unsigned)grid), dim3(256), 0, st,                \
                     (const float*)values, (const IdxT*)col, (const IdxT*)rp, m, (const float*)B, ldb, ncols,       \
                     (float)alpha, cc, ldc, (float)beta, (float*)out, ldo)
  switch (P) {
    case 1: TSP_NARROW(1, 8); break;
    case 2: TSP_NARROW(2, 8); break;
    case 4: TSP_NARROW(4, 8); break;
    case 8: TSP_NARROW(8, 8); break;
    case 16: TSP_NARROW(16, 4); break;
    default: TSP_NARROW(32, 2); break;
  }
#undef TSP_NARROW
  return tsp::check_launch("csr_spmm_narrow launch");
}

// CSR SDDMM on the matrix's own pattern (the values gradient of alpha A X):
// dv[p] = alpha * sum_c G[row p][c] * X[col p][c] over ncols columns. Lanes as
// in csr_spmm_narrow_kernel: P lanes per nonzero read V consecutive columns
// each (P V columns per pass, more passes for wider operands), G groups take
// every G-th nonzero of a row (U at a time), R rows per wavefront; the P
// partial dot products of a nonzero are summed with xor shuffles within its
// P lanes, which share every loop trip.
template <typename T, int V>
struct VecOf {
  typedef T type __attribute__((ext_vector_type(V)));
  __device__ static T hsum(type v) {
    T s = v[0];
#pragma unroll
    for (int i = 1; i < V; ++i) s += v[i];
    return s;
  }
};
template <typename T>
struct VecOf<T, 1> {
  typedef T type;
  __device__ static T hsum(T v) { return v; }
};

template <typename IdxT, typename T, int V, int P, int G>
__global__ __launch_bounds__(256) void csr_sddmm_kernel(const IdxT* __restrict__ cols, const IdxT* __restrict__ ptr,
                                                        int64_t m, const T* __restrict__ Gm, int64_t ldg,
                                                        const T* __restrict__ X, int64_t ldx, int64_t ncols, T alpha,
                                                        T* __restrict__ dv) {
  constexpr int R = 64 / (P * G);
  constexpr int U = 4;
  typedef VecOf<T, V> VT;
  typedef typename VT::type vt;
  const int lane = threadIdx.x & 63;
  const int cq = lane % P, gi = (lane / P) % G, rs = lane / (P * G);
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x / 64);
  for (int64_t rc = wave; rc < tsp::ceil_div(m, R); rc += nwaves) {
    const int64_t r = rc * R + rs;
    int64_t a = 0, e = 0;
    if (r < m) {
      a = (int64_t)ptr[r];
      e = (int64_t)ptr[r + 1];
    }
    for (int64_t j0 = a + gi; j0 < e; j0 += (int64_t)G * U) {
      int64_t cj[U];
      T dot[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t j = j0 + (int64_t)u * G;
        cj[u] = j < e ? (int64_t)cols[j] : -1;
        dot[u] = 0;
      }
      for (int64_t c0 = (int64_t)V * cq; c0 < ncols; c0 += (int64_t)V * P) {
        const vt gv = *(const vt*)(Gm + r * ldg + c0);
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (cj[u] >= 0) dot[u] += VT::hsum(gv * *(const vt*)(X + cj[u] * ldx + c0));
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int o = 1; o < P; o <<= 1) dot[u] += __shfl_xor(dot[u], o, 64);
      if (cq == 0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t j = j0 + (int64_t)u * G;
          if (j < e) dv[j] = alpha * dot[u];
        }
      }
    }
  }
}

template <typename IdxT, typename T, int V>
int sddmm_launch_v(const void* col, const void* rp, int64_t m, const void* Gm, int64_t ldg, const void* X, int64_t ldx,
                   int64_t ncols, double alpha, void* dv, hipStream_t st) {
  const int64_t units = tsp::ceil_div(ncols, V);
  int P = 1;
  while (P < units && P < 32) P <<= 1;
  const int G = P >= 16 ? 64 / P : 8;
  const int64_t R = 64 / (P * G);
  int64_t grid = tsp::ceil_div(tsp::ceil_div(m, R), 4);
  if (grid > 65536) grid = 65536;
#define TSP_SDDMM(PP, GG)                                                                                           \
  hipLaunchKernelGGL((csr_sddmm_kernel<IdxT, T, V, PP, GG>), dim3((unsigned)grid), dim3(256), 0, st,                \
                     (const IdxT*)col, (const IdxT*)rp, m, (const T*)Gm, ldg, (const T*)X, ldx, ncols, (T)alpha,   \
                     (T*)dv)
  switch (P) {
    case 1: TSP_SDDMM(1, 8); break;
    case 2: TSP_SDDMM(2, 8); break;
    case 4: TSP_SDDMM(4, 8); break;
    case 8: TSP_SDDMM(8, 8); break;
    case 16: TSP_SDDMM(16, 4); break;
    default: TSP_SDDMM(32, 2); break;
  }
#undef TSP_SDDMM
  return tsp::check_launch("csr_sddmm launch");
}

template <typename IdxT, typename T>
int sddmm_launch(const void* col, const void* rp, int64_t m, const void* Gm, int64_t ldg, const void* X, int64_t ldx,
                 int64_t ncols, double alpha, void* dv, hipStream_t st) {
  constexpr int VW = 16 / (int)sizeof(T);
  if (ncols % VW == 0 && ldg % VW == 0 && ldx % VW == 0 && ((uintptr_t)Gm % 16) == 0 && ((uintptr_t)X % 16) == 0)
    return sddmm_launch_v<IdxT, T, VW>(col, rp, m, Gm, ldg, X, ldx, ncols, alpha, dv, st);
  return sddmm_launch_v<IdxT, T, 1>(col, rp, m, Gm, ldg, X, ldx, ncols, alpha, dv, st);
}

template <typename IdxT>
int plan_launch(const void* row_ptrs, int64_t m, int64_t nwin, int64_t* win, hipStream_t st) {
  const int64_t grid = tsp::ceil_div(m + 1, 256);
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_plan: too many rows");
  hipLaunchKernelGGL((csr_plan_kernel<IdxT>), dim3((unsigned)grid), dim3(256), 0, st, (const IdxT*)row_ptrs, m, nwin, win);
  return tsp::check_launch("csr_plan launch");
}

template <typename IdxT, typename T>
int spmv_launch(const void* values, const void* col, const void* rp, const int64_t* win, int64_t nwin, const void* x,
                double alpha, const void* y, double beta, void* out, hipStream_t st) {
  if (nwin > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_spmv: too many windows");
  const T* yy = (y && beta != 0.0) ? (const T*)y : nullptr;
  hipLaunchKernelGGL((csr_spmv_kernel<IdxT, T>), dim3((unsigned)nwin), dim3(SPMV_THREADS), 0, st, (const T*)values,
                     (const IdxT*)col, (const IdxT*)rp, win, (const T*)x, (T)alpha, yy, (T)beta, (T*)out);
  return tsp::check_launch("csr_spmv launch");
}

template <typename IdxT, typename T>
int spmm_launch(const void* values, const void* col, const void* rp, int64_t m, const void* B, int64_t ldb,
                int64_t ncols, double alpha, const void* C, int64_t ldc, double beta, void* out, int64_t ldo,
                hipStream_t st) {
  const T* cc = (C && beta != 0.0) ? (const T*)C : nullptr;
  int64_t grid = tsp::ceil_div(m, 4);
  if (grid > 65536) grid = 65536;
#define TSP_SPMM(NC)                                                                                          \
  hipLaunchKernelGGL((csr_spmm_kernel<IdxT, T, NC>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)values, \
                     (const IdxT*)col, (const IdxT*)rp, m, (const T*)B, ldb, ncols, (T)alpha, cc, ldc, (T)beta,   \
                     (T*)out, ldo)
  if (ncols <= 64)
    TSP_SPMM(1);
  else if (ncols <= 128)
    TSP_SPMM(2);
  else
    TSP_SPMM(4);
#undef TSP_SPMM
  return tsp::check_launch("csr_spmm launch");
}

int check_types(const char* who, int dtype, int index_type) {
  if (dtype != TSP_F32 && dtype != TSP_F64) return tsp::fail(TSP_EUNSUPPORTED, "%s: dtype %d not supported (f32, f64)", who, dtype);
  if (index_type != TSP_I32 && index_type != TSP_I64) return tsp::fail(TSP_EINVAL, "%s: bad index_type %d", who, index_type);
  return TSP_OK;
}

}  // namespace

extern "C" int64_t tsp_csr_plan_size(int64_t m, int64_t nnz) {
  if (m < 0 || nnz < 0) return -1;
  return (m + nnz) / CAP + 2;  // nwin + 1 entries
}

extern "C" int tsp_csr_plan(const void* row_ptrs, int index_type, int64_t m, int64_t nnz, int64_t* windows, void* stream) {
  if (m < 0 || nnz < 0) return tsp::fail(TSP_EINVAL, "tsp_csr_plan: negative size");
  if (index_type != TSP_I32 && index_type != TSP_I64) return tsp::fail(TSP_EINVAL, "tsp_csr_plan: bad index_type");
  if (!row_ptrs || !windows) return tsp::fail(TSP_EINVAL, "tsp_csr_plan: null pointer");
  const int64_t nwin = (m + nnz) / CAP + 1;
  hipStream_t st = (hipStream_t)stream;
  return index_type == TSP_I64 ? plan_launch<int64_t>(row_ptrs, m, nwin, windows, st)
                               : plan_launch<int32_t>(row_ptrs, m, nwin, windows, st);
}

extern "C" int tsp_csr_spmv(const void* values, int dtype, const void* col_indices, const void* row_ptrs, int index_type,
                            int64_t m, int64_t n, int64_t nnz, const int64_t* windows, const void* x, double alpha,
                            const void* y, double beta, void* out, void* stream) {
  int st0 = check_types("tsp_csr_spmv", dtype, index_type);
  if (st0) return st0;
  if (m < 0 || n < 0 || nnz < 0) return tsp::fail(TSP_EINVAL, "tsp_csr_spmv: negative size");
  if (m == 0) return TSP_OK;
  if (!row_ptrs || !windows || !out || (nnz > 0 && (!values || !col_indices || !x)))
    return tsp::fail(TSP_EINVAL, "tsp_csr_spmv: null pointer");
  const int64_t nwin = (m + nnz) / CAP + 1;
  hipStream_t st = (hipStream_t)stream;
  if (index_type == TSP_I64)
    return dtype == TSP_F32 ? spmv_launch<int64_t, float>(values, col_indices, row_ptrs, windows, nwin, x, alpha, y, beta, out, st)
                            : spmv_launch<int64_t, double>(values, col_indices, row_ptrs, windows, nwin, x, alpha, y, beta, out, st);
  return dtype == TSP_F32 ? spmv_launch<int32_t, float>(values, col_indices, row_ptrs, windows, nwin, x, alpha, y, beta, out, st)
                          : spmv_launch<int32_t, double>(values, col_indices, row_ptrs, windows, nwin, x, alpha, y, beta, out, st);
}

extern "C" int tsp_csr_spmm(const void* values, int dtype, const void* col_indices, const void* row_ptrs, int index_type,
                            int64_t m, int64_t n, int64_t nnz, const void* B, int64_t ldb, int64_t ncols, double alpha,
                            const void* C, int64_t ldc, double beta, void* out, int64_t ldo, void* stream) {
  int st0 = check_types("tsp_csr_spmm", dtype, index_type);
  if (st0) return st0;
  if (m < 0 || n < 0 || nnz < 0 || ncols < 0) return tsp::fail(TSP_EINVAL, "tsp_csr_spmm: negative size");
  if (ldb < ncols || ldo < ncols || (C && beta != 0.0 && ldc < ncols))
    return tsp::fail(TSP_EINVAL, "tsp_csr_spmm: leading dimension < ncols");
  if (m == 0 || ncols == 0) return TSP_OK;
  if (!row_ptrs || !out || (nnz > 0 && (!values || !col_indices || !B)))
    return tsp::fail(TSP_EINVAL, "tsp_csr_spmm: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const bool a16 = ((uintptr_t)B % 16) == 0 && ((uintptr_t)out % 16) == 0 &&
                   (!(C && beta != 0.0) || (((uintptr_t)C % 16) == 0 && ldc % 4 == 0));
  if (dtype == TSP_F32 && ncols % 4 == 0 && ldb % 4 == 0 && ldo % 4 == 0 && a16)
    return index_type == TSP_I64
               ? spmm_narrow_launch<int64_t>(values, col_indices, row_ptrs, m, B, ldb, ncols, alpha, C, ldc, beta, out, ldo, st)
               : spmm_narrow_launch<int32_t>(values, col_indices, row_ptrs, m, B, ldb, ncols, alpha, C, ldc, beta, out, ldo, st);
  if (index_type == TSP_I64)
    return dtype == TSP_F32 ? spmm_launch<int64_t, float>(values, col_indices, row_ptrs, m, B, ldb, ncols, alpha, C, ldc, beta, out, ldo, st)
                            : spmm_launch<int64_t, double>(values, col_indices, row_ptrs, m, B, ldb, ncols, alpha, C, ldc, beta, out, ldo, st);
  return dtype == TSP_F32 ? spmm_launch<int32_t, float>(values, col_indices, row_ptrs, m, B, ldb, ncols, alpha, C, ldc, beta, out, ldo, st)
                          : spmm_launch<int32_t, double>(values, col_indices, row_ptrs, m, B, ldb, ncols, alpha, C, ldc, beta, out, ldo, st);
}

extern "C" int tsp_csr_sddmm(const void* col_indices, const void* row_ptrs, int index_type, int64_t m, int64_t n,
                             int64_t nnz, const void* G, int64_t ldg, const void* X, int64_t ldx, int64_t ncols,
                             int dtype, double alpha, void* out_values, void* stream) {
  int st0 = check_types("tsp_csr_sddmm", dtype, index_type);
  if (st0) return st0;
  if (m < 0 || n < 0 || nnz < 0 || ncols < 0) return tsp::fail(TSP_EINVAL, "tsp_csr_sddmm: negative size");
  if (ldg < ncols || ldx < ncols) return tsp::fail(TSP_EINVAL, "tsp_csr_sddmm: leading dimension < ncols");
  if (nnz == 0 || m == 0) return TSP_OK;
  if (!col_indices || !row_ptrs || !out_values || (ncols > 0 && (!G || !X)))
    return tsp::fail(TSP_EINVAL, "tsp_csr_sddmm: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (ncols == 0) {  // empty dot products
    return tsp::zero_fill(out_values, nnz * (dtype == TSP_F64 ? 8 : 4), st);
  }
  if (index_type == TSP_I64)
    return dtype == TSP_F32 ? sddmm_launch<int64_t, float>(col_indices, row_ptrs, m, G, ldg, X, ldx, ncols, alpha, out_values, st)
                            : sddmm_launch<int64_t, double>(col_indices, row_ptrs, m, G, ldg, X, ldx, ncols, alpha, out_values, st);
  return dtype == TSP_F32 ? sddmm_launch<int32_t, float>(col_indices, row_ptrs, m, G, ldg, X, ldx, ncols, alpha, out_values, st)
                          : sddmm_launch<int32_t, double>(col_indices, row_ptrs, m, G, ldg, X, ldx, ncols, alpha, out_values, st);
}
