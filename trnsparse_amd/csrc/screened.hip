// Schwarz-screened dense SpMM for gfx950:  C = (A * mask) @ B.
//
// Semantics follow the reference spec (trnsparse/ops.py:262-277):
//   Q[i]      = sqrt(|diag[i]|)                    (in diag's dtype)
//   mask[i,k] = Q[i] * Q[k] > sqrt(threshold)      (product and compare in
//               diag's dtype; torch converts the Python float threshold to it)
//   C         = (A * mask.to(A.dtype)) @ B
// The mask is never materialised: it is applied to A while A's k-slabs are
// staged (A * 1 or A * 0, so inf * 0 = NaN as in the reference), and the
// reference NKI kernel's soft mask (trnsparse/nki/kernels.py:129-134) is not
// used — the compare is the exact one.
//
// Tile skip: for the 128x128 tile pair (I, K), if fl(Qmax_I * Qmax_K) <= thr
// then every pair in it is masked (all Q >= 0 and rounded multiplication is
// monotonic), so the K tile is skipped. With finite A and B this is exactly
// the reference result; with non-finite entries inside a fully masked tile
// the reference would propagate NaN from inf * 0 and the skip does not.
//
// Kernels
//   screened_q          Q and the per-128-row-tile maximum of Q (workspace).
//   screened_f32_mfma   fp32, 128x128 C tile per workgroup on the shared MFMA
//                       core (mfma_f32.h); the K loop visits active k-tiles.
//   screened_generic    f64 or unaligned operands: one thread per output.
#include "mfma_f32.h"

namespace {

namespace T32 = tsp::f32tile;
constexpr int TILE = 128;
constexpr int KC = 64;

template <typename QT>
__device__ inline QT qsqrt(QT v);
template <>
__device__ inline float qsqrt<float>(float v) { return __fsqrt_rn(fabsf(v)); }
template <>
__device__ inline double qsqrt<double>(double v) { return __dsqrt_rn(fabs(v)); }

template <typename QT>
__global__ __launch_bounds__(TILE) void screened_q(const QT* __restrict__ diag, int64_t m, QT* __restrict__ Q,
                                                   QT* __restrict__ qmax) {
  __shared__ QT red[TILE / 64];
  const int64_t i = (int64_t)blockIdx.x * TILE + threadIdx.x;
  QT q = 0;
  if (i < m) {
    q = qsqrt<QT>(diag[i]);
    Q[i] = q;
  }
  // max ignoring NaN (a NaN Q never passes the compare)
  QT mx = q == q ? q : (QT)0;
  for (int o = 32; o > 0; o >>= 1) {
    QT other = __shfl_xor(mx, o, 64);
    mx = other > mx ? other : mx;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) qmax[blockIdx.x] = red[0] > red[1] ? red[0] : red[1];
}

template <typename QT>
struct ScreenedSlabs {
  const float* __restrict__ A;
  const float* __restrict__ B;
  const QT* __restrict__ Q;
  const QT* __restrict__ qmax;
  int64_t lda, ldb, m, ncols, row0, n0;
  QT thr, qI;
  int nkt;
  int kt;  // k tile of the current slab group (advanced as slabs are requested in order)
  T32::Coords<KC> q;

  __device__ bool active(int t) const { return qI * qmax[t] > thr; }
  __device__ int count() const {
    int c = 0;
    for (int t = 0; t < nkt; ++t) c += active(t) ? 1 : 0;
    return c;
  }
  __device__ void load(int s, f32x4 (&a)[T32::Slab<KC>::NA], f32x4 (&b)[T32::Slab<KC>::NB]) {
    constexpr int PER = TILE / KC;  // slabs per k tile
    if ((s % PER) == 0) {
      ++kt;
      while (!active(kt)) ++kt;
    }
    const int kk = (s % PER) * KC;
    const int64_t kc = (int64_t)kt * TILE + kk + q.ac;
    QT qk[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qk[i] = kc + i < m ? Q[kc + i] : (QT)0;
#pragma unroll
    for (int j = 0; j < T32::Slab<KC>::NA; ++j) {
      const int64_t r = row0 + q.ar + j * q.astep;
      a[j] = T32::load4_guard(A, r, kc, m, m, lda);
      const QT qa = r < m ? Q[r] : (QT)0;
#pragma unroll
      for (int i = 0; i < 4; ++i) a[j][i] *= (qa * qk[i] > thr) ? 1.0f : 0.0f;
    }
    const int64_t brow = (int64_t)kt * TILE + kk + q.br;
#pragma unroll
    for (int j = 0; j < T32::Slab<KC>::NB; ++j) b[j] = T32::load4_guard(B, brow + 16 * j, n0 + q.bc, m, ncols, ldb);
  }
};

template <typename QT>
__global__ __launch_bounds__(T32::NTHR) void screened_f32_mfma(
    const float* __restrict__ A, int64_t lda, const QT* __restrict__ Q, const QT* __restrict__ qmax, QT thr,
    int64_t m, const float* __restrict__ B, int64_t ldb, int64_t ncols, float* __restrict__ C, int64_t ldc, int nmt,
    int nnt) {
  __shared__ __attribute__((aligned(16))) float lds[T32::Slab<KC>::LDS_FLOATS];
  // XCD-aware: the column tiles of one row panel of A share an XCD (and its L2).
  int64_t mt64;
  int nt;
  if (!T32::tile_item(blockIdx.x, nmt, nnt, nullptr, mt64, nt)) return;
  const int mt = (int)mt64;

  ScreenedSlabs<QT> src;
  src.A = A;
  src.B = B;
  src.Q = Q;
  src.qmax = qmax;
  src.lda = lda;
  src.ldb = ldb;
  src.m = m;
  src.ncols = ncols;
  src.row0 = (int64_t)mt * TILE;
  src.n0 = (int64_t)nt * T32::BN;
  src.thr = thr;
  src.qI = qmax[mt];
  src.nkt = (int)tsp::ceil_div(m, TILE);
  src.kt = -1;
  const int nsteps = src.count() * (TILE / KC);

  f32x16 acc0 = {}, acc1 = {};
  T32::run<KC>(src, nsteps, lds, src.q, acc0, acc1);
  T32::store_tile(C, ldc, src.row0, src.n0, m, ncols, src.q, acc0, acc1, [](float v) { return v; });
}

template <typename T, typename QT>
__global__ __launch_bounds__(256) void screened_generic(const T* __restrict__ A, int64_t lda, const QT* __restrict__ Q,
                                                       QT thr, int64_t m, const T* __restrict__ B, int64_t ldb,
                                                       int64_t ncols, T* __restrict__ C, int64_t ldc) {
  typedef typename tsp::Acc<T>::type AccT;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= m * ncols) return;
  const int64_t i = t / ncols, c = t - i * ncols;
  const QT qi = Q[i];
  AccT acc = 0;
  for (int64_t k = 0; k < m; ++k) {
    const T a = A[i * lda + k] * ((qi * Q[k] > thr) ? (T)1 : (T)0);
    acc += (AccT)a * (AccT)B[k * ldb + c];
  }
  C[i * ldc + c] = (T)acc;
}

template <typename QT>
int launch(const void* A, int dtype, int64_t lda, const void* diag, double thr_sqrt, int64_t m, const void* B,
           int64_t ldb, int64_t ncols, void* C, int64_t ldc, void* ws, hipStream_t st) {
  const int64_t nmt = tsp::ceil_div(m, TILE);
  QT* Q = (QT*)ws;
  QT* qmax = Q + nmt * TILE;
  const QT thr = (QT)thr_sqrt;
  if (nmt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm: too many rows");
  hipLaunchKernelGGL((screened_q<QT>), dim3((unsigned)nmt), dim3(TILE), 0, st, (const QT*)diag, m, Q, qmax);
  int rc = tsp::check_launch("screened_q launch");
  if (rc) return rc;
  if (dtype == TSP_F32 && (lda % 4) == 0 && (ldb % 4) == 0 && ((uintptr_t)A % 16) == 0 && ((uintptr_t)B % 16) == 0) {
    const int64_t nnt = tsp::ceil_div(ncols, T32::BN);
    const int64_t grid = tsp::ceil_div(nmt, 8) * 8 * nnt;
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm: problem too large");
    hipLaunchKernelGGL((screened_f32_mfma<QT>), dim3((unsigned)grid), dim3(T32::NTHR), 0, st, (const float*)A, lda,
                       (const QT*)Q, (const QT*)qmax, thr, m, (const float*)B, ldb, ncols, (float*)C, ldc, (int)nmt,
                       (int)nnt);
    return tsp::check_launch("screened_f32_mfma launch");
  }
  const int64_t grid = tsp::ceil_div(m * ncols, 256);
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm: problem too large for the generic kernel");
  if (dtype == TSP_F32)
    hipLaunchKernelGGL((screened_generic<float, QT>), dim3((unsigned)grid), dim3(256), 0, st, (const float*)A, lda,
                       (const QT*)Q, thr, m, (const float*)B, ldb, ncols, (float*)C, ldc);
  else
    hipLaunchKernelGGL((screened_generic<double, QT>), dim3((unsigned)grid), dim3(256), 0, st, (const double*)A, lda,
                       (const QT*)Q, thr, m, (const double*)B, ldb, ncols, (double*)C, ldc);
  return tsp::check_launch("screened_generic launch");
}

}  // namespace

extern "C" int64_t tsp_screened_workspace_size(int64_t m, int diag_dtype) {
  if (m < 0 || (diag_dtype != TSP_F32 && diag_dtype != TSP_F64)) return -1;
  const int64_t nmt = tsp::ceil_div(m, TILE);
  return (nmt * TILE + nmt) * (diag_dtype == TSP_F64 ? 8 : 4);
}

extern "C" int tsp_screened_spmm(const void* A, int dtype, int64_t lda, const void* diag, int diag_dtype,
                                 double threshold_sqrt, int64_t m, const void* B, int64_t ldb, int64_t ncols, void* C,
                                 int64_t ldc, void* workspace, void* stream) {
  if (dtype != TSP_F32 && dtype != TSP_F64) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm: dtype %d not supported", dtype);
  if (diag_dtype != TSP_F32 && diag_dtype != TSP_F64)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm: diag dtype %d not supported", diag_dtype);
  if (m < 0 || ncols < 0) return tsp::fail(TSP_EINVAL, "tsp_screened_spmm: negative size");
  if (lda < m || ldb < ncols || ldc < ncols) return tsp::fail(TSP_EINVAL, "tsp_screened_spmm: leading dimension too small");
  if (m == 0 || ncols == 0) return TSP_OK;
  if (!A || !diag || !B || !C || !workspace) return tsp::fail(TSP_EINVAL, "tsp_screened_spmm: null pointer");
  hipStream_t st = (hipStream_t)stream;
  return diag_dtype == TSP_F32
             ? launch<float>(A, dtype, lda, diag, threshold_sqrt, m, B, ldb, ncols, C, ldc, workspace, st)
             : launch<double>(A, dtype, lda, diag, threshold_sqrt, m, B, ldb, ncols, C, ldc, workspace, st);
}
