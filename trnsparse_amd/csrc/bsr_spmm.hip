// Block-sparse (BSR) x dense SpMM for gfx950.
//
// Semantics follow the reference spec `_bsr_spmm_pytorch`
// (trnsparse/ops.py:162-192): for every block row i and every stored block
// idx in block_row_ptrs[i]:block_row_ptrs[i+1] with column block j,
//   C[i*b:(i+1)*b] += blocks[idx] @ B[j*b:(j+1)*b]
// with B rows beyond n read as zero (the reference pads B, :179-183) and only
// the first m rows of C produced (:192). Unlike the reference NKI path
// (trnsparse/nki/dispatch.py:230-287) no gathered copy of B is ever built:
// each workgroup reads the B row-panels of its block row in place.
//
// Kernels
//   bsr_spmm_f32_mfma  b == 128, fp32.  One workgroup = one 128x128 tile of C
//                      (block row i, column tile t). 8 waves in a 4(M)x2(N)
//                      grid, each wave a 32x64 sub-tile as two 32x32 MFMA
//                      accumulators (v_mfma_f32_32x32x2_f32). The K loop runs
//                      over the row's blocks in 32-wide k-slabs staged through
//                      a double-buffered LDS ring; the next slab's global
//                      loads are in flight while the current one is consumed.
//   bsr_spmm_generic   any block size / dtype (f32, f64, bf16): one thread per
//                      output element, a plain dot product over stored blocks.
//
// Scheduling: the grid is mapped XCD-aware. Consecutive workgroup ids go
// round-robin over the 8 XCDs, so item (row rank k, column tile t) is placed
// on XCD k%8 with the column tiles of one block row in consecutive slots of
// that XCD: the tiles sharing an A block run side by side on one L2. Rows are
// visited heaviest first (tsp_bsr_row_order), so the hardware dispatcher acts
// as a longest-processing-time list scheduler within each XCD.
#include "common.h"

namespace {

constexpr int BS = 128;          // block size served by the MFMA kernel
constexpr int TN = 128;          // C columns per workgroup
constexpr int KC = 32;           // k-slab per pipeline step
constexpr int NTHR = 512;        // 8 wavefronts
constexpr int A_LD = KC + 4;     // LDS row stride (floats) of the A slab [m][k]
constexpr int B_LD = TN + 4;     // LDS row stride (floats) of the B slab [k][n]
constexpr int A_SLAB = BS * A_LD;
constexpr int B_SLAB = KC * B_LD;
constexpr int STAGE = A_SLAB + B_SLAB;

// Load four consecutive B elements of row r starting at column c, zero-filled
// outside [0,n) x [0,ncols). Vector path needs c%4==0, ldb%4==0, 16B base.
__device__ inline f32x4 load_b4(const float* __restrict__ B, int64_t r, int64_t c, int64_t n,
                                int64_t ncols, int64_t ldb) {
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  if (r < n) {
    const float* p = B + r * ldb + c;
    if (c + 3 < ncols) {
      v = *(const f32x4*)p;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c + i < ncols) v[i] = p[i];
    }
  }
  return v;
}

template <typename OutT>
__device__ inline OutT cvt_out(float v);
template <>
__device__ inline float cvt_out<float>(float v) { return v; }
template <>
__device__ inline uint16_t cvt_out<uint16_t>(float v) { return tsp::f32_to_bf16_bits(v); }

template <typename OutT>
__global__ __launch_bounds__(NTHR) void bsr_spmm_f32_mfma(
    const float* __restrict__ blocks, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci,
    int64_t mb, int nt, int64_t m, int64_t n, const float* __restrict__ B, int64_t ldb,
    int64_t ncols, OutT* __restrict__ C, int64_t ldc, const int32_t* __restrict__ order) {
  __shared__ __attribute__((aligned(16))) float lds[2 * STAGE];

  // ---- work item (XCD-aware, heaviest rows first)
  const int g = blockIdx.x;
  const int xcd = g & 7, slot = g >> 3;
  const int64_t k = (int64_t)(slot / nt) * 8 + xcd;
  if (k >= mb) return;
  const int ntile = slot % nt;
  const int64_t row = order ? (int64_t)order[k] : k;
  const int64_t n0 = (int64_t)ntile * TN;
  const int64_t start = rp[row];
  const int nsteps = (int)(rp[row + 1] - start) * (BS / KC);

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wm = w & 3, wn = w >> 2;
  const int h = lane >> 5, l32 = lane & 31;

  // ---- staging coordinates: A slab 128x32, B slab 32x128, 2 float4 each
  const int ar = tid >> 3, ac = (tid & 7) * 4;
  const int br = tid >> 5, bc = (tid & 31) * 4;

  f32x4 ra0, ra1, rb0, rb1;
  auto gload = [&](int s) {
    const int64_t idx = start + (s >> 2);
    const int kk = (s & 3) * KC;
    const float* a = blocks + idx * (BS * BS) + kk;
    ra0 = *(const f32x4*)(a + ar * BS + ac);
    ra1 = *(const f32x4*)(a + (ar + 64) * BS + ac);
    const int64_t brow = ci[idx] * BS + kk + br;
    rb0 = load_b4(B, brow, n0 + bc, n, ncols, ldb);
    rb1 = load_b4(B, brow + 16, n0 + bc, n, ncols, ldb);
  };
  auto lstore = [&](float* st) {
    float* As = st;
    float* Bs = st + A_SLAB;
    *(f32x4*)(As + ar * A_LD + ac) = ra0;
    *(f32x4*)(As + (ar + 64) * A_LD + ac) = ra1;
    *(f32x4*)(Bs + br * B_LD + bc) = rb0;
    *(f32x4*)(Bs + (br + 16) * B_LD + bc) = rb1;
  };

  f32x16 acc0 = {}, acc1 = {};
  // MFMA k-step s of a group of 8 k values uses k = k0 + s (lanes 0-31) and
  // k = k0 + 4 + s (lanes 32-63): each lane reads its 4 A values as one
  // 16-byte LDS load. A and B use the same k permutation, so the sum is the
  // plain dot product over the 8 values.
  auto compute = [&](const float* st) {
    const float* As = st;
    const float* Bs = st + A_SLAB;
#pragma unroll
    for (int k0 = 0; k0 < KC; k0 += 8) {
      const f32x4 a = *(const f32x4*)(As + (wm * 32 + l32) * A_LD + k0 + 4 * h);
      const float* bp = Bs + (k0 + 4 * h) * B_LD + wn * 64 + l32;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float b0 = bp[s * B_LD];
        const float b1 = bp[s * B_LD + 32];
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b1, acc1, 0, 0, 0);
      }
    }
  };

  if (nsteps > 0) {
    gload(0);
    lstore(lds);
    __syncthreads();
    for (int s = 0; s < nsteps; ++s) {
      const float* cur = lds + (s & 1) * STAGE;
      float* nxt = lds + ((s + 1) & 1) * STAGE;
      const bool more = s + 1 < nsteps;
      if (more) gload(s + 1);
      compute(cur);
      if (more) lstore(nxt);
      __syncthreads();
    }
  }

  // ---- epilogue: 32x32 accumulator layout, lane holds column l32 and rows
  // 8*(v/4) + 4*h + v%4 for v = 0..15.
  const int64_t rbase = row * BS + wm * 32 + 4 * h;
  const int64_t c0 = n0 + wn * 64 + l32;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t r = rbase + 8 * (v >> 2) + (v & 3);
    if (r < m) {
      OutT* crow = C + r * ldc;
      if (c0 < ncols) crow[c0] = cvt_out<OutT>(acc0[v]);
      if (c0 + 32 < ncols) crow[c0 + 32] = cvt_out<OutT>(acc1[v]);
    }
  }
}

template <typename T, typename OutT>
__global__ __launch_bounds__(256) void bsr_spmm_generic(
    const T* __restrict__ blocks, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci,
    int64_t bs, int64_t m, int64_t n, const T* __restrict__ B, int64_t ldb, int64_t ncols,
    OutT* __restrict__ C, int64_t ldc) {
  typedef typename tsp::Acc<T>::type AccT;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= m * ncols) return;
  const int64_t r = t / ncols, c = t - r * ncols;
  const int64_t i = r / bs, rr = r - i * bs;
  AccT acc = 0;
  const int64_t e = rp[i + 1];
  for (int64_t idx = rp[i]; idx < e; ++idx) {
    const int64_t j0 = ci[idx] * bs;
    const T* a = blocks + (idx * bs + rr) * bs;
    const int64_t kmax = (n - j0) < bs ? (n - j0) : bs;
    for (int64_t cc = 0; cc < kmax; ++cc)
      acc += tsp::to_acc<T>(a[cc]) * tsp::to_acc<T>(B[(j0 + cc) * ldb + c]);
  }
  C[r * ldc + c] = tsp::from_acc<OutT>(acc);
}

// Heaviest-first ordering of block rows: counting sort on stored blocks per
// row (lengths clamped to NBIN-1; the order is only a schedule).
constexpr int NBIN = 1024;
__global__ __launch_bounds__(1024) void bsr_row_order_kernel(const int64_t* __restrict__ rp,
                                                             int64_t mb, int32_t* __restrict__ order) {
  __shared__ int cnt[NBIN];
  const int tid = threadIdx.x;
  for (int i = tid; i < NBIN; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  for (int64_t r = tid; r < mb; r += blockDim.x) {
    int64_t len = rp[r + 1] - rp[r];
    int bin = (int)(NBIN - 1 - (len < NBIN - 1 ? len : NBIN - 1));
    atomicAdd(&cnt[bin], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int i = 0; i < NBIN; ++i) {
      int c = cnt[i];
      cnt[i] = run;
      run += c;
    }
  }
  __syncthreads();
  for (int64_t r = tid; r < mb; r += blockDim.x) {
    int64_t len = rp[r + 1] - rp[r];
    int bin = (int)(NBIN - 1 - (len < NBIN - 1 ? len : NBIN - 1));
    int pos = atomicAdd(&cnt[bin], 1);
    order[pos] = (int32_t)r;
  }
}

template <typename T, typename OutT>
int launch_generic(const void* blocks, const int64_t* rp, const int64_t* ci, int64_t bs, int64_t m,
                   int64_t n, const void* B, int64_t ldb, int64_t ncols, void* C, int64_t ldc,
                   hipStream_t st) {
  const int64_t total = m * ncols;
  const int64_t grid = tsp::ceil_div(total, 256);
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm: output too large for the generic kernel");
  hipLaunchKernelGGL((bsr_spmm_generic<T, OutT>), dim3((unsigned)grid), dim3(256), 0, st,
                     (const T*)blocks, rp, ci, bs, m, n, (const T*)B, ldb, ncols, (OutT*)C, ldc);
  return tsp::check_launch("bsr_spmm_generic launch");
}

}  // namespace

extern "C" int tsp_bsr_row_order(const int64_t* block_row_ptrs, int64_t n_block_rows, int32_t* order,
                                 void* stream) {
  if (n_block_rows < 0) return tsp::fail(TSP_EINVAL, "tsp_bsr_row_order: n_block_rows < 0");
  if (n_block_rows == 0) return TSP_OK;
  if (!block_row_ptrs || !order) return tsp::fail(TSP_EINVAL, "tsp_bsr_row_order: null pointer");
  if (n_block_rows > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_row_order: too many block rows");
  hipLaunchKernelGGL(bsr_row_order_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, block_row_ptrs,
                     n_block_rows, order);
  return tsp::check_launch("bsr_row_order launch");
}

extern "C" int tsp_bsr_spmm(const void* blocks, int dtype, const int64_t* block_row_ptrs,
                            const int64_t* block_col_indices, int64_t n_blocks, int64_t block_size,
                            int64_t m, int64_t n, const void* B, int64_t ldb, int64_t ncols, void* C,
                            int64_t ldc, int out_dtype, const int32_t* row_order, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  if (block_size <= 0) return tsp::fail(TSP_EINVAL, "tsp_bsr_spmm: block_size must be positive");
  if (m < 0 || n < 0 || ncols < 0 || n_blocks < 0)
    return tsp::fail(TSP_EINVAL, "tsp_bsr_spmm: negative size");
  if (ldb < ncols || ldc < ncols) return tsp::fail(TSP_EINVAL, "tsp_bsr_spmm: leading dimension < ncols");
  const bool ok_types = (dtype == TSP_F32 && out_dtype == TSP_F32) || (dtype == TSP_F64 && out_dtype == TSP_F64) ||
                        (dtype == TSP_BF16 && (out_dtype == TSP_BF16 || out_dtype == TSP_F32));
  if (!ok_types) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm: dtype %d -> out_dtype %d not supported", dtype, out_dtype);
  if (m == 0 || ncols == 0) return TSP_OK;
  if (!block_row_ptrs || !C || (n > 0 && !B) || (n_blocks > 0 && (!blocks || !block_col_indices)))
    return tsp::fail(TSP_EINVAL, "tsp_bsr_spmm: null pointer");
  const int64_t mb = tsp::ceil_div(m, block_size);

  if (dtype == TSP_F32 && block_size == BS && (ldb % 4) == 0 && ((uintptr_t)B % 16) == 0 &&
      ((uintptr_t)blocks % 16) == 0) {
    const int64_t nt = tsp::ceil_div(ncols, TN);
    const int64_t grid = tsp::ceil_div(mb, 8) * 8 * nt;
    if (grid > INT32_MAX || nt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm: problem too large");
    hipLaunchKernelGGL((bsr_spmm_f32_mfma<float>), dim3((unsigned)grid), dim3(NTHR), 0, st, (const float*)blocks,
                       block_row_ptrs, block_col_indices, mb, (int)nt, m, n, (const float*)B, ldb, ncols,
                       (float*)C, ldc, row_order);
    return tsp::check_launch("bsr_spmm_f32_mfma launch");
  }
  if (dtype == TSP_F32) return launch_generic<float, float>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
  if (dtype == TSP_F64) return launch_generic<double, double>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
  if (out_dtype == TSP_F32) return launch_generic<uint16_t, float>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
  return launch_generic<uint16_t, uint16_t>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
}
