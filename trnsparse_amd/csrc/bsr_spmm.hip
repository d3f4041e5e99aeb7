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
//                      over the row's blocks in 64-wide k-slabs staged through
//                      a double-buffered LDS ring (137 KiB: one workgroup per
//                      CU); the next slab's loads are in flight while the
//                      current one is consumed.
//   bsr_spmm_bf16_mfma b == 128, bf16 in, fp32 accumulation, fp32/bf16 out
//                      (v_mfma_f32_32x32x16_bf16, B slabs transposed in LDS).
//   bsr_spmm_generic   any block size / dtype (f32, f64, bf16): one thread per
//                      output element, a plain dot product over stored blocks.
//
// Scheduling: rows are ranked heaviest first (tsp_bsr_row_order) and dealt
// to the 8 XCDs in boustrophedon order; the column tiles of one block row sit
// in consecutive slots of one XCD, so the tiles sharing an A block run side
// by side on one L2 (mfma_f32.h, tile_item). With one workgroup per CU the
// in-order hardware dispatcher is then a longest-processing-time list
// scheduler within each XCD.
#include "common.h"

#include "mfma_f32.h"

namespace {

namespace T32 = tsp::f32tile;
constexpr int BS = 128;  // block size served by the MFMA kernels
constexpr int KC = 64;   // fp32 k-slab (two slabs per stored block)

// Slab source of one (block row, column tile) item: slab s is k-slab s%2 of
// the (s/2)-th stored block of the row; B rows come straight from the
// row-panel of that block's column (no gathered copy of B).
struct BsrSlabs {
  const float* __restrict__ blocks;
  const int64_t* __restrict__ ci;
  const float* __restrict__ B;
  int64_t start, n, ncols, ldb, n0;
  T32::Coords<KC> q;
  __device__ void load(int s, f32x4 (&a)[T32::Slab<KC>::NA], f32x4 (&b)[T32::Slab<KC>::NB]) const {
    const int64_t idx = start + s / (BS / KC);
    const int kk = (s % (BS / KC)) * KC;
    const float* ab = blocks + idx * (BS * BS) + kk + q.ac;
#pragma unroll
    for (int i = 0; i < T32::Slab<KC>::NA; ++i) a[i] = *(const f32x4*)(ab + (q.ar + i * q.astep) * BS);
    const int64_t brow = ci[idx] * BS + kk + q.br;
#pragma unroll
    for (int i = 0; i < T32::Slab<KC>::NB; ++i) b[i] = T32::load4_guard(B, brow + 16 * i, n0 + q.bc, n, ncols, ldb);
  }
};

template <typename OutT>
__device__ inline OutT cvt_out(float v);
template <>
__device__ inline float cvt_out<float>(float v) { return v; }
template <>
__device__ inline uint16_t cvt_out<uint16_t>(float v) { return tsp::f32_to_bf16_bits(v); }

template <typename OutT>
__global__ __launch_bounds__(T32::NTHR) void bsr_spmm_f32_mfma(
    const float* __restrict__ blocks, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci,
    int64_t mb, int nt, int64_t m, int64_t n, const float* __restrict__ B, int64_t ldb,
    int64_t ncols, OutT* __restrict__ C, int64_t ldc, const int32_t* __restrict__ order) {
  __shared__ __attribute__((aligned(16))) float lds[T32::Slab<KC>::LDS_FLOATS];
  int64_t row;
  int ntile;
  if (!T32::tile_item(blockIdx.x, mb, nt, order, row, ntile)) return;

  BsrSlabs src;
  src.blocks = blocks;
  src.ci = ci;
  src.B = B;
  src.start = rp[row];
  src.n = n;
  src.ncols = ncols;
  src.ldb = ldb;
  src.n0 = (int64_t)ntile * T32::BN;
  const int nsteps = (int)(rp[row + 1] - src.start) * (BS / KC);

  f32x16 acc0 = {}, acc1 = {};
  T32::run<KC>(src, nsteps, lds, src.q, acc0, acc1);
  T32::store_tile(C, ldc, row * BS, src.n0, m, ncols, src.q, acc0, acc1, cvt_out<OutT>);
}

// ---------------------------------------------------------------- bf16 MFMA
//
// bsr_spmm_bf16_mfma: b == 128, bf16 operands, fp32 accumulation, fp32 or
// bf16 output. Same tile (128x128 of C per workgroup, 8 waves of 32x64) and
// scheduling as the fp32 kernel, with v_mfma_f32_32x32x16_bf16 on 64-wide
// k-slabs. Both MFMA operands need 8 consecutive k per lane: A blocks are
// [m][k] already; B panels are [k][n], so each B slab is transposed while
// staged (4 k x 8 n register patches written as 8-byte rows of Bt[n][k]).
namespace bf {
constexpr int KC = 64;
constexpr int LD = KC + 8;            // LDS row stride (bf16) of As[m][k] and Bt[n][k]
constexpr int A_ELEMS = 128 * LD;
constexpr int STAGE = 2 * A_ELEMS;    // As + Bt
}  // namespace bf

template <typename OutT>
__global__ __launch_bounds__(512) void bsr_spmm_bf16_mfma(
    const uint16_t* __restrict__ blocks, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci,
    int64_t mb, int nt, int64_t m, int64_t n, const uint16_t* __restrict__ B, int64_t ldb, int64_t ncols,
    OutT* __restrict__ C, int64_t ldc, const int32_t* __restrict__ order) {
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * bf::STAGE];

  int64_t row;
  int ntile;
  if (!T32::tile_item(blockIdx.x, mb, nt, order, row, ntile)) return;
  const int64_t n0 = (int64_t)ntile * 128;
  const int64_t start = rp[row];
  const int nsteps = (int)(rp[row + 1] - start) * (BS / bf::KC);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 3, wn = w >> 2, h = lane >> 5, l32 = lane & 31;
  // staging: A slab 128 x 64 -> 2 chunks of 8 per thread; B slab 64 x 128 as
  // 4k x 8n patches -> 256 patches, threads 0..255 one each
  const int ar = tid >> 3, ac = (tid & 7) * 8;       // rows ar, ar+64
  const int pk = (tid & 15) * 4, pn = (tid >> 4) * 8;  // patch (k 4, n 8), valid for tid < 256
  const bool bstage = tid < 256;

  u16x8 ra0, ra1, rb[4];
  auto gload = [&](int s) {
    const int64_t idx = start + (s >> 1);
    const int kk = (s & 1) * bf::KC;
    const uint16_t* a = blocks + idx * (BS * BS) + kk;
    ra0 = *(const u16x8*)(a + ar * BS + ac);
    ra1 = *(const u16x8*)(a + (ar + 64) * BS + ac);
    if (bstage) {
      const int64_t brow = ci[idx] * BS + kk + pk;
      const int64_t c = n0 + pn;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
        if (brow + j < n) {
          const uint16_t* p = B + (brow + j) * ldb + c;
          if (c + 7 < ncols) {
            v = *(const u16x8*)p;
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
              if (c + i < ncols) v[i] = p[i];
          }
        }
        rb[j] = v;
      }
    }
  };
  auto lstore = [&](uint16_t* st) {
    uint16_t* As = st;
    uint16_t* Bt = st + bf::A_ELEMS;
    *(u16x8*)(As + ar * bf::LD + ac) = ra0;
    *(u16x8*)(As + (ar + 64) * bf::LD + ac) = ra1;
    if (bstage) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u16x4 t = {rb[0][i], rb[1][i], rb[2][i], rb[3][i]};
        *(u16x4*)(Bt + (pn + i) * bf::LD + pk) = t;
      }
    }
  };

  f32x16 acc0 = {}, acc1 = {};
  auto compute = [&](const uint16_t* st) {
    const uint16_t* As = st;
    const uint16_t* Bt = st + bf::A_ELEMS;
#pragma unroll
    for (int ks = 0; ks < bf::KC / 16; ++ks) {
      const bf16x8 a = *(const bf16x8*)(As + (wm * 32 + l32) * bf::LD + 16 * ks + 8 * h);
      const bf16x8 b0 = *(const bf16x8*)(Bt + (wn * 64 + l32) * bf::LD + 16 * ks + 8 * h);
      const bf16x8 b1 = *(const bf16x8*)(Bt + (wn * 64 + 32 + l32) * bf::LD + 16 * ks + 8 * h);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b1, acc1, 0, 0, 0);
    }
  };

  if (nsteps > 0) {
    gload(0);
    lstore(lds);
    __syncthreads();
    for (int s = 0; s < nsteps; ++s) {
      const uint16_t* cur = lds + (s & 1) * bf::STAGE;
      uint16_t* nxt = lds + ((s + 1) & 1) * bf::STAGE;
      const bool more = s + 1 < nsteps;
      if (more) gload(s + 1);
      compute(cur);
      if (more) lstore(nxt);
      __syncthreads();
    }
  }
  T32::Coords<64> q;
  T32::store_tile(C, ldc, row * BS, n0, m, ncols, q, acc0, acc1, cvt_out<OutT>);
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
    const int64_t nt = tsp::ceil_div(ncols, T32::BN);
    const int64_t grid = tsp::ceil_div(mb, 8) * 8 * nt;
    if (grid > INT32_MAX || nt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm: problem too large");
    hipLaunchKernelGGL((bsr_spmm_f32_mfma<float>), dim3((unsigned)grid), dim3(T32::NTHR), 0, st, (const float*)blocks,
                       block_row_ptrs, block_col_indices, mb, (int)nt, m, n, (const float*)B, ldb, ncols,
                       (float*)C, ldc, row_order);
    return tsp::check_launch("bsr_spmm_f32_mfma launch");
  }
  if (dtype == TSP_BF16 && block_size == BS && (ldb % 8) == 0 && ((uintptr_t)B % 16) == 0 &&
      ((uintptr_t)blocks % 16) == 0) {
    const int64_t nt = tsp::ceil_div(ncols, 128);
    const int64_t grid = tsp::ceil_div(mb, 8) * 8 * nt;
    if (grid > INT32_MAX || nt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm: problem too large");
    if (out_dtype == TSP_F32)
      hipLaunchKernelGGL((bsr_spmm_bf16_mfma<float>), dim3((unsigned)grid), dim3(512), 0, st, (const uint16_t*)blocks,
                         block_row_ptrs, block_col_indices, mb, (int)nt, m, n, (const uint16_t*)B, ldb, ncols, (float*)C,
                         ldc, row_order);
    else
      hipLaunchKernelGGL((bsr_spmm_bf16_mfma<uint16_t>), dim3((unsigned)grid), dim3(512), 0, st,
                         (const uint16_t*)blocks, block_row_ptrs, block_col_indices, mb, (int)nt, m, n,
                         (const uint16_t*)B, ldb, ncols, (uint16_t*)C, ldc, row_order);
    return tsp::check_launch("bsr_spmm_bf16_mfma launch");
  }
  if (dtype == TSP_F32) return launch_generic<float, float>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
  if (dtype == TSP_F64) return launch_generic<double, double>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
  if (out_dtype == TSP_F32) return launch_generic<uint16_t, float>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
  return launch_generic<uint16_t, uint16_t>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
}
