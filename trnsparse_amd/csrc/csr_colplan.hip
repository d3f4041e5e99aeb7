// CSR SpMV over a cached column-sorted plan ("colplan") for gfx950.
//
// Semantics are the reference's spmv (trnsparse/ops.py:30-48):
//   out = alpha * (A @ x)   then  + beta * y   only if y and beta != 0.
//
// Why a plan. With the reference's CSR layout every nonzero gathers one
// 4-byte x value from a random column; on cfg2 (1 M x 1 M, 16 per row,
// uniform columns) each gather is its own L1->L2 request (18.8 M requests
// per SpMV, L2 hit rate 82 %, the misses refetching x lines from the MALL).
// The plan reorders the nonzeros once per pattern so that the gathers of
// one wavefront instruction fall on a few x lines:
//
//   tile (rb, g) = rows [rb*R, rb*R + R) x columns [g*Cg, g*Cg + Cg)
//   a tile's entries sorted by column (ties in row order), cut into epochs
//   of E = 4096 entries (the last one padded)
//
// A 64-lane instruction then covers 64 consecutive nonzeros in column
// order of R rows: at cfg2 density (R = 16384 rows, 0.25 nonzeros per
// column) about 256 columns, 8 lines of 128 bytes, coalesced by the address
// unit into 8 requests instead of 64. Each tile still reads its whole x
// slice through L1 once, so the x traffic is (m / R) x n x 4 bytes. 16384-
// row tiles (128 KiB of int64 LDS row sums, one 1024-thread workgroup per
// CU) in 4 column groups measured fastest on cfg2 (51.8 us; 8192-row tiles
// two per CU 61.2, 4096-row 73.2, 8 column groups 64.7).
//
// Row sums in exact fixed point. Float add atomics in LDS (ds_add_f32) run
// at a small fraction of the rate of integer LDS atomics on gfx950 (a tile
// kernel built on them took 108 us on cfg2 against 46 us with ds_add_u64),
// and integer sums do not depend on the order of the additions. So the plan
// keeps each value scaled by a power of two per row, v' = v * 2^(61 - e_r)
// with sum_j |v_rj| < 2^e_r (e_r from the row's largest value and entry
// count), a pre-pass finds max |x| < 2^e_x, and the tile kernel adds
// rint(v' * x * 2^-e_x) to the row's int64 sum in LDS with ds_add_u64: every
// partial sum stays below 2^61 units, a product of at least 2^23 units is
// an integer already (so the sum is the exact sum of the fp32 products), and
// a smaller nonzero one sets the row's bit in an inexact mask. Wavefronts
// run through their epochs with no barrier (the previous form of this
// kernel ordered every epoch's products by row through a 16-bit row-order
// position per entry and two LDS phases per epoch: 57.5 us on cfg2 against
// 51.8 us now, Zipf rows 185 against 161). The sums do not depend on the
// order of the additions, so results are the same on every run.
// With G column groups each tile writes its row sums (as fp32, in units of
// 2^(e_r + e_x - 61)) and its inexact mask to the workspace, and the finish
// kernel adds the G partials per row in group order, scales them and
// applies alpha / beta. It sums a row again from the caller's CSR arrays
// (fp32 products in CSR order, an fp64 sum) when x holds inf or NaN, when
// the row holds a non-finite value or a nonzero value that the scaling
// would push below the normal range, or when one of the row's products was
// rounded and the result is below cnt * 2^23 units (the rounding could then
// exceed 2^-24 of it).
//
// Plan buffer (device): toff (T+1 int64, first sorted entry of each tile),
// eoff (T+1 int64, first epoch of each tile), ent (8 bytes per padded entry:
// scaled value bits << 32 | row_in_tile << cbits | column_in_group), pos
// (uint32 per padded entry: position k in the pattern's entries, for new
// values on the same pattern, read at values[row_ptrs[0] + k]; 0xffffffff
// for padding), a 256-byte header holding row_ptrs[0] (int64), then the row
// exponents (int16 per row of the matrix). Inside an epoch, ent and pos are
// stored in the SpMV kernel's lane order (entry_slot below): one 16-byte
// load gives a lane two of its chunks' entries. The two per-entry arrays
// hold one more epoch of zeros past the last tile's, which the SpMV
// kernel's prefetch reads when a tile has no epoch left to prefetch.
#include <algorithm>

#include "common.h"

#include "radix_sort.h"

namespace {

constexpr int GEOM_RBITS = 0, GEOM_NRB = 1, GEOM_CBITS = 2, GEOM_G = 3, GEOM_T = 4, GEOM_KEYBITS = 5,
              GEOM_PLAN_BYTES = 6, GEOM_BUILD_BYTES = 7, GEOM_SPMV_BYTES = 8, GEOM_PMAX = 9;

constexpr int EBITS = 12;
constexpr int E = 1 << EBITS;  // entries per epoch
constexpr uint32_t POS_PAD = 0xffffffffu;
constexpr int SPMV_NT = 1024;                  // threads of the SpMV workgroup
constexpr int SPMV_W = SPMV_NT / 64;           // wavefronts of the SpMV workgroup

constexpr int SPMV_K = E / 64 / SPMV_W;       // 64-entry chunks per wavefront and epoch
static_assert(SPMV_K == 4, "a lane's entries are loaded as two 16-byte pieces");

// Fixed-point row sums: a plan value of row r is v * 2^(FX_TOP - e_r), so
// the values of a row add up to less than 2^FX_TOP; with x scaled by
// 2^-e_x (max |x| < 2^e_x) every partial sum of a row's products stays
// below 2^FX_TOP + (rounding), inside int64.
constexpr int FX_TOP = 61;
constexpr int16_t RX_REDO = 32767;  // row exponent of a row summed from the CSR arrays
constexpr int XMAX_BLOCKS = 1024;   // partial maxima of |x| written by the pre-pass (at most)

// Where column-order entry li = (j * W + w) * 64 + l of an epoch (chunk j of
// wavefront w, lane l) is stored: wavefront w's entries are one contiguous
// E/W block, in which 16-byte piece q of lane l holds its chunks 2q and
// 2q + 1, so each load of a wavefront reads 1 KiB contiguously.
__host__ __device__ constexpr int entry_slot(int li) {
  return ((li >> 6) % SPMV_W) * (E / SPMV_W) + (((li >> 6) / SPMV_W) >> 1) * 128 + 2 * (li & 63) +
         (((li >> 6) / SPMV_W) & 1);
}

int ilog2_ceil(int64_t v) {
  int b = 0;
  while (((int64_t)1 << b) < v) ++b;
  return b;
}

int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

__device__ inline int64_t upper_bound_i64(const int64_t* __restrict__ a, int64_t n, int64_t v) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (a[mid] <= v)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// ------------------------------------------------------------ plan build

// Sort key (tile, column in group) and payload (row in tile, CSR position)
// of every entry, entry-parallel: a workgroup takes KTILE consecutive
// entries, finds the rows they span by binary search of row_ptrs, stages
// those row pointers in LDS when there are at most KSPAN of them, and gives
// each entry its row by a search of the staged span (one thread per row
// would read the column indices uncoalesced and stall on a long row).
constexpr int KTILE = 4096;
constexpr int KSPAN = 2048;

template <typename IdxT>
__device__ inline int64_t row_of(const IdxT* __restrict__ ptr, int64_t m, int64_t p) {
  int64_t lo = 0, hi = m;  // ptr[lo] <= p < ptr[hi]: the last row starting at or before p
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)ptr[mid] <= p)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

template <typename IdxT, typename K>
__global__ __launch_bounds__(256) void colplan_keys_kernel(const IdxT* __restrict__ col, const IdxT* __restrict__ ptr,
                                                           int64_t m, int64_t nnz, int rbits, int cbits, int64_t G,
                                                           K* __restrict__ keys, uint64_t* __restrict__ payload,
                                                           int64_t* __restrict__ plan_base) {
  __shared__ int64_t srp[KSPAN + 1];
  __shared__ int64_t span[2];
  // p = base + k: position in the caller's arrays; k < nnz: position in the
  // sort, the one the plan keeps (base may be any row_ptrs[0])
  const int64_t base = (int64_t)ptr[0];
  if (blockIdx.x == 0 && threadIdx.x == 0) plan_base[0] = base;
  const int64_t e0 = (int64_t)blockIdx.x * KTILE;
  const int64_t e1 = e0 + KTILE < nnz ? e0 + KTILE : nnz;
  if (threadIdx.x == 0) {
    span[0] = row_of(ptr, m, base + e0);
    span[1] = row_of(ptr, m, base + e1 - 1);
  }
  __syncthreads();
  const int64_t rlo = span[0], nr = span[1] - rlo + 1;
  const bool staged = nr <= KSPAN;
  if (staged)
    for (int64_t i = threadIdx.x; i <= nr; i += 256) srp[i] = (int64_t)ptr[rlo + i];
  __syncthreads();
  const int64_t rmask = ((int64_t)1 << rbits) - 1, cmask = ((int64_t)1 << cbits) - 1;
  for (int64_t k = e0 + threadIdx.x; k < e1; k += 256) {
    const int64_t p = base + k;
    int64_t r;
    if (staged) {
      int lo = 0, hi = (int)nr;  // srp[lo] <= p < srp[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (srp[mid] <= p)
          lo = mid;
        else
          hi = mid;
      }
      r = rlo + lo;
    } else {
      r = row_of(ptr, m, p);
    }
    const int64_t c = (int64_t)col[p];
    const int64_t tile = (r >> rbits) * G + (c >> cbits);
    keys[k] = (K)((tile << cbits) | (c & cmask));
    payload[k] = ((uint64_t)(r & rmask) << 32) | (uint64_t)k;
  }
}

// toff[t] = first sorted entry of tile t (lower bound of t << cbits).
template <typename K>
__global__ __launch_bounds__(256) void colplan_offsets_kernel(const K* __restrict__ keys, int64_t nnz, int cbits,
                                                              int64_t T, int64_t* __restrict__ toff) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t > T) return;
  const K target = (K)t << cbits;
  int64_t lo = 0, hi = nnz;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < target)
      lo = mid + 1;
    else
      hi = mid;
  }
  toff[t] = lo;
}

// eoff = exclusive scan of the tiles' epoch counts (one workgroup).
__global__ __launch_bounds__(1024) void colplan_epochs_kernel(const int64_t* __restrict__ toff, int64_t T,
                                                              int64_t* __restrict__ eoff) {
  __shared__ int64_t part[1024];
  const int tid = threadIdx.x;
  const int64_t per = (T + 1023) / 1024;
  const int64_t t0 = tid * per, t1 = t0 + per < T ? t0 + per : T;
  int64_t s = 0;
  for (int64_t t = t0; t < t1; ++t) s += (toff[t + 1] - toff[t] + E - 1) >> EBITS;
  part[tid] = s;
  __syncthreads();
  if (tid == 0) {
    int64_t run = 0;
    for (int i = 0; i < 1024; ++i) {
      const int64_t v = part[i];
      part[i] = run;
      run += v;
    }
  }
  __syncthreads();
  s = part[tid];
  for (int64_t t = t0; t < t1; ++t) {
    eoff[t] = s;
    s += (toff[t + 1] - toff[t] + E - 1) >> EBITS;
  }
  if (tid == 1023) eoff[T] = s;
}

__global__ __launch_bounds__(256) void colplan_fill_kernel(uint64_t* __restrict__ ent, uint32_t* __restrict__ pos,
                                                           int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  ent[i] = 0;
  pos[i] = POS_PAD;
}

// Row exponent e_r of the fixed-point row sums: with cnt entries and
// max |v| < 2^emx, sum |v| < 2^(emx + ceil(log2 cnt)) = 2^e_r, so the plan's
// values v * 2^(FX_TOP - e_r) add up to less than 2^FX_TOP in magnitude.
// RX_REDO marks a row the finish kernel always sums from the CSR arrays
// instead: a non-finite value, or a smallest nonzero value that scaling
// would push below the normal range (its products would lose bits).
__device__ inline int16_t row_exponent(uint32_t mx, uint32_t mn, int64_t cnt) {
  if (mx == 0) return 0;  // no nonzero value: every product is zero
  if (mx >= 0x7f800000u) return RX_REDO;
  const int emx = (int)(mx >> 23) == 0 ? -126 : (int)(mx >> 23) - 126;
  const int lg = cnt > 1 ? 64 - __builtin_clzll((uint64_t)(cnt - 1)) : 0;
  const int er = emx + lg;
  const int emn = (int)(mn >> 23) == 0 ? -149 : (int)(mn >> 23) - 127;  // mn >= 2^emn
  if (emn + FX_TOP - er < -126) return RX_REDO;
  return (int16_t)er;
}

// LANES lanes per row (build and refresh only): lanes stride the row's
// entries, xor shuffles combine the max and the smallest nonzero. 16 lanes
// when rows average at most 32 entries, else 64: a wavefront then waits on
// one row instead of on the longest of four.
template <typename IdxT, int LANES>
__global__ __launch_bounds__(256) void colplan_rowexp_kernel(const float* __restrict__ vals,
                                                             const IdxT* __restrict__ ptr, int64_t m,
                                                             int16_t* __restrict__ rexp) {
  const int64_t r = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / LANES;
  const int sub = threadIdx.x % LANES;
  int64_t p0 = 0, p1 = 0;
  if (r < m) {
    p0 = (int64_t)ptr[r];
    p1 = (int64_t)ptr[r + 1];
  }
  uint32_t mx = 0, mn = 0xffffffffu;
  for (int64_t p = p0 + sub; p < p1; p += LANES) {
    const uint32_t b = __float_as_uint(vals[p]) & 0x7fffffffu;
    mx = b > mx ? b : mx;
    if (b != 0 && b < mn) mn = b;
  }
  for (int o = LANES / 2; o > 0; o >>= 1) {
    const uint32_t a = (uint32_t)__shfl_xor((int)mx, o, LANES);
    const uint32_t c = (uint32_t)__shfl_xor((int)mn, o, LANES);
    mx = a > mx ? a : mx;
    mn = c < mn ? c : mn;
  }
  if (r < m && sub == 0) rexp[r] = row_exponent(mx, mn, p1 - p0);
}

// The plan's form of value v in global row r: v * 2^(FX_TOP - e_r) (zero
// for the rows summed from the CSR arrays).
__device__ inline uint32_t plan_value(float v, int16_t er) {
  return er == RX_REDO ? 0u : __float_as_uint(ldexpf(v, FX_TOP - (int)er));
}

// Sorted entry i of tile t is column-order entry j % E of epoch eoff[t] + j / E
// (j = i - toff[t]), stored at entry_slot(j % E) of that epoch.
template <typename K>
__global__ __launch_bounds__(256) void colplan_scatter_kernel(const K* __restrict__ keys,
                                                              const uint64_t* __restrict__ payload,
                                                              const float* __restrict__ vals, int64_t nnz, int rbits,
                                                              int cbits, int64_t G, const int64_t* __restrict__ toff,
                                                              const int64_t* __restrict__ eoff, int64_t T,
                                                              const int64_t* __restrict__ plan_base,
                                                              const int16_t* __restrict__ rexp,
                                                              uint64_t* __restrict__ ent, uint32_t* __restrict__ pos) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  const int64_t t = upper_bound_i64(toff, T + 1, i) - 1;
  const int64_t j = i - toff[t];
  const int64_t P = ((eoff[t] + (j >> EBITS)) << EBITS) + entry_slot((int)(j & (E - 1)));
  const uint64_t pl = payload[i];
  const uint32_t p = (uint32_t)pl;  // position k in the sort; the value sits at base + k
  const uint32_t rl = (uint32_t)(pl >> 32);
  const uint32_t cin = (uint32_t)(keys[i] & (((K)1 << cbits) - 1));
  const int64_t row = ((t / G) << rbits) | rl;
  ent[P] = ((uint64_t)plan_value(vals[plan_base[0] + p], rexp[row]) << 32) | (uint64_t)((rl << cbits) | cin);
  pos[P] = p;
}

// New values on the plan's pattern: plan position i holds CSR position
// pos[i]; its row block comes from the tile of its epoch.
__global__ __launch_bounds__(256) void colplan_refresh_kernel(const float* __restrict__ vals,
                                                              const uint32_t* __restrict__ pos, int64_t n,
                                                              const int64_t* __restrict__ plan_base,
                                                              const int64_t* __restrict__ eoff, int64_t T, int64_t G,
                                                              int rbits, int cbits, const int16_t* __restrict__ rexp,
                                                              uint64_t* __restrict__ ent) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t p = pos[i];
  uint32_t bits = 0;
  if (p != POS_PAD) {
    const int64_t t = upper_bound_i64(eoff, T + 1, i >> EBITS) - 1;
    const int64_t row = ((t / G) << rbits) | ((uint32_t)ent[i] >> cbits);
    bits = plan_value(vals[plan_base[0] + p], rexp[row]);
  }
  ent[i] = ((uint64_t)bits << 32) | (ent[i] & 0xffffffffull);
}

// ----------------------------------------------------------------- SpMV

// Partial maxima of |x| as float bits without the sign (an integer max
// orders them like the values; inf and NaN come out >= 0x7f800000): one
// 16-byte load per thread and trip (vec4, x 16-byte aligned), so a cold x
// takes one memory round trip.
__global__ __launch_bounds__(256) void colplan_xmax_kernel(const float* __restrict__ x, int64_t n, int vec4,
                                                           uint32_t* __restrict__ xpart) {
  __shared__ uint32_t wm[4];
  uint32_t mx = 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t t0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  auto take = [&](float f) {
    const uint32_t b = __float_as_uint(f) & 0x7fffffffu;
    mx = b > mx ? b : mx;
  };
  if (vec4) {
    const int64_t n4 = n >> 2;
    for (int64_t i = t0; i < n4; i += stride) {
      const f32x4 v = reinterpret_cast<const f32x4*>(x)[i];
      take(v[0]);
      take(v[1]);
      take(v[2]);
      take(v[3]);
    }
    for (int64_t i = (n4 << 2) + t0; i < n; i += stride) take(x[i]);
  } else {
    for (int64_t i = t0; i < n; i += stride) take(x[i]);
  }
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t v = (uint32_t)__shfl_xor((int)mx, o, 64);
    mx = v > mx ? v : mx;
  }
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t v = wm[0];
    for (int i = 1; i < 4; ++i) v = wm[i] > v ? wm[i] : v;
    xpart[blockIdx.x] = v;
  }
}

// Max |x| bits from the pre-pass's partial maxima, read by wavefront 0 of
// the calling workgroup into *dst (LDS).
__device__ inline void reduce_xmax(const uint32_t* __restrict__ xpart, int nxpart, uint32_t* dst) {
  if (threadIdx.x < 64) {
    uint32_t mx = 0;
#pragma unroll 4
    for (int i = threadIdx.x; i < nxpart; i += 64) {
      const uint32_t v = xpart[i];
      mx = v > mx ? v : mx;
    }
    for (int o = 32; o > 0; o >>= 1) {
      const uint32_t v = (uint32_t)__shfl_xor((int)mx, o, 64);
      mx = v > mx ? v : mx;
    }
    if (threadIdx.x == 0) *dst = mx;
  }
}

// e_x with max |x| < 2^e_x (0 when x is all zeros: every product is zero).
__device__ inline int x_exponent(uint32_t xm) {
  if (xm == 0) return 0;
  return (int)(xm >> 23) == 0 ? -126 : (int)(xm >> 23) - 126;
}

// One workgroup per tile: the tile's entries in column order, epoch by
// epoch. Each product p = v' * (x * 2^-e_x) (v' the plan's scaled value)
// is rounded to an integer and added to the row's int64 sum in LDS with
// ds_add_u64: integer sums do not depend on the order of the additions, so
// the wavefronts run through their epochs without barriers and the result
// is the same on every run. A product of magnitude >= 2^23 is an integer
// already (the rounding is exact); a smaller nonzero one sets the row's bit
// in the tile's inexact mask, which the finish kernel weighs against the
// row's result. The tile writes its row sums (in units of the row's
// 2^(e_r + e_x - FX_TOP), as fp32) and its inexact mask to the workspace.
template <int RBITS, int NT>
__global__ __launch_bounds__(NT) void colplan_spmv_fx(const uint64_t* __restrict__ ent,
                                                      const int64_t* __restrict__ toff,
                                                      const int64_t* __restrict__ eoff, const float* __restrict__ x,
                                                      uint32_t* __restrict__ xpart, int nxpart, int cbits,
                                                      int64_t G, int64_t nrb, int64_t pmax, int xcd_map,
                                                      float* __restrict__ partial, uint32_t* __restrict__ inexact) {
  constexpr int R = 1 << RBITS;
  constexpr int W = NT / 64;
  constexpr int K = E / 64 / W;  // chunks per wavefront and epoch
  constexpr int SPAN = E / W;    // entries per wavefront and epoch
  static_assert(W == SPMV_W && K == SPMV_K, "the plan's layout is made for this workgroup size");
  typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
  __shared__ unsigned long long acc[R];
  __shared__ uint32_t flag[R / 32];
  __shared__ uint32_t xm_s;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t T = nrb * G;
  // q runs over tiles group-major; with xcd_map, XCD k (= blockIdx % 8)
  // takes the k-th eighth of that order, so an XCD works on one column
  // group (or a run of consecutive groups) and keeps its x slice in L2.
  const int64_t q = xcd_map ? (int64_t)(blockIdx.x & 7) * (T >> 3) + (blockIdx.x >> 3) : (int64_t)blockIdx.x;
  const int64_t g = q / nrb, rb = q - g * nrb;
  const int64_t t = rb * G + g;

  const int64_t cnt_t = toff[t + 1] - toff[t];
  const int64_t ep0 = eoff[t], nep = eoff[t + 1] - ep0;
  const float* __restrict__ xg = x + (g << cbits);
  const uint32_t cmask = (1u << cbits) - 1u;

  // Software pipeline over epochs with three register sets of entries and
  // two of gathered x values: in epoch k a wavefront issues the x gathers
  // of epoch k + 1, adds epoch k's products (x gathered one epoch earlier)
  // and refills epoch k's entry set with epoch k + 3. Chunks past the
  // tile's entries read the plan's zero epoch after all tiles, so every
  // load is unconditional and the padding is never fetched.
  uint64_t evA[K], evB[K], evC[K];
  float xa[K], xb[K];
  auto load_epoch = [&](uint64_t (&ev)[K], int64_t k) {
    const int64_t left = cnt_t - (k << EBITS);  // entries of epoch k (<= 0 past the tile's end)
    const int64_t eb = (ep0 + k) << EBITS;
#pragma unroll
    for (int h = 0; h < K / 2; ++h) {
      // the pair's first chunk 2h starts at column-order entry (2h * W + w) * 64
      const int64_t src = (int64_t)((2 * h * W + w) * 64) < left ? eb : pmax;
      const u64x2 v = __builtin_nontemporal_load(reinterpret_cast<const u64x2*>(ent + src + w * SPAN) + h * 64 + lane);
      ev[2 * h] = v.x;
      ev[2 * h + 1] = v.y;
    }
  };
  auto gather = [&](float (&xv)[K], const uint64_t (&ev)[K]) {
#pragma unroll
    for (int j = 0; j < K; ++j) xv[j] = xg[(uint32_t)ev[j] & cmask];
  };
  // the first epochs' loads go out before the row sums are cleared and the
  // x maximum is read, so their latency overlaps both
  if (nep > 0) {
    load_epoch(evA, 0);
    load_epoch(evB, 1);
    load_epoch(evC, 2);
  }
  for (int i = tid; i < R; i += NT) acc[i] = 0ull;
  for (int i = tid; i < R / 32; i += NT) flag[i] = 0u;
  reduce_xmax(xpart, nxpart, &xm_s);
  if (nep > 0) gather(xa, evA);
  __syncthreads();
  const uint32_t xm = xm_s;
  if (blockIdx.x == 0 && tid == 0) xpart[XMAX_BLOCKS] = xm;  // for the finish kernel
  if (xm >= 0x7f800000u) return;  // x holds inf or NaN: the finish kernel sums every row from the CSR arrays
  const int nex = -x_exponent(xm);

  auto epoch = [&](uint64_t (&ev)[K], const float (&xv)[K], const uint64_t (&evn)[K], float (&xvn)[K], int64_t k) {
    const int64_t left = cnt_t - (k << EBITS);
    const int cnt = left < E ? (int)left : E;
    gather(xvn, evn);
#pragma unroll
    for (int j = 0; j < K; ++j) {
      // column-order index (j * W + w) * 64 + lane < cnt, with the chunk
      // offset moved to the (uniform) right-hand side
      if (w * 64 + lane < cnt - j * W * 64) {
        const float v = __uint_as_float((uint32_t)(ev[j] >> 32));
        const float p = v * ldexpf(xv[j], nex);
        const uint32_t row = ((uint32_t)ev[j] >> cbits) & (R - 1);
        atomicAdd(&acc[row], (unsigned long long)(long long)rintf(p));
        if (fabsf(p) < 8388608.f && v != 0.f && xv[j] != 0.f) atomicOr(&flag[row >> 5], 1u << (row & 31));
      }
    }
    // unconditional (past the tile's end it reads the zero epoch), so no
    // path without these loads makes the compiler wait for them early
    load_epoch(ev, k + 3);
  };

  // Six epochs per trip (the period of three entry sets and two x sets),
  // the rest after the loop: with later epochs of a trip conditional, the
  // compiler's wait analysis assumes the paths that skip them and waits for
  // the newest stream loads.
  int64_t k = 0;
  for (; k + 5 < nep; k += 6) {
    epoch(evA, xa, evB, xb, k);
    epoch(evB, xb, evC, xa, k + 1);
    epoch(evC, xa, evA, xb, k + 2);
    epoch(evA, xb, evB, xa, k + 3);
    epoch(evB, xa, evC, xb, k + 4);
    epoch(evC, xb, evA, xa, k + 5);
  }
  if (k < nep) epoch(evA, xa, evB, xb, k);
  if (k + 1 < nep) epoch(evB, xb, evC, xa, k + 1);
  if (k + 2 < nep) epoch(evC, xa, evA, xb, k + 2);
  if (k + 3 < nep) epoch(evA, xb, evB, xa, k + 3);
  if (k + 4 < nep) epoch(evB, xa, evC, xb, k + 4);
  __syncthreads();

  // the workspace holds nrb * R rows per group (rows past m stay zero)
  float* __restrict__ pg = partial + (g * nrb + rb) * R;
  for (int i = tid; i < R; i += NT) pg[i] = (float)(long long)acc[i];
  uint32_t* __restrict__ fg = inexact + (g * nrb + rb) * (R / 32);
  for (int i = tid; i < R / 32; i += NT) fg[i] = flag[i];
}

// Row r of the result: y_r = the sum of the G group partials (added in
// group order) scaled by 2^(e_r + e_x - FX_TOP), then alpha * y_r (+ beta *
// y[r]). The row is summed from the CSR arrays instead (fp32 products in
// CSR order, an fp64 sum) when x holds inf or NaN, when the row's exponent
// says so, or when one of its products was rounded and |y_r| is below
// cnt * 2^23 units: then the rounding (at most half a unit per product)
// could exceed 2^-24 of the result. Rows of up to REDO_SERIAL entries are
// summed by their own thread; longer ones by the whole wavefront (lanes
// stride the row, fp64 partial sums, then a fixed xor tree), so a long
// row on the slow path costs a few memory round trips, not one per entry.
constexpr int REDO_SERIAL = 32;

template <typename IdxT>
__device__ inline double redo_serial(int64_t r, const float* __restrict__ vals, const IdxT* __restrict__ cols,
                                     const IdxT* __restrict__ ptr, const float* __restrict__ x) {
  double a = 0.0;
  for (int64_t p = (int64_t)ptr[r]; p < (int64_t)ptr[r + 1]; ++p) a += (double)(vals[p] * x[(int64_t)cols[p]]);
  return a;
}

// Four rows per thread (m % 4 == 0, 16-byte aligned out and y: VEC) or one.
// Every lane stays to the end (the wavefront-wide sums need all lanes).
template <typename IdxT, bool VEC>
__global__ __launch_bounds__(256) void colplan_finish_fx(const float* __restrict__ partial,
                                                         const uint32_t* __restrict__ inexact, int64_t prows,
                                                         int64_t G, const int16_t* __restrict__ rexp,
                                                         const uint32_t* __restrict__ xmax,
                                                         const float* __restrict__ vals,
                                                         const IdxT* __restrict__ cols, const IdxT* __restrict__ ptr,
                                                         const float* __restrict__ x, int64_t m, float alpha,
                                                         const float* __restrict__ y, float beta,
                                                         float* __restrict__ out) {
  constexpr int NR = VEC ? 4 : 1;
  const int64_t r0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * NR;
  const bool live = r0 < m;
  const int lane = threadIdx.x & 63;
  const uint32_t xm = *xmax;
  float s[NR];
  uint32_t fl = 0;  // inexact bits of the NR rows
  int16_t er[NR];
  if (live) {
    if (VEC) {
      f32x4 acc = *reinterpret_cast<const f32x4*>(partial + r0);
      fl = inexact[r0 >> 5];
      for (int64_t g = 1; g < G; ++g) {
        acc += *reinterpret_cast<const f32x4*>(partial + g * prows + r0);
        fl |= inexact[g * (prows >> 5) + (r0 >> 5)];
      }
      typedef short s16x4 __attribute__((ext_vector_type(4)));
      const s16x4 e4 = *reinterpret_cast<const s16x4*>(rexp + r0);
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        s[i] = acc[i];
        er[i] = e4[i];
      }
    } else {
      s[0] = 0.f;
      for (int64_t g = 0; g < G; ++g) {
        s[0] += partial[g * prows + r0];
        fl |= inexact[g * (prows >> 5) + (r0 >> 5)];
      }
      er[0] = rexp[r0];
    }
    fl >>= (r0 & 31);
  }
  // which rows need the CSR arrays: bit i of `lng` = long row i of this lane
  uint32_t lng = 0;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    if (!live) break;
    const int64_t r = r0 + i;
    bool redo = xm >= 0x7f800000u || er[i] == RX_REDO;
    if (!redo) {
      const int sh = (int)er[i] + x_exponent(xm) - FX_TOP;
      s[i] = ldexpf(s[i], sh);
      if (((fl >> i) & 1u) && fabsf(s[i]) < ldexpf((float)((int64_t)ptr[r + 1] - (int64_t)ptr[r]), sh + 23))
        redo = true;
    }
    if (redo) {
      if ((int64_t)ptr[r + 1] - (int64_t)ptr[r] <= REDO_SERIAL)
        s[i] = (float)redo_serial(r, vals, cols, ptr, x);
      else
        lng |= 1u << i;
    }
  }
  // long rows, one at a time, by the whole wavefront
  for (;;) {
    const int mine = lng ? __builtin_ctz(lng) : -1;
    const uint64_t b = __ballot(mine >= 0);
    if (b == 0) break;
    const int src = __builtin_ctzll(b);
    const int which = __shfl(mine, src, 64);
    const int64_t r = ((int64_t)__shfl((int)(r0 >> 32), src, 64) << 32 | (uint32_t)__shfl((int)(uint32_t)r0, src, 64)) + which;
    const int64_t p0 = (int64_t)ptr[r], p1 = (int64_t)ptr[r + 1];
    double a = 0.0;
    for (int64_t p = p0 + lane; p < p1; p += 64) a += (double)(vals[p] * x[(int64_t)cols[p]]);
    for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o, 64);
    if (lane == src) {
#pragma unroll
      for (int i = 0; i < NR; ++i)
        if (i == which) s[i] = (float)a;
      lng &= ~(1u << which);
    }
  }
  if (!live) return;
  float res[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    res[i] = alpha * s[i];
    if (y) res[i] = res[i] + beta * y[r0 + i];
  }
  if (VEC)
    *reinterpret_cast<f32x4*>(out + r0) = f32x4{res[0], res[1 % NR], res[2 % NR], res[3 % NR]};
  else
    out[r0] = res[0];
}

// ------------------------------------------------------------- geometry

constexpr int RBITS_MAX = 14;          // 16384 rows: 128 KiB of int64 row sums per workgroup
constexpr int RBITS_DEFAULT = 14;      // one x-slice read per 16384 rows (the gathers' L1 fill halves against 8192)
constexpr int64_t TILES_TARGET = 256;  // one 1024-thread workgroup per CU

int geometry(int64_t m, int64_t n, int64_t nnz, int rbits_hint, int64_t tiles_hint, int64_t* g) {
  if (m <= 0 || n <= 0 || nnz < 0) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_geometry: bad size");
  if (nnz > (int64_t)UINT32_MAX - 1) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan: more than 2^32-2 entries");
  const int rbits = rbits_hint > 0 ? rbits_hint : RBITS_DEFAULT;
  if (rbits < 12 || rbits > RBITS_MAX)
    return tsp::fail(TSP_EINVAL, "tsp_csr_colplan: rows per tile 2^%d outside 2^12..2^14", rbits);
  const int64_t nrb = tsp::ceil_div(m, (int64_t)1 << rbits);
  const int64_t target = tiles_hint > 0 ? tiles_hint : TILES_TARGET;
  int64_t gw = tsp::ceil_div(target, nrb);
  if (gw < 1) gw = 1;
  int cbits = ilog2_ceil(tsp::ceil_div(n, gw));
  if (cbits < 6) cbits = 6;
  if (rbits + cbits > 32) cbits = 32 - rbits;
  const int64_t G = tsp::ceil_div(n, (int64_t)1 << cbits);
  const int64_t T = nrb * G;
  if (T > INT32_MAX / 2) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan: too many tiles");
  const int keybits = ilog2_ceil(T + 1) + cbits;
  if (keybits > 63) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan: key wider than 63 bits");
  const int64_t pmax = nnz + T * (int64_t)E;  // padded entries, at most
  if ((pmax >> EBITS) > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan: too many epochs");
  const int64_t ksz = keybits <= 32 ? 4 : 8;
  size_t tmp = 0;
  hipError_t e = keybits <= 32
                     ? tsp::rsort::radix_sort_pairs(nullptr, tmp, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                                    (const uint64_t*)nullptr, (uint64_t*)nullptr, nnz, 0, keybits)
                     : tsp::rsort::radix_sort_pairs(nullptr, tmp, (const uint64_t*)nullptr, (uint64_t*)nullptr,
                                                    (const uint64_t*)nullptr, (uint64_t*)nullptr, nnz, 0, keybits);
  if (e != hipSuccess) return tsp::check_hip(e, "tsp_csr_colplan: sort size query");
  g[GEOM_RBITS] = rbits;
  g[GEOM_NRB] = nrb;
  g[GEOM_CBITS] = cbits;
  g[GEOM_G] = G;
  g[GEOM_T] = T;
  g[GEOM_KEYBITS] = keybits;
  g[GEOM_PLAN_BYTES] = 2 * align256((T + 1) * 8) + align256((pmax + E) * 8) + align256((pmax + E) * 4) +
                        256 + align256(m * 2);  // + the header (row_ptrs[0] of the built pattern), row exponents
  g[GEOM_BUILD_BYTES] = 2 * align256(nnz * ksz) + 2 * align256(nnz * 8) + align256((int64_t)tmp);
  const int64_t prows = nrb << rbits;  // rows of one group's partial sums
  g[GEOM_SPMV_BYTES] = align256(G * prows * 4) + align256(G * (prows >> 5) * 4) + (XMAX_BLOCKS + 1) * 4;
  g[GEOM_PMAX] = pmax;
  return TSP_OK;
}

template <typename IdxT>
void launch_rowexp(const float* vals, const IdxT* ptr, int64_t m, int64_t nnz, int16_t* rexp, hipStream_t st) {
  if (nnz > 32 * m)
    hipLaunchKernelGGL((colplan_rowexp_kernel<IdxT, 64>), dim3((unsigned)tsp::ceil_div(m * 64, 256)), dim3(256), 0, st,
                       vals, ptr, m, rexp);
  else
    hipLaunchKernelGGL((colplan_rowexp_kernel<IdxT, 16>), dim3((unsigned)tsp::ceil_div(m * 16, 256)), dim3(256), 0, st,
                       vals, ptr, m, rexp);
}

struct PlanView {
  int64_t* toff;
  int64_t* eoff;
  uint64_t* ent;
  uint32_t* pos;
  int16_t* rexp;  // row exponents (one per row of the matrix)
  int64_t* base;  // row_ptrs[0] of the pattern the plan was built from
  int64_t pmax;
};

PlanView plan_view(void* plan, const int64_t* g) {
  uint8_t* p = (uint8_t*)plan;
  const int64_t T = g[GEOM_T];
  PlanView v;
  v.pmax = g[GEOM_PMAX];
  v.toff = (int64_t*)p;
  p += align256((T + 1) * 8);
  v.eoff = (int64_t*)p;
  p += align256((T + 1) * 8);
  v.ent = (uint64_t*)p;
  p += align256((v.pmax + E) * 8);
  v.pos = (uint32_t*)p;
  p += align256((v.pmax + E) * 4);
  v.base = (int64_t*)p;
  v.rexp = (int16_t*)(p + 256);  // after the 256-byte header, one per row
  return v;
}

// The geometry comes back from the caller: everything the kernels index
// with must follow from (m, n, nnz) and the two tiling choices.
int check_geom(const char* who, int64_t m, int64_t n, int64_t nnz, const int64_t* geom) {
  if (!geom) return tsp::fail(TSP_EINVAL, "%s: null geometry", who);
  if (m <= 0 || n <= 0 || nnz < 0) return tsp::fail(TSP_EINVAL, "%s: bad size", who);
  const int64_t rbits = geom[GEOM_RBITS], cbits = geom[GEOM_CBITS];
  if (rbits < 12 || rbits > RBITS_MAX || cbits < 6 || rbits + cbits > 32 ||
      geom[GEOM_NRB] != tsp::ceil_div(m, (int64_t)1 << rbits) ||
      geom[GEOM_G] != tsp::ceil_div(n, (int64_t)1 << cbits) || geom[GEOM_T] != geom[GEOM_NRB] * geom[GEOM_G] ||
      geom[GEOM_KEYBITS] != ilog2_ceil(geom[GEOM_T] + 1) + cbits || geom[GEOM_PMAX] != nnz + geom[GEOM_T] * (int64_t)E)
    return tsp::fail(TSP_EINVAL, "%s: geometry does not belong to a %lld x %lld matrix with %lld entries", who,
                     (long long)m, (long long)n, (long long)nnz);
  return TSP_OK;
}

template <typename IdxT, typename K>
int build_typed(const float* vals, const void* col, const void* ptr, int64_t m, int64_t nnz, const int64_t* g,
                void* plan, void* work, hipStream_t st) {
  const int rbits = (int)g[GEOM_RBITS], cbits = (int)g[GEOM_CBITS];
  const int64_t G = g[GEOM_G], T = g[GEOM_T];
  uint8_t* w = (uint8_t*)work;
  K* kin = (K*)w;
  w += align256(nnz * (int64_t)sizeof(K));
  K* kout = (K*)w;
  w += align256(nnz * (int64_t)sizeof(K));
  uint64_t* pin = (uint64_t*)w;
  w += align256(nnz * 8);
  uint64_t* pout = (uint64_t*)w;
  w += align256(nnz * 8);
  void* tmp = w;
  size_t tmp_bytes = 0;
  hipError_t e = tsp::rsort::radix_sort_pairs(nullptr, tmp_bytes, (const K*)kin, kout, (const uint64_t*)pin, pout, nnz,
                                              0, (int)g[GEOM_KEYBITS], st);
  if (e != hipSuccess) return tsp::check_hip(e, "tsp_csr_colplan_build: sort size query");
  PlanView v = plan_view(plan, g);
  hipLaunchKernelGGL(colplan_fill_kernel, dim3((unsigned)tsp::ceil_div(v.pmax + E, 256)), dim3(256), 0, st, v.ent,
                     v.pos, v.pmax + E);
  int rc = tsp::check_launch("colplan_fill launch");
  if (rc) return rc;
  if (nnz > 0) {
    if (tsp::ceil_div(nnz, KTILE) > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan_build: too many entries");
    hipLaunchKernelGGL((colplan_keys_kernel<IdxT, K>), dim3((unsigned)tsp::ceil_div(nnz, KTILE)), dim3(256), 0, st,
                       (const IdxT*)col, (const IdxT*)ptr, m, nnz, rbits, cbits, G, kin, pin, v.base);
    rc = tsp::check_launch("colplan_keys launch");
    if (rc) return rc;
    e = tsp::rsort::radix_sort_pairs(tmp, tmp_bytes, (const K*)kin, kout, (const uint64_t*)pin, pout, nnz, 0,
                                     (int)g[GEOM_KEYBITS], st);
    if (e != hipSuccess) return tsp::check_hip(e, "tsp_csr_colplan_build: radix sort");
  }
  hipLaunchKernelGGL((colplan_offsets_kernel<K>), dim3((unsigned)tsp::ceil_div(T + 1, 256)), dim3(256), 0, st,
                     kout, nnz, cbits, T, v.toff);
  rc = tsp::check_launch("colplan_offsets launch");
  if (rc) return rc;
  hipLaunchKernelGGL(colplan_epochs_kernel, dim3(1), dim3(1024), 0, st, v.toff, T, v.eoff);
  rc = tsp::check_launch("colplan_epochs launch");
  if (rc) return rc;
  launch_rowexp(vals, (const IdxT*)ptr, m, nnz, v.rexp, st);
  rc = tsp::check_launch("colplan_rowexp launch");
  if (rc || nnz == 0) return rc;
  hipLaunchKernelGGL((colplan_scatter_kernel<K>), dim3((unsigned)tsp::ceil_div(nnz, 256)), dim3(256), 0, st, kout,
                     pout, vals, nnz, rbits, cbits, G, v.toff, v.eoff, T, v.base, v.rexp, v.ent, v.pos);
  return tsp::check_launch("colplan_scatter launch");
}

template <int RBITS>
void launch_spmv(const PlanView& v, const float* x, uint32_t* xpart, int nxpart, const int64_t* g,
                 float* partial, uint32_t* inexact, hipStream_t st) {
  const int64_t T = g[GEOM_T];
  const int xcd_map = (T % 8) == 0 ? 1 : 0;
  hipLaunchKernelGGL((colplan_spmv_fx<RBITS, SPMV_NT>), dim3((unsigned)T), dim3(SPMV_NT), 0, st, v.ent, v.toff, v.eoff,
                     x, xpart, nxpart, (int)g[GEOM_CBITS], g[GEOM_G], g[GEOM_NRB], v.pmax, xcd_map, partial, inexact);
}

}  // namespace

extern "C" int tsp_csr_colplan_geometry(int64_t m, int64_t n, int64_t nnz, int rows_per_block_log2,
                                        int64_t tiles_hint, int64_t* geometry_out) {
  if (!geometry_out) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_geometry: null output");
  if (tiles_hint < 0 || rows_per_block_log2 < 0) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_geometry: negative hint");
  return geometry(m, n, nnz, rows_per_block_log2, tiles_hint, geometry_out);
}

extern "C" int tsp_csr_colplan_build(const void* values, int dtype, const void* col_indices, const void* row_ptrs,
                                     int index_type, int64_t m, int64_t n, int64_t nnz, const int64_t* geometry,
                                     void* plan, void* workspace, void* stream) {
  if (dtype != TSP_F32) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan_build: dtype %d (the plan holds fp32 values)", dtype);
  if (index_type != TSP_I32 && index_type != TSP_I64) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_build: bad index_type");
  int rc = check_geom("tsp_csr_colplan_build", m, n, nnz, geometry);
  if (rc) return rc;
  if (!row_ptrs || !plan || !workspace || (nnz > 0 && (!values || !col_indices)))
    return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_build: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const bool k32 = geometry[GEOM_KEYBITS] <= 32;
  if (index_type == TSP_I64)
    return k32 ? build_typed<int64_t, uint32_t>((const float*)values, col_indices, row_ptrs, m, nnz, geometry, plan, workspace, st)
               : build_typed<int64_t, uint64_t>((const float*)values, col_indices, row_ptrs, m, nnz, geometry, plan, workspace, st);
  return k32 ? build_typed<int32_t, uint32_t>((const float*)values, col_indices, row_ptrs, m, nnz, geometry, plan, workspace, st)
             : build_typed<int32_t, uint64_t>((const float*)values, col_indices, row_ptrs, m, nnz, geometry, plan, workspace, st);
}

extern "C" int tsp_csr_colplan_refresh(const void* values, int dtype, const void* row_ptrs, int index_type, int64_t m,
                                       int64_t n, int64_t nnz, const int64_t* geometry, void* plan, void* stream) {
  if (dtype != TSP_F32) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan_refresh: dtype %d (the plan holds fp32 values)", dtype);
  if (index_type != TSP_I32 && index_type != TSP_I64) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_refresh: bad index_type");
  int rc = check_geom("tsp_csr_colplan_refresh", m, n, nnz, geometry);
  if (rc) return rc;
  if (!row_ptrs || !plan || (nnz > 0 && !values)) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_refresh: null pointer");
  hipStream_t st = (hipStream_t)stream;
  PlanView v = plan_view(plan, geometry);
  if (index_type == TSP_I64)
    launch_rowexp((const float*)values, (const int64_t*)row_ptrs, m, nnz, v.rexp, st);
  else
    launch_rowexp((const float*)values, (const int32_t*)row_ptrs, m, nnz, v.rexp, st);
  rc = tsp::check_launch("colplan_rowexp launch");
  if (rc || nnz == 0) return rc;
  hipLaunchKernelGGL(colplan_refresh_kernel, dim3((unsigned)tsp::ceil_div(v.pmax, 256)), dim3(256), 0, st,
                     (const float*)values, v.pos, v.pmax, v.base, v.eoff, geometry[GEOM_T], geometry[GEOM_G],
                     (int)geometry[GEOM_RBITS], (int)geometry[GEOM_CBITS], v.rexp, v.ent);
  return tsp::check_launch("colplan_refresh launch");
}

extern "C" int tsp_csr_colplan_spmv(const void* plan, int dtype, int64_t m, int64_t n, int64_t nnz,
                                    const int64_t* geometry, const void* values, const void* col_indices,
                                    const void* row_ptrs, int index_type, const void* x, double alpha, const void* y,
                                    double beta, void* out, void* workspace, void* stream) {
  if (dtype != TSP_F32) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan_spmv: dtype %d (the plan holds fp32 values)", dtype);
  if (index_type != TSP_I32 && index_type != TSP_I64) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_spmv: bad index_type");
  int rc = check_geom("tsp_csr_colplan_spmv", m, n, nnz, geometry);
  if (rc) return rc;
  if (!plan || !x || !out || !workspace || !row_ptrs || (nnz > 0 && (!values || !col_indices)))
    return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_spmv: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const float* yy = (y && beta != 0.0) ? (const float*)y : nullptr;
  PlanView v = plan_view((void*)plan, geometry);
  const int64_t G = geometry[GEOM_G], prows = geometry[GEOM_NRB] << geometry[GEOM_RBITS];
  uint8_t* w = (uint8_t*)workspace;
  float* partial = (float*)w;
  w += align256(G * prows * 4);
  uint32_t* inexact = (uint32_t*)w;
  w += align256(G * (prows >> 5) * 4);
  uint32_t* xpart = (uint32_t*)w;  // XMAX_BLOCKS partial maxima, then the maximum
  const int vec4 = ((uintptr_t)x % 16) == 0;
  const int nxpart = (int)std::min<int64_t>(XMAX_BLOCKS, tsp::ceil_div(n, vec4 ? 1024 : 256));
  hipLaunchKernelGGL(colplan_xmax_kernel, dim3((unsigned)nxpart), dim3(256), 0, st, (const float*)x, n, vec4, xpart);
  rc = tsp::check_launch("colplan_xmax launch");
  if (rc) return rc;
  switch (geometry[GEOM_RBITS]) {
    case 12: launch_spmv<12>(v, (const float*)x, xpart, nxpart, geometry, partial, inexact, st); break;
    case 13: launch_spmv<13>(v, (const float*)x, xpart, nxpart, geometry, partial, inexact, st); break;
    default: launch_spmv<14>(v, (const float*)x, xpart, nxpart, geometry, partial, inexact, st); break;
  }
  rc = tsp::check_launch("colplan_spmv launch");
  if (rc) return rc;
  const bool vec = m % 4 == 0 && ((uintptr_t)out % 16) == 0 && ((uintptr_t)yy % 16) == 0;
  const unsigned fgrid = (unsigned)tsp::ceil_div(vec ? m / 4 : m, 256);
  const uint32_t* xm = xpart + XMAX_BLOCKS;
#define TSP_FINISH(IT, V)                                                                                             \
  hipLaunchKernelGGL((colplan_finish_fx<IT, V>), dim3(fgrid), dim3(256), 0, st, partial, inexact, prows, G, v.rexp, xm, \
                     (const float*)values, (const IT*)col_indices, (const IT*)row_ptrs, (const float*)x, m,           \
                     (float)alpha, yy, (float)beta, (float*)out)
  if (index_type == TSP_I64) {
    if (vec) TSP_FINISH(int64_t, true); else TSP_FINISH(int64_t, false);
  } else {
    if (vec) TSP_FINISH(int32_t, true); else TSP_FINISH(int32_t, false);
  }
#undef TSP_FINISH
  return tsp::check_launch("colplan_finish launch");
}
