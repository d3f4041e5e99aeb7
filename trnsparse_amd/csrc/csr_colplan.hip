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
// slice through L1 once, so the x traffic is (m / R) x n x 4 bytes: 16384-
// row tiles (64 KiB of LDS row sums, one 1024-thread workgroup per CU) read
// half what 8192-row tiles (two 512-thread workgroups per CU) read, and
// were measured faster on cfg2 (61.6 us against 66.8 us).
//
// Row sums without atomics. Float add atomics in LDS (ds_add_f32) run at a
// small fraction of the rate of other LDS operations on gfx950 (measured:
// they made this kernel 2.2x slower than plain LDS read-modify-write, with
// or without bank conflicts), so each epoch runs in two phases separated by
// a barrier:
//   phase 1  wavefronts take 64-entry chunks round robin, gather x, and
//            store product and row into LDS at the entry's position in row
//            order (the plan's per-epoch inverse permutation, 16 bits per
//            entry);
//   phase 2  wavefront w owns positions w*E/W .. (w+1)*E/W - 1 of the
//            epoch and lane l of it the 4 consecutive positions from
//            w*E/W + 4l (two 16-byte LDS reads). The lane adds its runs of
//            equal rows in order; a run that ends inside the lane is added
//            to the tile's LDS row sum by a plain read-modify-write. Runs
//            that cross lanes are joined by one segmented scan of the lanes'
//            last runs (key: row), so each row is written by exactly one
//            lane, except the wavefront's first row, whose sum goes to a
//            carry slot that wavefront 0 adds after the epoch's closing
//            barrier, in wavefront order. (The first form of this phase
//            scanned every 64-position chunk across lanes: several times
//            the VALU work, 82 us against 67 us on cfg2.)
// Every sum is taken in a fixed order, so results are deterministic.
// With G > 1 column groups each tile writes its row sums to a partial
// vector and a second kernel adds the G partials per row in group order
// and applies alpha / beta.
//
// Plan buffer (device): toff (T+1 int64, first sorted entry of each tile),
// eoff (T+1 int64, first epoch of each tile), ent (8 bytes per padded entry:
// value bits << 32 | row_in_tile << cbits | column_in_group), pinv (uint16
// per padded entry: the entry's position in the epoch's row order, swizzled
// for phase 2's 16-byte reads), pos (uint32 per padded entry: position k in
// the pattern's entries, for new values on the same pattern, read at
// values[row_ptrs[0] + k]; 0xffffffff for padding), and a 256-byte header
// holding row_ptrs[0] (int64). Inside an epoch, ent and pos are stored in the SpMV
// kernel's lane order (entry_slot below): one 16-byte load gives a lane two
// of its chunks' entries, and pinv holds a lane's 4 positions in 8
// consecutive bytes. The three per-entry arrays hold one more epoch of zeros
// past the last tile's, which the SpMV kernel's prefetch reads when a tile
// has no epoch left to prefetch.
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
constexpr int SPMV_PL = E / SPMV_W / 64;      // phase-2 row-order positions per lane
static_assert(SPMV_K == 4 && SPMV_PL == 4, "a lane's entries and positions are loaded in 16- and 8-byte pieces");

// Where column-order entry li = (j * W + w) * 64 + l of an epoch (chunk j of
// wavefront w, lane l) is stored: wavefront w's entries are one contiguous
// E/W block, in which 16-byte piece q of lane l holds its chunks 2q and
// 2q + 1, so each load of a wavefront reads 1 KiB contiguously.
__host__ __device__ constexpr int entry_slot(int li) {
  return ((li >> 6) % SPMV_W) * (E / SPMV_W) + (((li >> 6) / SPMV_W) >> 1) * 128 + 2 * (li & 63) +
         (((li >> 6) / SPMV_W) & 1);
}

// LDS slot of row-order position s: position pairs P = s/2 are XOR-swizzled
// (P ^ ((P >> 3) & 1)) so that phase 2's 16-byte reads, lane l at pairs
// 2l and 2l + 1, put 8 consecutive lanes on 8 different 16-byte bank groups.
__host__ __device__ constexpr int pos_slot(int s) {
  return ((((s >> 1) ^ ((s >> 4) & 1))) << 1) | (s & 1);
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

__global__ __launch_bounds__(256) void colplan_fill_kernel(uint64_t* __restrict__ ent, uint16_t* __restrict__ pinv,
                                                           uint32_t* __restrict__ pos, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  ent[i] = 0;
  pinv[i] = 0;
  pos[i] = POS_PAD;
}

// Sorted entry i of tile t is column-order entry j % E of epoch eoff[t] + j / E
// (j = i - toff[t]), stored at entry_slot(j % E) of that epoch.
template <typename K>
__global__ __launch_bounds__(256) void colplan_scatter_kernel(const K* __restrict__ keys,
                                                              const uint64_t* __restrict__ payload,
                                                              const float* __restrict__ vals, int64_t nnz, int cbits,
                                                              const int64_t* __restrict__ toff,
                                                              const int64_t* __restrict__ eoff, int64_t T,
                                                              const int64_t* __restrict__ plan_base,
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
  ent[P] = ((uint64_t)__builtin_bit_cast(uint32_t, vals[plan_base[0] + p]) << 32) | (uint64_t)((rl << cbits) | cin);
  pos[P] = p;
}

// One workgroup per epoch: each entry's position in the epoch's (row,
// column order) order, by a stable LSD radix sort in LDS of the E keys
// row << EBITS | li on the row bits (two 8-bit passes; padding entries take
// row 2^rbits and sort last). A pass ranks each key among equal digits: the
// lanes of a wavefront holding the same digit come from 8 ballots, and the
// counts per (round, wavefront, digit) are prefixed in key order, so equal
// rows keep their column order. Column-order entry li = (j * W + w) * 64 + l
// (chunk j of wavefront w, lane l in the SpMV kernel's phase 1) stores
// pos_slot(its position) in uint16 (w * 64 + l) * K + j: a lane loads the
// positions of its K entries with one 16-byte load.
__global__ __launch_bounds__(1024) void colplan_perm_kernel(const uint64_t* __restrict__ ent,
                                                            const int64_t* __restrict__ toff,
                                                            const int64_t* __restrict__ eoff, int64_t T, int rbits,
                                                            int cbits, uint16_t* __restrict__ pinv) {
  constexpr int NR = E / 1024;  // keys per thread (rounds)
  __shared__ uint32_t key[2][E];
  __shared__ uint16_t cnt[NR][16][256];  // per (round, wavefront, digit): count, then start (< E)
  __shared__ uint32_t dbase[256];
  __shared__ uint32_t wtot[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t ep = blockIdx.x;
  if (ep >= eoff[T]) return;  // the grid covers the epoch count's upper bound
  const int64_t t = upper_bound_i64(eoff, T + 1, ep) - 1;
  const int64_t left = (toff[t + 1] - toff[t]) - ((ep - eoff[t]) << EBITS);
  const int count = left < E ? (int)left : E;
  const uint64_t* __restrict__ e = ent + (ep << EBITS);
  for (int i = tid; i < E; i += 1024) {
    const uint32_t row = i < count ? (uint32_t)e[entry_slot(i)] >> cbits : (1u << rbits);
    key[0][i] = (row << EBITS) | (uint32_t)i;
  }
  const uint64_t lt = (1ull << lane) - 1;
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {  // rows < 2^15: bits EBITS .. EBITS + 15
    const uint32_t* src = key[pass];
    uint32_t* dst = key[pass ^ 1];
    const int shift = EBITS + 8 * pass;
    for (int i = tid; i < NR * 16 * 256 / 2; i += 1024) ((uint32_t*)&cnt[0][0][0])[i] = 0;
    __syncthreads();
    uint32_t kv[NR], dg[NR], rk[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      kv[r] = src[r * 1024 + tid];
      dg[r] = (kv[r] >> shift) & 255u;
      uint64_t peers = ~0ull;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const bool bit = (dg[r] >> b) & 1;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
      }
      rk[r] = (uint32_t)__popcll(peers & lt);
      if (rk[r] == 0) cnt[r][w][dg[r]] = (uint16_t)__popcll(peers);
    }
    __syncthreads();
    // digit tid (< 256): starts of its (round, wavefront) groups, then its start in the epoch
    uint32_t tot = 0;
    if (tid < 256)
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t c = cnt[r][v][tid];
          cnt[r][v][tid] = (uint16_t)tot;
          tot += c;
        }
    uint32_t x = tot;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    if (tid < 256 && lane == 63) wtot[w] = x;
    __syncthreads();
    if (tid < 256) {
      uint32_t before = 0;
      for (int i = 0; i < w; ++i) before += wtot[i];
      dbase[tid] = before + x - tot;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NR; ++r) dst[dbase[dg[r]] + cnt[r][w][dg[r]] + rk[r]] = kv[r];
    __syncthreads();
  }
  uint16_t* __restrict__ out = pinv + (ep << EBITS);
  for (int s = tid; s < E; s += 1024) {
    const int i = (int)(key[0][s] & (E - 1));
    const int c = i >> 6, j = c / SPMV_W, w2 = c % SPMV_W, l = i & 63;
    out[(w2 * 64 + l) * SPMV_K + j] = (uint16_t)pos_slot(s);
  }
}

__global__ __launch_bounds__(256) void colplan_refresh_kernel(const float* __restrict__ vals,
                                                              const uint32_t* __restrict__ pos, int64_t n,
                                                              const int64_t* __restrict__ plan_base,
                                                              uint64_t* __restrict__ ent) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t p = pos[i];
  const uint32_t bits = p == POS_PAD ? 0u : __builtin_bit_cast(uint32_t, vals[plan_base[0] + p]);
  ent[i] = ((uint64_t)bits << 32) | (ent[i] & 0xffffffffull);
}

// ----------------------------------------------------------------- SpMV

// One step of a segmented inclusive scan with DPP: add the value of the
// lane the DPP control names when it holds the same row (rows ascend
// across the lanes, so equal rows mean every lane between is in the run).
template <int CTRL, int ROW_MASK>
__device__ inline float seg_step(float s, uint32_t r) {
  const uint32_t ro = (uint32_t)__builtin_amdgcn_update_dpp((int)0xffffffffu, (int)r, CTRL, ROW_MASK, 0xf, false);
  const float so = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), CTRL, ROW_MASK,
                                                                         0xf, false));
  return ro == r ? s + so : s;
}

// Inclusive sums of runs of equal r over the 64 lanes, without LDS: shifts
// by 1, 2, 4, 8 inside each 16-lane row, then lane 15 of each row into the
// next row and lane 31 into the upper half (row_bcast:15 / :31).
__device__ inline float seg_scan(float s, uint32_t r) {
  s = seg_step<0x111, 0xf>(s, r);  // row_shr:1
  s = seg_step<0x112, 0xf>(s, r);  // row_shr:2
  s = seg_step<0x114, 0xf>(s, r);  // row_shr:4
  s = seg_step<0x118, 0xf>(s, r);  // row_shr:8
  s = seg_step<0x142, 0xa>(s, r);  // row_bcast:15 -> rows 1 and 3
  s = seg_step<0x143, 0xc>(s, r);  // row_bcast:31 -> rows 2 and 3
  return s;
}

template <int RBITS, int NT>
__global__ __launch_bounds__(NT) void colplan_spmv_f32(const uint64_t* __restrict__ ent,
                                                       const uint16_t* __restrict__ pinv,
                                                       const int64_t* __restrict__ toff,
                                                       const int64_t* __restrict__ eoff, const float* __restrict__ x,
                                                       int64_t m, int cbits, int64_t G, int64_t nrb, int64_t pmax,
                                                       int xcd_map,
                                                       float alpha, const float* __restrict__ y, float beta,
                                                       float* __restrict__ out, float* __restrict__ partial) {
  constexpr int R = 1 << RBITS;
  constexpr int W = NT / 64;
  constexpr int K = E / 64 / W;  // chunks per wavefront in phase 1
  constexpr int SPAN = E / W;    // phase-2 positions per wavefront
  constexpr int PL = SPAN / 64;  // phase-2 positions per lane
  static_assert(W == SPMV_W && K == SPMV_K && PL == SPMV_PL, "the plan's layout is made for this workgroup size");
  constexpr uint32_t NONE = 0xffffffffu;
  typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
  __shared__ float acc[R + 1];                          // acc[R]: the padding positions' row
  __shared__ __attribute__((aligned(16))) u32x2 slot[E];  // (product bits, row) at pos_slot(position)
  __shared__ uint32_t crow[W];
  __shared__ float cval[W];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t T = nrb * G;
  // q runs over tiles group-major; with xcd_map, XCD k (= blockIdx % 8)
  // takes the k-th eighth of that order, so an XCD works on one column
  // group (or a run of consecutive groups) and keeps its x slice in L2.
  const int64_t q = xcd_map ? (int64_t)(blockIdx.x & 7) * (T >> 3) + (blockIdx.x >> 3) : (int64_t)blockIdx.x;
  const int64_t g = q / nrb, rb = q - g * nrb;
  const int64_t t = rb * G + g;

  for (int i = tid; i <= R; i += NT) acc[i] = 0.f;

  const int64_t cnt_t = toff[t + 1] - toff[t];
  const int64_t ep0 = eoff[t], nep = eoff[t + 1] - ep0;
  const float* __restrict__ xg = x + (g << cbits);
  const uint32_t cmask = (1u << cbits) - 1u;

  // Software pipeline over epochs, with three register sets for the
  // entries and positions and two for the gathered x values. In epoch k a
  // wavefront issues the x gathers of epoch k + 1, multiplies epoch k's
  // entries by its x values (gathered one epoch earlier), and refills
  // epoch k's entry set with epoch k + 3. Vector memory loads complete in
  // order, so waiting for epoch k's x covers the stream of epoch k + 1
  // (issued two epochs earlier) but never the newer loads: the stream gets
  // two epochs of lead and the gathers one.
  uint64_t evA[K], evB[K], evC[K];
  uint32_t pwA[K / 2], pwB[K / 2], pwC[K / 2];
  float xa[K], xb[K];
  // k past the tile's last epoch: the plan's zero epoch after all tiles
  // A chunk pair (or a lane's positions) holding no entry of the epoch (the
  // padding of a tile's last epoch, every chunk past the tile's end) reads
  // the plan's zero epoch instead: the load stays unconditional, and the
  // padding is never fetched from HBM (about 6 % of the plan on cfg2).
  auto load_epoch = [&](uint64_t (&ev)[K], uint32_t (&pw)[K / 2], int64_t k) {
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
    const int64_t psrc = (int64_t)(w * 64) < left ? eb : pmax;
    const u32x2 pv = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(pinv + psrc) + w * 64 + lane);
    pw[0] = pv.x;
    pw[1] = pv.y;
  };
  // gathers of an epoch's x (past the tile's end the zero epoch's column 0,
  // which is inside x)
  auto gather = [&](float (&xv)[K], const uint64_t (&ev)[K]) {
#pragma unroll
    for (int j = 0; j < K; ++j) xv[j] = xg[(uint32_t)ev[j] & cmask];
  };
  if (nep > 0) {
    load_epoch(evA, pwA, 0);
    load_epoch(evB, pwB, 1);
    load_epoch(evC, pwC, 2);
  }
  __syncthreads();

  auto epoch = [&](uint64_t (&ev)[K], uint32_t (&pw)[K / 2], const float (&xv)[K], const uint64_t (&evn)[K],
                   float (&xvn)[K], int64_t k) {
    const int64_t left = cnt_t - (k << EBITS);
    const int cnt = left < E ? (int)left : E;
    gather(xvn, evn);
    // ---- phase 1: products and rows in column order
#pragma unroll
    for (int j = 0; j < K; ++j) {
      // column-order index (j * W + w) * 64 + lane < cnt, with the chunk
      // offset moved to the (uniform) right-hand side
      const bool real = w * 64 + lane < cnt - j * W * 64;
      const float pr = __builtin_bit_cast(float, (uint32_t)(ev[j] >> 32)) * xv[j];
      if (real)  // the padding's positions (cnt .. E - 1 in row order) are never read
        slot[(pw[j >> 1] >> (16 * (j & 1))) & 0xffffu] = u32x2{__builtin_bit_cast(uint32_t, pr), (uint32_t)ev[j] >> cbits};
    }
    // unconditional (past the tile's end it reads the zero epoch), so no
    // path without these loads makes the compiler wait for them early
    load_epoch(ev, pw, k + 3);
    __syncthreads();
    // ---- phase 2: lane l adds positions pb .. pb + PL - 1 in row order
    const int pb = w * SPAN + PL * lane;
    uint32_t rr[PL];
    float sm[PL];
    const u32x4* __restrict__ s2 = reinterpret_cast<const u32x4*>(slot);
#pragma unroll
    for (int h = 0; h < PL / 2; ++h) {
      const int P = (pb >> 1) + h;
      const u32x4 v = s2[P ^ ((P >> 3) & 1)];  // pos_slot of positions 2P, 2P + 1
      // (component by component: __builtin_bit_cast of a vector component
      // reads component 0 with this compiler, so __uint_as_float)
      // padding sorts after every row: positions cnt .. E - 1 (not written in
      // phase 1) are the padding row R with nothing to add
      const bool p0 = pb + 2 * h < cnt, p1 = pb + 2 * h + 1 < cnt;
      sm[2 * h] = p0 ? __uint_as_float(v.x) : 0.f;
      rr[2 * h] = p0 ? v.y : (uint32_t)R;
      sm[2 * h + 1] = p1 ? __uint_as_float(v.z) : 0.f;
      rr[2 * h + 1] = p1 ? v.w : (uint32_t)R;
    }
    float old[PL];  // the rows' sums before this epoch (only this lane writes a row it ends)
#pragma unroll
    for (int i = 0; i < PL; ++i) old[i] = acc[rr[i]];
#pragma unroll
    for (int i = 1; i < PL; ++i) sm[i] = rr[i] == rr[i - 1] ? sm[i - 1] + sm[i] : sm[i];
    // sm[i]: sum of the lane's run through position i
    const uint32_t r0 = rr[0], rl = rr[PL - 1];
    // Tl: the lane's last run plus the same row's runs in the lanes before
    // (a lane whose positions hold one row passes its whole sum on)
    const float Tl = seg_scan(sm[PL - 1], rl);
    const uint32_t next_r0 = (uint32_t)__builtin_amdgcn_update_dpp((int)NONE, (int)r0, 0x130, 0xf, 0xf, false);  // wave_shl:1
    const uint32_t prev_rl = (uint32_t)__builtin_amdgcn_update_dpp((int)NONE, (int)rl, 0x138, 0xf, 0xf, false);  // wave_shr:1
    const float prev_T =
        __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, Tl), 0x138, 0xf, 0xf, false));
    const float inc = r0 == prev_rl ? prev_T : 0.f;  // what flows into the lane's first run
    const uint32_t first = __builtin_amdgcn_readfirstlane(r0);
    // the wavefront's first row may continue the previous wavefront's last
    // one: its sum goes to the carry slot (w > 0)
    const bool to_carry = w > 0;
    bool cf = false;
    float cv = 0.f;
#pragma unroll
    for (int i = 0; i < PL - 1; ++i) {
      if (rr[i] != rr[i + 1]) {  // a run ends inside the lane
        const float v = sm[i] + (rr[i] == r0 ? inc : 0.f);
        if (to_carry && rr[i] == first) {
          cf = true;
          cv = v;
        } else {
          acc[rr[i]] = old[i] + v;
        }
      }
    }
    if (next_r0 != rl) {  // the lane's last run ends here (lane 63: always)
      if (to_carry && rl == first) {
        cf = true;
        cv = Tl;
      } else {
        acc[rl] = old[PL - 1] + Tl;
      }
    }
    const uint64_t cm = __ballot(cf);  // at most one lane: the lane that ends the first row
    // read that lane with the whole wavefront active: inside the lane-0 branch
    // the compiler may compute cv for lane 0 only (a readlane of an inactive
    // lane returns a stale register)
    const float cvl = __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv), cm ? (int)__builtin_ctzll(cm) : 0));
    if (lane == 0) {
      crow[w] = cm ? first : NONE;
      cval[w] = cm ? cvl : 0.f;
    }
    __syncthreads();
    if (w == 0) {  // the carries, in wavefront order: rows ascend with w
      const uint32_t cr = lane < W ? crow[lane] : NONE;
      const float cs = seg_scan(lane < W ? cval[lane] : 0.f, cr);
      const uint32_t crn = (uint32_t)__builtin_amdgcn_update_dpp((int)NONE, (int)cr, 0x130, 0xf, 0xf, false);
      if (cr != NONE && (lane == 63 || crn != cr)) acc[cr] += cs;
    }
  };

  // Six epochs per trip (the period of three entry sets and two x sets),
  // the rest after the loop: with later epochs of a trip conditional, the
  // compiler's wait analysis assumes the paths that skip them and waits for
  // the newest stream loads.
  if (nep > 0) gather(xa, evA);
  int64_t k = 0;
  for (; k + 5 < nep; k += 6) {
    epoch(evA, pwA, xa, evB, xb, k);
    epoch(evB, pwB, xb, evC, xa, k + 1);
    epoch(evC, pwC, xa, evA, xb, k + 2);
    epoch(evA, pwA, xb, evB, xa, k + 3);
    epoch(evB, pwB, xa, evC, xb, k + 4);
    epoch(evC, pwC, xb, evA, xa, k + 5);
  }
  if (k < nep) epoch(evA, pwA, xa, evB, xb, k);
  if (k + 1 < nep) epoch(evB, pwB, xb, evC, xa, k + 1);
  if (k + 2 < nep) epoch(evC, pwC, xa, evA, xb, k + 2);
  if (k + 3 < nep) epoch(evA, pwA, xb, evB, xa, k + 3);
  if (k + 4 < nep) epoch(evB, pwB, xa, evC, xb, k + 4);
  __syncthreads();

  const int64_t r0 = rb << RBITS;
  if (G == 1) {
    for (int i = tid; i < R; i += NT) {
      const int64_t r = r0 + i;
      if (r < m) {
        float res = alpha * acc[i];
        if (y) res = res + beta * y[r];
        out[r] = res;
      }
    }
  } else {
    float* __restrict__ pg = partial + g * m;
    for (int i = tid; i < R; i += NT) {
      const int64_t r = r0 + i;
      if (r < m) pg[r] = acc[i];
    }
  }
}

// out[r] = alpha * (partial[0][r] + ... + partial[G-1][r]) (+ beta * y[r]),
// the groups added in increasing order.
__global__ __launch_bounds__(256) void colplan_finish_f32(const float* __restrict__ partial, int64_t m, int64_t G,
                                                          float alpha, const float* __restrict__ y, float beta,
                                                          float* __restrict__ out) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= m) return;
  float s = partial[r];
  for (int64_t g = 1; g < G; ++g) s += partial[g * m + r];
  float res = alpha * s;
  if (y) res = res + beta * y[r];
  out[r] = res;
}

// The same for m a multiple of 4 with 16-byte aligned y and out: four rows
// per thread, 16-byte loads and stores (the same additions in the same order).
__global__ __launch_bounds__(256) void colplan_finish4_f32(const float* __restrict__ partial, int64_t m, int64_t G,
                                                           float alpha, const float* __restrict__ y, float beta,
                                                           float* __restrict__ out) {
  const int64_t r = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (r >= m) return;
  f32x4 s = *reinterpret_cast<const f32x4*>(partial + r);
  for (int64_t g = 1; g < G; ++g) s += *reinterpret_cast<const f32x4*>(partial + g * m + r);
  f32x4 res = alpha * s;
  if (y) res = res + beta * *reinterpret_cast<const f32x4*>(y + r);
  *reinterpret_cast<f32x4*>(out + r) = res;
}

// ------------------------------------------------------------- geometry

constexpr int RBITS_MAX = 14;          // 16384 rows: 64 KiB of fp32 row sums per workgroup
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
  g[GEOM_PLAN_BYTES] = 2 * align256((T + 1) * 8) + align256((pmax + E) * 8) + align256((pmax + E) * 2) +
                        align256((pmax + E) * 4) + 256;  // + the header (row_ptrs[0] of the built pattern)
  g[GEOM_BUILD_BYTES] = 2 * align256(nnz * ksz) + 2 * align256(nnz * 8) + align256((int64_t)tmp);
  g[GEOM_SPMV_BYTES] = G > 1 ? G * m * 4 : 0;
  g[GEOM_PMAX] = pmax;
  return TSP_OK;
}

struct PlanView {
  int64_t* toff;
  int64_t* eoff;
  uint64_t* ent;
  uint16_t* pinv;
  uint32_t* pos;
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
  v.pinv = (uint16_t*)p;
  p += align256((v.pmax + E) * 2);
  v.pos = (uint32_t*)p;
  p += align256((v.pmax + E) * 4);
  v.base = (int64_t*)p;
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
                     v.pinv, v.pos, v.pmax + E);
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
  if (rc || nnz == 0) return rc;
  hipLaunchKernelGGL((colplan_scatter_kernel<K>), dim3((unsigned)tsp::ceil_div(nnz, 256)), dim3(256), 0, st, kout,
                     pout, vals, nnz, cbits, v.toff, v.eoff, T, v.base, v.ent, v.pos);
  rc = tsp::check_launch("colplan_scatter launch");
  if (rc) return rc;
  // one workgroup per epoch; the grid covers the upper bound pmax / E
  hipLaunchKernelGGL(colplan_perm_kernel, dim3((unsigned)(v.pmax >> EBITS)), dim3(1024), 0, st, v.ent, v.toff,
                     v.eoff, T, rbits, cbits, v.pinv);
  return tsp::check_launch("colplan_perm launch");
}

template <int RBITS>
void launch_spmv(const PlanView& v, const float* x, int64_t m, const int64_t* g, float alpha, const float* y,
                 float beta, float* out, float* partial, hipStream_t st) {
  const int64_t T = g[GEOM_T];
  const int xcd_map = (T % 8) == 0 ? 1 : 0;
  hipLaunchKernelGGL((colplan_spmv_f32<RBITS, SPMV_NT>), dim3((unsigned)T), dim3(SPMV_NT), 0, st, v.ent, v.pinv, v.toff,
                     v.eoff, x, m, (int)g[GEOM_CBITS], g[GEOM_G], g[GEOM_NRB], v.pmax, xcd_map, alpha, y, beta, out,
                     partial);
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

extern "C" int tsp_csr_colplan_refresh(const void* values, int dtype, int64_t m, int64_t n, int64_t nnz,
                                       const int64_t* geometry, void* plan, void* stream) {
  if (dtype != TSP_F32) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan_refresh: dtype %d (the plan holds fp32 values)", dtype);
  int rc = check_geom("tsp_csr_colplan_refresh", m, n, nnz, geometry);
  if (rc) return rc;
  if (nnz == 0) return TSP_OK;
  if (!values || !plan) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_refresh: null pointer");
  PlanView v = plan_view(plan, geometry);
  hipLaunchKernelGGL(colplan_refresh_kernel, dim3((unsigned)tsp::ceil_div(v.pmax, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const float*)values, v.pos, v.pmax, v.base, v.ent);
  return tsp::check_launch("colplan_refresh launch");
}

extern "C" int tsp_csr_colplan_spmv(const void* plan, int dtype, int64_t m, int64_t n, int64_t nnz,
                                    const int64_t* geometry, const void* x, double alpha, const void* y, double beta,
                                    void* out, void* workspace, void* stream) {
  if (dtype != TSP_F32) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_colplan_spmv: dtype %d (the plan holds fp32 values)", dtype);
  int rc = check_geom("tsp_csr_colplan_spmv", m, n, nnz, geometry);
  if (rc) return rc;
  if (!plan || !x || !out) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_spmv: null pointer");
  const int64_t G = geometry[GEOM_G];
  if (G > 1 && !workspace) return tsp::fail(TSP_EINVAL, "tsp_csr_colplan_spmv: null workspace (%lld column groups)", (long long)G);
  hipStream_t st = (hipStream_t)stream;
  const float* yy = (y && beta != 0.0) ? (const float*)y : nullptr;
  PlanView v = plan_view((void*)plan, geometry);
  switch (geometry[GEOM_RBITS]) {
    case 12: launch_spmv<12>(v, (const float*)x, m, geometry, (float)alpha, yy, (float)beta, (float*)out, (float*)workspace, st); break;
    case 13: launch_spmv<13>(v, (const float*)x, m, geometry, (float)alpha, yy, (float)beta, (float*)out, (float*)workspace, st); break;
    default: launch_spmv<14>(v, (const float*)x, m, geometry, (float)alpha, yy, (float)beta, (float*)out, (float*)workspace, st); break;
  }
  rc = tsp::check_launch("colplan_spmv launch");
  if (rc || G == 1) return rc;
  const bool vec4 = m % 4 == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)yy & 15) == 0 &&
                    ((uintptr_t)workspace & 15) == 0;
  if (vec4)
    hipLaunchKernelGGL(colplan_finish4_f32, dim3((unsigned)tsp::ceil_div(m / 4, 256)), dim3(256), 0, st,
                       (const float*)workspace, m, G, (float)alpha, yy, (float)beta, (float*)out);
  else
    hipLaunchKernelGGL(colplan_finish_f32, dim3((unsigned)tsp::ceil_div(m, 256)), dim3(256), 0, st,
                       (const float*)workspace, m, G, (float)alpha, yy, (float)beta, (float*)out);
  return tsp::check_launch("colplan_finish launch");
}
