// Device-wide prefix sums and a stable LSD radix sort of (key, value) pairs,
// hand-written for gfx950 (wave64). Used by the format constructors (COO ->
// CSR, the CSR transpose, duplicate summation) and the SpMV column-plan
// build.
//
// Scan: blocks of 256 threads x 16 consecutive elements; a three-phase
// reduce / scan-of-block-sums / apply, the block sums scanned recursively.
//
// Sort: 8-bit digits over bits [begin_bit, end_bit), tiles of 256 threads x
// 16 keys (4096; in the scatter, round i of lane l in wavefront w is key
// 1024 w + 64 i + l).
// Per pass:
//   rs_count    per-tile digit counts into a tile-major table
//               counts[tile * 256 + d] (one coalesced row per tile);
//   offsets     the table turned in place into the output start of digit
//               d's keys from each tile (all of digits < d first, then the
//               tiles before it), by a scan along the tiles of each digit
//               (column): chunk sums of 32 or more tiles, one workgroup
//               (4 x 256 threads) scanning the chunk sums of every digit
//               and adding the digit bases, then each chunk's tiles in
//               order;
//   rs_scatter  each key's rank among equal digits of its tile: each
//               wavefront owns a contiguous quarter of the tile and keeps a
//               running count per digit in LDS across its rounds; lanes of a
//               round with the same digit are found by 8 ballots; the tile
//               is reordered by digit in LDS and written as runs, so
//               consecutive lanes write consecutive addresses.
// Equal digits keep their input order within and across tiles, so every
// pass and the sort are stable. Passes alternate between the output and a
// temporary buffer so the last one lands in the output.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace tsp {
namespace rsort {

constexpr int NT = 256;             // threads per block
constexpr int NW = NT / 64;         // wavefronts per block
constexpr int SCAN_IPT = 16;        // scan elements per thread
constexpr int SCAN_TILE = NT * SCAN_IPT;
// sort keys per thread: 16 (4096-key tiles)
template <typename K, typename V>
constexpr int sort_ipt() {
  return 16;
}
constexpr int RADIX = 256;
static_assert(NT == RADIX, "the sort kernels give each thread one digit's table entry");

inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// ------------------------------------------------------------------ scan

// Exclusive scan of one value per thread over the 256 threads of a block;
// `total` receives the block's sum. Every thread must call it.
template <typename T>
__device__ inline T block_exclusive_scan(T v, T& total) {
  __shared__ T wsum[NW];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  T x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const T y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  T before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const T s = wsum[i];
    if (i < w) before += s;
    all += s;
  }
  __syncthreads();  // wsum may be reused by a later call
  total = all;
  return before + x - v;
}

template <typename T>
__global__ __launch_bounds__(NT) void scan_reduce_kernel(const T* __restrict__ in, int64_t n, T* __restrict__ sums) {
  const int64_t base = (int64_t)blockIdx.x * SCAN_TILE + (int64_t)threadIdx.x * SCAN_IPT;
  T s = 0;
#pragma unroll
  for (int i = 0; i < SCAN_IPT; ++i)
    if (base + i < n) s += in[base + i];
  T total;
  block_exclusive_scan(s, total);
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// out[i] = init + offs[block] + (sum of in[block start .. i), or .. i] when inclusive).
// in == out is allowed: each thread reads its elements before writing them.
template <typename T>
__global__ __launch_bounds__(NT) void scan_apply_kernel(const T* in, T* out, int64_t n, const T* __restrict__ offs,
                                                        int inclusive, T init) {
  const int64_t base = (int64_t)blockIdx.x * SCAN_TILE + (int64_t)threadIdx.x * SCAN_IPT;
  T v[SCAN_IPT];
  T s = 0;
#pragma unroll
  for (int i = 0; i < SCAN_IPT; ++i) {
    v[i] = base + i < n ? in[base + i] : T(0);
    s += v[i];
  }
  T total;
  T run = block_exclusive_scan(s, total) + init + (offs ? offs[blockIdx.x] : T(0));
#pragma unroll
  for (int i = 0; i < SCAN_IPT; ++i) {
    if (base + i < n) out[base + i] = inclusive ? run + v[i] : run;
    run += v[i];
  }
}

// Temporary bytes for scan() over n elements: the block sums of every level.
inline size_t scan_tmp_bytes(int64_t n, size_t elem) {
  size_t b = 0;
  int64_t nb = (n + SCAN_TILE - 1) / SCAN_TILE;
  while (nb > 1) {
    b += 2 * align256((size_t)nb * elem);
    nb = (nb + SCAN_TILE - 1) / SCAN_TILE;
  }
  return b + 256;
}

// Prefix sums of in[0, n) into out (in place allowed), plus init.
template <typename T>
hipError_t scan(void* tmp, const T* in, T* out, int64_t n, bool inclusive, T init, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const int64_t nb = (n + SCAN_TILE - 1) / SCAN_TILE;
  if (nb > INT32_MAX) return hipErrorInvalidValue;
  if (nb == 1) {
    hipLaunchKernelGGL(scan_apply_kernel<T>, dim3(1), dim3(NT), 0, st, in, out, n, (const T*)nullptr,
                       inclusive ? 1 : 0, init);
    return hipGetLastError();
  }
  T* sums = (T*)tmp;
  T* offs = (T*)((char*)tmp + align256((size_t)nb * sizeof(T)));
  void* next = (char*)tmp + 2 * align256((size_t)nb * sizeof(T));
  hipLaunchKernelGGL(scan_reduce_kernel<T>, dim3((unsigned)nb), dim3(NT), 0, st, in, n, sums);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = scan(next, (const T*)sums, offs, nb, false, T(0), st);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(scan_apply_kernel<T>, dim3((unsigned)nb), dim3(NT), 0, st, in, out, n, (const T*)offs,
                     inclusive ? 1 : 0, init);
  return hipGetLastError();
}

// rocPRIM-style entry points: tmp == nullptr stores the temporary size.
template <typename T>
hipError_t inclusive_scan(void* tmp, size_t& tmp_bytes, const T* in, T* out, int64_t n, hipStream_t st = 0) {
  if (!tmp) {
    tmp_bytes = scan_tmp_bytes(n, sizeof(T));
    return hipSuccess;
  }
  return scan(tmp, in, out, n, true, T(0), st);
}
template <typename T>
hipError_t exclusive_scan(void* tmp, size_t& tmp_bytes, const T* in, T* out, T init, int64_t n,
                          hipStream_t st = 0) {
  if (!tmp) {
    tmp_bytes = scan_tmp_bytes(n, sizeof(T));
    return hipSuccess;
  }
  return scan(tmp, in, out, n, false, init, st);
}

// ------------------------------------------------------------------ sort

template <typename K>
__device__ inline uint32_t digit_of(K k, int shift, uint32_t mask) {
  return (uint32_t)(k >> shift) & mask;
}

template <typename K, int IPT>
__global__ __launch_bounds__(NT) void rs_count_kernel(const K* __restrict__ keys, int64_t n, int shift,
                                                      uint32_t mask, uint32_t* __restrict__ counts) {
  __shared__ uint32_t h[NW][RADIX];
  const int tid = threadIdx.x, w = tid >> 6;
  for (int i = tid; i < NW * RADIX; i += NT) (&h[0][0])[i] = 0;
  __syncthreads();
  constexpr int TILE = NT * IPT;
  const int64_t base = (int64_t)blockIdx.x * TILE;
  if (base + TILE <= n && ((uintptr_t)keys & 15) == 0) {
    // full tile: counting ignores order, so each thread takes IPT consecutive keys in 16-byte loads
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    constexpr int PER = 16 / (int)sizeof(K), NV = IPT / PER;
    const u32x4* p = (const u32x4*)(keys + base + (int64_t)tid * IPT);
    u32x4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = p[j];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const K* kk = (const K*)&v[j];
#pragma unroll
      for (int e = 0; e < PER; ++e) atomicAdd(&h[w][digit_of(kk[e], shift, mask)], 1u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      const int64_t idx = base + i * NT + tid;
      if (idx < n) atomicAdd(&h[w][digit_of(keys[idx], shift, mask)], 1u);
    }
  }
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) s += h[i][tid];
  counts[(int64_t)blockIdx.x * RADIX + tid] = s;
}

// Column scan of the tile-major count table (thread d = digit d), each
// column walk 8 loads deep:
// csum[c][d] = sum of the counts of chunk c's tiles (ch tiles per chunk).
template <typename C>
__global__ __launch_bounds__(NT) void rs_chunk_sum_kernel(const C* __restrict__ counts, int64_t ntiles, int64_t ch,
                                                          C* __restrict__ csum) {
  const int64_t t0 = (int64_t)blockIdx.x * ch;
  const int64_t t1 = t0 + ch < ntiles ? t0 + ch : ntiles;
  const C* col = counts + threadIdx.x;
  C s = 0;
  int64_t t = t0;
  for (; t + 8 <= t1; t += 8) {
    C v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = col[(t + j) * RADIX];
#pragma unroll
    for (int j = 0; j < 8; ++j) s += v[j];
  }
  for (; t < t1; ++t) s += col[t * RADIX];
  csum[(int64_t)blockIdx.x * RADIX + threadIdx.x] = s;
}
// Exclusive scan along a column of rows [r0, r1) of a RADIX-wide table, in
// place, starting from run, 16 loads in flight; returns run plus the total.
template <typename C>
__device__ inline C rs_column_scan(C* __restrict__ col, int64_t r0, int64_t r1, C run) {
  int64_t t = r0;
  for (; t + 16 <= r1; t += 16) {
    C v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = col[(t + j) * RADIX];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      col[(t + j) * RADIX] = run;
      run += v[j];
    }
  }
  for (; t < r1; ++t) {
    const C v = col[t * RADIX];
    col[t * RADIX] = run;
    run += v;
  }
  return run;
}
// One workgroup of 4 x 256 threads, thread (part p, digit d) owning a
// quarter of the chunk rows: csum[c][d] <- (sum over csum of the rows of d
// before c) + dbase[d], where dbase[d] = all keys of digits < d.
constexpr int CB_PARTS = 4;
template <typename C>
__global__ __launch_bounds__(NT * CB_PARTS) void rs_chunk_base_kernel(C* __restrict__ csum, int64_t nchunks) {
  __shared__ C part[CB_PARTS][RADIX];
  __shared__ C dbase[RADIX];
  const int d = threadIdx.x % RADIX, p = threadIdx.x / RADIX;
  const int64_t per = (nchunks + CB_PARTS - 1) / CB_PARTS;
  const int64_t r0 = p * per < nchunks ? p * per : nchunks;
  const int64_t r1 = r0 + per < nchunks ? r0 + per : nchunks;
  C* col = csum + d;
  C s = 0;
  int64_t t = r0;
  for (; t + 16 <= r1; t += 16) {
    C v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = col[(t + j) * RADIX];
#pragma unroll
    for (int j = 0; j < 16; ++j) s += v[j];
  }
  for (; t < r1; ++t) s += col[t * RADIX];
  part[p][d] = s;
  __syncthreads();
  if (threadIdx.x < 64) {  // one wavefront: exclusive scan of the 256 digit totals, 4 per lane
    const int l = threadIdx.x;
    C tot[4], acc = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tot[e] = 0;
#pragma unroll
      for (int q = 0; q < CB_PARTS; ++q) tot[e] += part[q][4 * l + e];
      acc += tot[e];
    }
    C x = acc;  // inclusive scan of the lane sums
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const C y = __shfl_up(x, o, 64);
      if (l >= o) x += y;
    }
    C run = x - acc;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dbase[4 * l + e] = run;
      run += tot[e];
    }
  }
  __syncthreads();
  C run = dbase[d];
  for (int q = 0; q < p; ++q) run += part[q][d];
  rs_column_scan<C>(col, r0, r1, run);
}
// counts[t][d] <- csum[c][d] + (counts of the chunk's tiles before t), in place.
template <typename C>
__global__ __launch_bounds__(NT) void rs_chunk_apply_kernel(C* __restrict__ counts, int64_t ntiles, int64_t ch,
                                                            const C* __restrict__ csum) {
  const int64_t t0 = (int64_t)blockIdx.x * ch;
  const int64_t t1 = t0 + ch < ntiles ? t0 + ch : ntiles;
  rs_column_scan<C>(counts + threadIdx.x, t0, t1, csum[(int64_t)blockIdx.x * RADIX + threadIdx.x]);
}

// Where a pass stores the value of output position i: a plain array, or in
// the last pass a caller's writer (e.g. fields to separate arrays).
template <typename V>
struct VStore {
  V* p;
  __device__ void operator()(int64_t i, const V& v) const { p[i] = v; }
};

template <typename K, typename V, int IPT, typename VW>
__global__ __launch_bounds__(NT) void rs_scatter_kernel(const K* __restrict__ kin, const V* __restrict__ vin,
                                                        K* __restrict__ kout, VW vout, int64_t n, int shift,
                                                        uint32_t mask, const uint32_t* __restrict__ offs) {
  constexpr int TILE = NT * IPT;
  constexpr int Q = TILE / NW;               // keys per wavefront, contiguous
  __shared__ uint16_t hw[NW][RADIX];         // per wavefront: running count of each digit, then its start
  __shared__ uint32_t gbase[RADIX];          // output start of digit d's keys from this tile
  __shared__ uint32_t lbase[RADIX];          // start of digit d in the tile reordered by digit
  __shared__ K sk[TILE];
  __shared__ V sv[TILE];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < NW * RADIX / 2; i += NT) ((uint32_t*)&hw[0][0])[i] = 0;
  gbase[tid] = offs[(int64_t)blockIdx.x * RADIX + tid];
  __syncthreads();
  const int64_t wbase = (int64_t)blockIdx.x * TILE + (int64_t)w * Q;  // round i, lane l: key wbase + 64 i + l
  const uint64_t lt = (1ull << lane) - 1;
  K k[IPT];
  V val[IPT];
  uint32_t dg[IPT], rk[IPT];
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int64_t idx = wbase + 64 * i + lane;
    if (idx < n) {
      k[i] = kin[idx];
      val[i] = vin[idx];
    } else {
      k[i] = K(0);
    }
  }
  // rank of each key among the equal digits before it in the wavefront's
  // keys: the wavefront's running count of the digit (LDS, read by every
  // lane of the group before its leader adds the group) plus the rank among
  // this round's lanes with the same digit (8 ballots)
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const bool valid = wbase + 64 * i + lane < n;
    dg[i] = digit_of(k[i], shift, mask);
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (dg[i] >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint32_t below = (uint32_t)__popcll(peers & lt);
    const uint32_t before = hw[w][dg[i]];
    rk[i] = before + below;
    if (valid && below == 0) hw[w][dg[i]] = (uint16_t)(before + __popcll(peers));
  }
  __syncthreads();
  // digit tid: starts of its wavefront groups in key order, and its tile total
  uint32_t run = 0;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    const uint32_t c = hw[v][tid];
    hw[v][tid] = (uint16_t)run;
    run += c;
  }
  uint32_t total;
  lbase[tid] = block_exclusive_scan(run, total);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    if (wbase + 64 * i + lane < n) {
      const uint32_t p = lbase[dg[i]] + hw[w][dg[i]] + rk[i];
      if (p < (uint32_t)TILE) {  // always true; keeps a miscount from writing outside the tile
        sk[p] = k[i];
        sv[p] = val[i];
      }
    }
  }
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * TILE;
  const int cnt_tile = (int)(n - base < TILE ? n - base : TILE);
  for (int j = tid; j < cnt_tile; j += NT) {
    const K kk = sk[j];
    const uint32_t d = digit_of(kk, shift, mask);
    const int64_t pos = (int64_t)gbase[d] + (j - (int64_t)lbase[d]);
    if (pos >= 0 && pos < n) {  // always true; keeps a miscount from writing outside the output
      kout[pos] = kk;
      vout(pos, sv[j]);
    }
  }
}

// zero key bits: the input in order, through the writer
template <typename K, typename V, typename VW>
__global__ __launch_bounds__(NT) void rs_copy_kernel(const K* __restrict__ kin, const V* __restrict__ vin,
                                                     K* __restrict__ kout, VW vout, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (i < n) {
    kout[i] = kin[i];
    vout(i, vin[i]);
  }
}

// Stable sort of (kin, vin)[0, n) by key bits [begin_bit, end_bit) into (kout, vout);
// the inputs are left unchanged. tmp == nullptr stores the temporary size.
// Keys must be unsigned; n < 2^32.
// radix_sort_pairs_to: the same, with the last pass's values stored by
// `last` (vout then only serves as scratch between passes).
template <typename K, typename V, typename LastW>
hipError_t radix_sort_pairs_to(void* tmp, size_t& tmp_bytes, const K* kin, K* kout, const V* vin, V* vout,
                               int64_t n, int begin_bit, int end_bit, LastW last, hipStream_t st = 0) {
  if (n < 0 || n > (int64_t)UINT32_MAX || begin_bit < 0 || end_bit > (int)(8 * sizeof(K)) || end_bit < begin_bit)
    return hipErrorInvalidValue;
  constexpr int IPT = sort_ipt<K, V>();
  constexpr int TILE = NT * IPT;
  const int64_t ntiles = (n + TILE - 1) / TILE;
  const int64_t table = (int64_t)RADIX * (ntiles > 0 ? ntiles : 1);
  // chunks of ch tiles for the column scan: at most 1024 chunks, so the
  // one-workgroup step walks at most 1024 rows
  const int64_t ch = ntiles > 32 * 1024 ? (ntiles + 1023) / 1024 : 32;
  const int64_t nchunks = ntiles > 0 ? (ntiles + ch - 1) / ch : 1;
  const size_t kb = align256((size_t)n * sizeof(K)), vb = align256((size_t)n * sizeof(V));
  const size_t cb = align256((size_t)table * sizeof(uint32_t));
  const size_t need = kb + vb + cb + align256((size_t)nchunks * RADIX * sizeof(uint32_t));
  if (!tmp) {
    tmp_bytes = need;
    return hipSuccess;
  }
  if (tmp_bytes < need) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  K* tk = (K*)tmp;
  V* tv = (V*)((char*)tmp + kb);
  uint32_t* counts = (uint32_t*)((char*)tmp + kb + vb);
  uint32_t* csum = (uint32_t*)((char*)tmp + kb + vb + cb);
  const int passes = (end_bit - begin_bit + 7) / 8;
  if (passes == 0) {
    hipLaunchKernelGGL((rs_copy_kernel<K, V, LastW>), dim3((unsigned)((n + NT - 1) / NT)), dim3(NT), 0, st, kin, vin,
                       kout, last, n);
    return hipGetLastError();
  }
  const K* sk = kin;
  const V* sv = vin;
  for (int p = 0; p < passes; ++p) {
    // the last pass writes the output: an odd count starts there, an even one in tmp
    const bool to_out = ((passes - 1 - p) & 1) == 0;
    K* dk = to_out ? kout : tk;
    V* dv = to_out ? vout : tv;
    const int shift = begin_bit + 8 * p;
    const int bits = end_bit - shift < 8 ? end_bit - shift : 8;
    const uint32_t mask = (1u << bits) - 1;
    hipLaunchKernelGGL((rs_count_kernel<K, IPT>), dim3((unsigned)ntiles), dim3(NT), 0, st, sk, n, shift, mask,
                       counts);
    hipLaunchKernelGGL(rs_chunk_sum_kernel<uint32_t>, dim3((unsigned)nchunks), dim3(NT), 0, st, (const uint32_t*)counts, ntiles,
                       ch, csum);
    hipLaunchKernelGGL(rs_chunk_base_kernel<uint32_t>, dim3(1), dim3(NT * CB_PARTS), 0, st, csum, nchunks);
    hipLaunchKernelGGL(rs_chunk_apply_kernel<uint32_t>, dim3((unsigned)nchunks), dim3(NT), 0, st, counts, ntiles, ch,
                       (const uint32_t*)csum);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p == passes - 1)
      hipLaunchKernelGGL((rs_scatter_kernel<K, V, IPT, LastW>), dim3((unsigned)ntiles), dim3(NT), 0, st, sk, sv, dk,
                         last, n, shift, mask, (const uint32_t*)counts);
    else
      hipLaunchKernelGGL((rs_scatter_kernel<K, V, IPT, VStore<V>>), dim3((unsigned)ntiles), dim3(NT), 0, st, sk, sv,
                         dk, VStore<V>{dv}, n, shift, mask, (const uint32_t*)counts);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    sk = dk;
    sv = dv;
  }
  return hipSuccess;
}

template <typename K, typename V>
hipError_t radix_sort_pairs(void* tmp, size_t& tmp_bytes, const K* kin, K* kout, const V* vin, V* vout, int64_t n,
                            int begin_bit, int end_bit, hipStream_t st = 0) {
  return radix_sort_pairs_to(tmp, tmp_bytes, kin, kout, vin, vout, n, begin_bit, end_bit, VStore<V>{vout}, st);
}

}  // namespace rsort
}  // namespace tsp
