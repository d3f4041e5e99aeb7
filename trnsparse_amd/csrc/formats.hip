// Device-side sparse format construction (reference trnsparse/formats.py),
// bit-exact in structure with the reference's rules:
//   BSR from_dense (formats.py:183-221): pad to a block multiple with zeros,
//     keep block (i, j) iff max |v| over the padded block > threshold (a NaN
//     in the block makes the max NaN: not kept), block rows in order, block
//     columns increasing within a row, blocks copied row-major with the
//     padding zero.
//   BSR to_dense (formats.py:233-251): every stored block written in place
//     (a later entry of the same block wins, as the reference's loop), the
//     rest zero, cropped to the unpadded shape.
//   CSR from_dense (formats.py:269-278): keep |v| > threshold, rows in order,
//     columns increasing (torch.where order, then the COO sort by row*n+col).
//   COO to_csr (formats.py:104-124): entries sorted by the key row*n + col
//     (stable: equal keys keep their input order), row_ptrs = cumulative
//     row counts.
//   CSR to_coo (formats.py:54-65): row index of every entry.
//   CSR to_dense (formats.py:49-52, torch sparse_csr to_dense): duplicate
//     entries of a row add up in entry order.
//   COO to CSR with duplicates summed (the coalesce of sparse_add,
//     ops.py:107-132): the sorted order above, one entry per distinct
//     (row, col) holding the sum of its duplicates in input order; explicit
//     zeros stay.
// Thresholds compare in the matrix dtype with the threshold rounded to it,
// as torch compares a tensor with a Python float (double -> float -> bf16
// for bf16).
//
// All of it is HBM-bound integer / byte work: no MFMA. Kernels read the
// dense matrix with 16-byte loads where the row stride and base allow.
#include "common.h"

#include "radix_sort.h"

namespace {

// ------------------------------------------------------------ element ops

template <typename T> struct Ops;
template <> struct Ops<float> {
  typedef float thr_t;
  static __device__ bool gt(float v, float t) { return fabsf(v) > t; }
  static __device__ bool nan(float v) { return v != v; }
};
template <> struct Ops<double> {
  typedef double thr_t;
  static __device__ bool gt(double v, double t) { return fabs(v) > t; }
  static __device__ bool nan(double v) { return v != v; }
};
template <> struct Ops<uint16_t> {  // bf16 bits
  typedef float thr_t;              // the bf16-rounded threshold, exact in float
  static __device__ bool gt(uint16_t v, float t) { return tsp::bf16_bits_to_f32(v & 0x7fff) > t; }
  static __device__ bool nan(uint16_t v) { return (v & 0x7fff) > 0x7f80; }
};

template <typename T> typename Ops<T>::thr_t round_threshold(double t);
template <> float round_threshold<float>(double t) { return (float)t; }
template <> double round_threshold<double>(double t) { return t; }
template <> float round_threshold<uint16_t>(double t) { return tsp::bf16_bits_to_f32(tsp::f32_to_bf16_bits((float)t)); }

// ------------------------------------------------------------------- scan

// out[0] = 0, out[i + 1] = sum_{k <= i} counts[i]; one workgroup of 1024.
__global__ __launch_bounds__(1024) void exclusive_scan_kernel(const int64_t* __restrict__ counts, int64_t n,
                                                              int64_t* __restrict__ out) {
  __shared__ int64_t part[1024];
  __shared__ int64_t carry;
  const int tid = threadIdx.x;
  if (tid == 0) {
    carry = 0;
    out[0] = 0;
  }
  __syncthreads();
  for (int64_t base = 0; base < n; base += 1024) {
    const int64_t i = base + tid;
    int64_t v = i < n ? counts[i] : 0;
    part[tid] = v;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {  // Hillis-Steele inclusive scan
      const int64_t add = tid >= o ? part[tid - o] : 0;
      __syncthreads();
      part[tid] += add;
      __syncthreads();
    }
    if (i < n) out[i + 1] = carry + part[tid];
    __syncthreads();
    if (tid == 1023) carry += part[1023];
    __syncthreads();
  }
}

int scan_counts(const int64_t* counts, int64_t n, int64_t* out, hipStream_t st) {
  hipLaunchKernelGGL(exclusive_scan_kernel, dim3(1), dim3(1024), 0, st, counts, n, out);
  return tsp::check_launch("exclusive_scan launch");
}

// Vector width (elements) of 16-byte loads for a row-major matrix with row
// stride ld elements at base p; 1 when the rows are not 16-byte aligned.
template <typename T> int vec_width(const void* p, int64_t ld) {
  const int v = 16 / (int)sizeof(T);
  return (((uintptr_t)p % 16) == 0 && ld % v == 0) ? v : 1;
}

template <typename T, int V> struct alignas(sizeof(T) * V) Vec { T e[V]; };

template <typename T, int V> __device__ inline Vec<T, V> load_vec(const T* p) {
  if constexpr (V == 1) {
    return Vec<T, V>{{*p}};
  } else {
    return *(const Vec<T, V>*)p;  // 16-byte aligned by construction
  }
}

// ------------------------------------------------------------ BSR from dense

// keep[i * nbc + j] for every block of the padded grid; one workgroup per
// block, threads over V-element pieces of the block's rows.
template <typename T, int V>
__global__ __launch_bounds__(256) void bsr_keep_kernel(const T* __restrict__ A, int64_t lda, int64_t m, int64_t n,
                                                       int64_t b, int64_t nbc, typename Ops<T>::thr_t thr,
                                                       uint8_t* __restrict__ keep) {
  const int64_t blk = blockIdx.x;
  const int64_t i = blk / nbc, j = blk % nbc;
  const int64_t r0 = i * b, c0 = j * b;
  const int64_t rows = m - r0 < b ? m - r0 : b, cols = n - c0 < b ? n - c0 : b;
  const int64_t pieces = b / V;  // b % V == 0 on the vector path
  int gt = 0, nan = 0;
  for (int64_t e = threadIdx.x; e < rows * pieces; e += 256) {
    const int64_t r = e / pieces, c = (e % pieces) * V;
    if (c >= cols) continue;
    const T* p = A + (r0 + r) * lda + c0 + c;
    if (V > 1 && c + V <= cols) {
      const Vec<T, V> v = load_vec<T, V>(p);
#pragma unroll
      for (int k = 0; k < V; ++k) {
        gt |= Ops<T>::gt(v.e[k], thr);
        nan |= Ops<T>::nan(v.e[k]);
      }
    } else {
      for (int64_t k = 0; k < V && c + k < cols; ++k) {
        gt |= Ops<T>::gt(p[k], thr);
        nan |= Ops<T>::nan(p[k]);
      }
    }
  }
  gt = __syncthreads_or(gt);
  nan = __syncthreads_or(nan);
  if (threadIdx.x == 0) {
    // the zero padding of an edge block takes part in the max
    const bool padded = rows < b || cols < b;
    const bool pad_gt = padded && (typename Ops<T>::thr_t)0 > thr;
    keep[blk] = (!nan && (gt || pad_gt)) ? 1 : 0;
  }
}

// counts[i] = number of kept blocks in block row i; one wavefront per row.
__global__ __launch_bounds__(256) void row_count_u8_kernel(const uint8_t* __restrict__ keep, int64_t rows,
                                                           int64_t cols, int64_t* __restrict__ counts) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  int64_t c = 0;
  for (int64_t j = lane; j < cols; j += 64) c += keep[r * cols + j];
  c = tsp::wave_sum(c);
  if (lane == 0) counts[r] = c;
}

// col_indices of block row i (kept columns in increasing order), one
// workgroup per block row: prefix sums of the keep flags in chunks of 256.
__global__ __launch_bounds__(256) void bsr_cols_kernel(const uint8_t* __restrict__ keep, int64_t nbc,
                                                       const int64_t* __restrict__ row_ptrs,
                                                       int64_t* __restrict__ col_indices) {
  __shared__ int part[256];
  const int64_t i = blockIdx.x;
  const int tid = threadIdx.x;
  int64_t pos = row_ptrs[i];
  for (int64_t base = 0; base < nbc; base += 256) {
    const int64_t j = base + tid;
    const int f = j < nbc ? keep[i * nbc + j] : 0;
    part[tid] = f;
    __syncthreads();
    for (int o = 1; o < 256; o <<= 1) {
      const int add = tid >= o ? part[tid - o] : 0;
      __syncthreads();
      part[tid] += add;
      __syncthreads();
    }
    if (f) col_indices[pos + part[tid] - 1] = j;
    pos += part[255];
    __syncthreads();
  }
}

// block row of stored block k: the last i with row_ptrs[i] <= k.
__device__ inline int64_t block_row_of(const int64_t* __restrict__ row_ptrs, int64_t mb, int64_t k) {
  int64_t lo = 0, hi = mb;  // row_ptrs[lo] <= k < row_ptrs[hi]
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (row_ptrs[mid] <= k)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

// blocks[k] = the padded b x b block (i_k, col_indices[k]) of A; one
// workgroup per stored block.
template <typename T, int V>
__global__ __launch_bounds__(256) void bsr_gather_kernel(const T* __restrict__ A, int64_t lda, int64_t m, int64_t n,
                                                         int64_t b, int64_t mb, const int64_t* __restrict__ row_ptrs,
                                                         const int64_t* __restrict__ col_indices,
                                                         T* __restrict__ blocks) {
  const int64_t k = blockIdx.x;
  const int64_t i = block_row_of(row_ptrs, mb, k), j = col_indices[k];
  const int64_t r0 = i * b, c0 = j * b;
  const int64_t rows = m - r0 < b ? m - r0 : b, cols = n - c0 < b ? n - c0 : b;
  const int64_t pieces = b / V;
  T* out = blocks + k * b * b;
  for (int64_t e = threadIdx.x; e < b * pieces; e += 256) {
    const int64_t r = e / pieces, c = (e % pieces) * V;
    Vec<T, V> v;
    if (V > 1 && r < rows && c + V <= cols) {
      v = load_vec<T, V>(A + (r0 + r) * lda + c0 + c);
    } else {
#pragma unroll
      for (int kk = 0; kk < V; ++kk) v.e[kk] = (r < rows && c + kk < cols) ? A[(r0 + r) * lda + c0 + c + kk] : T(0);
    }
    *(Vec<T, V>*)(out + r * b + c) = v;
  }
}

// ------------------------------------------------------------- BSR to dense

// out (m x n, row stride ldo): workgroup per output block (i, j); the last
// stored entry of block row i with column j supplies it, else zeros.
template <typename T>
__global__ __launch_bounds__(256) void bsr_to_dense_kernel(const T* __restrict__ blocks,
                                                           const int64_t* __restrict__ row_ptrs,
                                                           const int64_t* __restrict__ col_indices, int64_t b,
                                                           int64_t nbc, int64_t m, int64_t n, T* __restrict__ out,
                                                           int64_t ldo) {
  __shared__ unsigned long long found;  // 1 + index of the last match, 0: none
  const int64_t blk = blockIdx.x;
  const int64_t i = blk / nbc, j = blk % nbc;
  if (threadIdx.x == 0) found = 0;
  __syncthreads();
  const int64_t s = row_ptrs[i], e = row_ptrs[i + 1];
  for (int64_t k = s + threadIdx.x; k < e; k += 256)
    if (col_indices[k] == j) atomicMax(&found, (unsigned long long)(k + 1));
  __syncthreads();
  const int64_t k = (int64_t)found - 1;
  const int64_t r0 = i * b, c0 = j * b;
  const int64_t rows = m - r0 < b ? m - r0 : b, cols = n - c0 < b ? n - c0 : b;
  for (int64_t t = threadIdx.x; t < rows * cols; t += 256) {
    const int64_t r = t / cols, c = t % cols;
    out[(r0 + r) * ldo + c0 + c] = k >= 0 ? blocks[k * b * b + r * b + c] : T(0);
  }
}

// ------------------------------------------------------------ CSR from dense

// counts[r] = #{c : |A[r][c]| > thr}; one wavefront per row.
template <typename T, int V>
__global__ __launch_bounds__(256) void csr_count_kernel(const T* __restrict__ A, int64_t lda, int64_t m, int64_t n,
                                                        typename Ops<T>::thr_t thr, int64_t* __restrict__ counts) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= m) return;
  const T* row = A + r * lda;
  int64_t c = 0;
  for (int64_t base = (int64_t)lane * V; base < n; base += 64 * V) {
    if (V > 1 && base + V <= n) {
      const Vec<T, V> v = load_vec<T, V>(row + base);
#pragma unroll
      for (int k = 0; k < V; ++k) c += Ops<T>::gt(v.e[k], thr);
    } else {
      for (int64_t k = 0; k < V && base + k < n; ++k) c += Ops<T>::gt(row[base + k], thr);
    }
  }
  c = tsp::wave_sum(c);
  if (lane == 0) counts[r] = c;
}

// col_indices / values of row r in column order; one wavefront per row:
// per 64*V-column chunk, a lane's kept count, an exclusive scan over lanes,
// then each lane writes its kept entries in order.
template <typename T, int V>
__global__ __launch_bounds__(256) void csr_fill_kernel(const T* __restrict__ A, int64_t lda, int64_t m, int64_t n,
                                                       typename Ops<T>::thr_t thr, const int64_t* __restrict__ row_ptrs,
                                                       int64_t* __restrict__ col_indices, T* __restrict__ values) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= m) return;
  const T* row = A + r * lda;
  int64_t pos = row_ptrs[r];
  for (int64_t chunk = 0; chunk < n; chunk += 64 * V) {
    const int64_t base = chunk + (int64_t)lane * V;
    Vec<T, V> v;
    int cnt = 0;
    if (V > 1 && base + V <= n) {
      v = load_vec<T, V>(row + base);
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) v.e[k] = base + k < n ? row[base + k] : T(0);
    }
    unsigned keepm = 0;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const bool f = base + k < n && Ops<T>::gt(v.e[k], thr);
      keepm |= (unsigned)f << k;
      cnt += f;
    }
    // exclusive scan of cnt over the wavefront
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(incl, o, 64);
      if (lane >= o) incl += t;
    }
    const int total = __shfl(incl, 63, 64);
    int64_t w = pos + incl - cnt;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      if (keepm & (1u << k)) {
        col_indices[w] = base + k;
        values[w] = v.e[k];
        ++w;
      }
    }
    pos += total;
  }
}

// ------------------------------------------------------------- CSR to dense

// out zeroed beforehand; thread per row adds its entries in order.
template <typename T>
__global__ __launch_bounds__(256) void csr_to_dense_kernel(const T* __restrict__ values,
                                                           const int64_t* __restrict__ col_indices,
                                                           const int64_t* __restrict__ row_ptrs, int64_t m,
                                                           T* __restrict__ out, int64_t ldo) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= m) return;
  for (int64_t k = row_ptrs[r]; k < row_ptrs[r + 1]; ++k) {
    T* p = out + r * ldo + col_indices[k];
    if constexpr (sizeof(T) == 2)
      *p = tsp::f32_to_bf16_bits(tsp::bf16_bits_to_f32(*p) + tsp::bf16_bits_to_f32(values[k]));
    else
      *p += values[k];
  }
}

// out[r][c] = 0 for r < m, c < n (row stride ldo); thread per element.
template <typename T>
__global__ __launch_bounds__(256) void zero_rows_kernel(T* __restrict__ out, int64_t m, int64_t n, int64_t ldo) {
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < m * n; t += (int64_t)gridDim.x * 256)
    out[(t / n) * ldo + t % n] = T(0);
}

// ------------------------------------------------------------- CSR -> COO

// Entry -> row for CSR entries: fn(k, r) with r = the row of entry k (the
// last r with row_ptrs[r] <= k). A workgroup takes a tile of ETILE
// consecutive entries; two searches of row_ptrs bound the tile's rows, and
// when those span at most RSPAN row pointers they are staged in LDS, so each
// entry's search is a short one there (otherwise over row_ptrs itself).
constexpr int ETILE = 4096;
constexpr int RSPAN = 2048;

template <typename Fn>
__global__ __launch_bounds__(256) void entry_rows_kernel(const int64_t* __restrict__ row_ptrs, int64_t m, int64_t nnz,
                                                         Fn fn) {
  __shared__ int64_t srp[RSPAN + 1];
  __shared__ int64_t span[2];
  const int64_t e0 = (int64_t)blockIdx.x * ETILE;
  const int64_t e1 = e0 + ETILE < nnz ? e0 + ETILE : nnz;
  if (threadIdx.x == 0) {
    span[0] = block_row_of(row_ptrs, m, e0);
    span[1] = block_row_of(row_ptrs, m, e1 - 1);
  }
  __syncthreads();
  const int64_t rlo = span[0], nr = span[1] - rlo + 1;  // rows rlo .. rlo + nr - 1
  const bool staged = nr <= RSPAN;
  if (staged)
    for (int64_t i = threadIdx.x; i <= nr; i += 256) srp[i] = row_ptrs[rlo + i];
  __syncthreads();
  for (int64_t k = e0 + threadIdx.x; k < e1; k += 256) {
    int64_t r;
    if (staged) {
      int lo = 0, hi = (int)nr;  // srp[lo] <= k < srp[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (srp[mid] <= k)
          lo = mid;
        else
          hi = mid;
      }
      r = rlo + lo;
    } else {
      r = block_row_of(row_ptrs, m, k);
    }
    fn(k, r);
  }
}

struct RowsOut {
  int64_t* rows;
  __device__ void operator()(int64_t k, int64_t r) const { rows[k] = r; }
};

template <typename Fn>
int launch_entry_rows(const int64_t* row_ptrs, int64_t m, int64_t nnz, Fn fn, hipStream_t st, const char* what) {
  const int64_t g = tsp::ceil_div(nnz, ETILE);
  if (g > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "%s: too many entries", what);
  hipLaunchKernelGGL(entry_rows_kernel<Fn>, dim3((unsigned)g), dim3(256), 0, st, row_ptrs, m, nnz, fn);
  return tsp::check_launch(what);
}

// ------------------------------------------------------------- COO -> CSR

// K is uint32_t when every key, row_ptrs' bound m * n included, fits in 32
// bits: the radix sort then moves half the key bytes per pass.
template <typename K>
__global__ __launch_bounds__(256) void coo_keys_kernel(const int64_t* __restrict__ rows,
                                                       const int64_t* __restrict__ cols, int64_t nnz, int64_t n,
                                                       K* __restrict__ keys) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= nnz) return;
  keys[k] = (K)(rows[k] * n + cols[k]);
}

// column of each sorted key (key = row * n + col)
template <typename K>
__global__ __launch_bounds__(256) void key_cols_kernel(const K* __restrict__ keys, int64_t nnz, int64_t n,
                                                       int64_t* __restrict__ cols_out) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= nnz) return;
  cols_out[k] = (int64_t)(keys[k] % (K)n);
}

// row_ptrs[r] = first k with sorted key >= r * n (r = 0 .. m).
template <typename K>
__global__ __launch_bounds__(256) void coo_row_ptrs_kernel(const K* __restrict__ keys, int64_t nnz, int64_t m,
                                                           int64_t n, int64_t* __restrict__ row_ptrs) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r > m) return;
  const K key = (K)(r * n);
  int64_t lo = 0, hi = nnz;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < key)
      lo = mid + 1;
    else
      hi = mid;
  }
  row_ptrs[r] = lo;
}

// head[k] = 1 where sorted key k starts a run of equal keys
__global__ __launch_bounds__(256) void run_heads_kernel(const uint64_t* __restrict__ keys, int64_t nnz,
                                                        int64_t* __restrict__ head) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= nnz) return;
  head[k] = (k == 0 || keys[k] != keys[k - 1]) ? 1 : 0;
}

// for each run head k (seg[k] = its 1-based run index): the run's key, its
// column and the sum of its values (sorted along with the keys) in sorted
// (= input, the sort is stable) order
// Keys: row * n + col, or (PACKED) row << 32 | col.
template <bool PACKED>
__device__ inline int64_t key_col(uint64_t key, int64_t n) {
  return PACKED ? (int64_t)(key & 0xffffffffull) : (int64_t)(key % (uint64_t)n);
}
template <bool PACKED>
__device__ inline uint64_t row_key(int64_t r, int64_t n) {
  return PACKED ? (uint64_t)r << 32 : (uint64_t)(r * n);
}

template <typename T, bool PACKED = false>
__global__ __launch_bounds__(256) void run_sum_kernel(const uint64_t* __restrict__ keys,
                                                      const int64_t* __restrict__ seg,
                                                      const int64_t* __restrict__ head, const T* __restrict__ vals,
                                                      int64_t nnz, int64_t n, uint64_t* __restrict__ ukeys,
                                                      int64_t* __restrict__ cols_out, T* __restrict__ vals_out) {
  typedef typename tsp::Acc<T>::type AccT;
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= nnz || !head[k]) return;
  const int64_t s = seg[k] - 1;
  const uint64_t key = keys[k];
  AccT sum = tsp::to_acc(vals[k]);
  for (int64_t t = k + 1; t < nnz && keys[t] == key; ++t) sum += tsp::to_acc(vals[t]);
  ukeys[s] = key;
  cols_out[s] = key_col<PACKED>(key, n);
  vals_out[s] = tsp::from_acc<T>(sum);
}

// row_ptrs[r] = first run with key >= r * n, over the seg[nnz-1] runs
template <bool PACKED = false>
__global__ __launch_bounds__(256) void run_row_ptrs_kernel(const uint64_t* __restrict__ ukeys,
                                                           const int64_t* __restrict__ seg, int64_t nnz, int64_t m,
                                                           int64_t n, int64_t* __restrict__ row_ptrs) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r > m) return;
  const int64_t U = seg[nnz - 1];
  const uint64_t key = row_key<PACKED>(r, n);
  int64_t lo = 0, hi = U;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (ukeys[mid] < key)
      lo = mid + 1;
    else
      hi = mid;
  }
  row_ptrs[r] = lo;
}

// ------------------------------------------------------------- CSR sum
//
// Union sum of two CSR operands (the coalesce of sparse_add). Row r's
// entries j = 0..n-1 are A's entries of the row followed by B's (input
// order). Entry i heads its column when no earlier entry has the same
// column; the heads are the output entries, ranked by column, each holding
// the sum of its column's entries in input order — what a stable sort of the
// concatenated COO by (row, col) followed by a run sum gives. Two passes
// (count heads per row; after a scan, write them). Rows of at most 64
// entries take a wavefront each and sort their entries across its lanes;
// rows of up to SUM_CAP entries are staged in LDS with their neighbours in
// 64-row chunks; longer rows take a 256-thread workgroup each that streams
// the row through LDS in tiles and keeps the head flags in workspace.
constexpr int SUM_CAP = 4096;
constexpr int SUM_RPW = 64;
constexpr int LONG_TILE = 4096;

template <typename T>
struct SumRow {
  const T* av;
  const int64_t* ac;
  const T* bv;
  const int64_t* bc;
  int64_t a0, na, b0, n;
  __device__ uint32_t col(int64_t j) const { return (uint32_t)(j < na ? ac[a0 + j] : bc[b0 + j - na]); }
  __device__ typename tsp::Acc<T>::type val(int64_t j) const {
    return tsp::to_acc(j < na ? av[a0 + j] : bv[b0 + j - na]);
  }
};

template <typename T>
__device__ inline SumRow<T> sum_row(const T* av, const int64_t* ac, const int64_t* ar, const T* bv, const int64_t* bc,
                                    const int64_t* br, int64_t r) {
  const int64_t a0 = ar[r], na = ar[r + 1] - a0, b0 = br[r];
  return SumRow<T>{av, ac, bv, bc, a0, na, b0, na + (br[r + 1] - b0)};
}

// rows with n <= 64: a wavefront takes two rows at a time. Each row's
// (column, position) keys are sorted across lanes by a bitonic network —
// both rows side by side in the two 32-lane halves when both hold at most
// 32 entries, else one row at a time over all 64 lanes — so heads, their
// ranks (a ballot prefix count) and each run (the lanes that follow with
// the same column, in input order) come from lane shuffles. Keys are 32-bit
// (column << 6 | position) when the columns fit 26 bits, else 64-bit.
constexpr int WAVE_ROW = 64;

template <typename K>
__device__ inline K sum_key(uint32_t c, int pos) {
  return sizeof(K) == 4 ? (K)((c << 6) | (uint32_t)pos) : (K)(((uint64_t)c << 32) | (uint64_t)pos);
}
template <typename K>
__device__ inline uint32_t key_col_of(K k) {
  return sizeof(K) == 4 ? (uint32_t)(k >> 6) : (uint32_t)((uint64_t)k >> 32);
}

// Value of lane ^ J (J a power of two below 64) without ds_bpermute: DPP
// quad permutes (1, 2), DPP row rotates (4: rotate by 4 or 12, picked per
// lane; 8), and the gfx950 swaps of rows 16 apart and halves 32 apart
// (both operands x: the pair holds the values of the two rows / halves).
template <int J>
__device__ inline uint32_t xor_lane32(uint32_t x) {
  const int lane = (int)(threadIdx.x & 63);
  if constexpr (J == 1) {
    return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (J == 2) {
    return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (J == 4) {
    const uint32_t a = __builtin_amdgcn_mov_dpp(x, 0x124, 0xF, 0xF, false);  // row_ror:4
    const uint32_t b = __builtin_amdgcn_mov_dpp(x, 0x12C, 0xF, 0xF, false);  // row_ror:12
    return (lane & 4) ? a : b;
  } else if constexpr (J == 8) {
    return __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else {
    static_assert(J == 32, "xor distance");
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}
template <int J, typename K>
__device__ inline K xor_lane(K x) {
  if constexpr (sizeof(K) == 4) {
    return (K)xor_lane32<J>((uint32_t)x);
  } else {
    const uint64_t u = (uint64_t)x;
    return (K)(((uint64_t)xor_lane32<J>((uint32_t)(u >> 32)) << 32) | xor_lane32<J>((uint32_t)u));
  }
}

// bitonic sort of one key per lane across groups of G lanes (G = 32: each
// half on its own), ascending in every group; l = lane % G
template <typename K, int KK, int J>
__device__ inline K bitonic_merge(K key, int l) {
  const K other = xor_lane<J>(key);
  const bool keep_min = ((l & J) == 0) == ((l & KK) == 0);
  key = keep_min ? (other < key ? other : key) : (other > key ? other : key);
  if constexpr (J > 1)
    return bitonic_merge<K, KK, J / 2>(key, l);
  else
    return key;
}
template <typename K, int G, int KK>
__device__ inline K bitonic_stages(K key, int l) {
  key = bitonic_merge<K, KK, KK / 2>(key, l);
  if constexpr (KK < G)
    return bitonic_stages<K, G, KK * 2>(key, l);
  else
    return key;
}
template <typename K, int G>
__device__ inline K lane_sort(K key, int lane) {
  return bitonic_stages<K, G, 2>(key, lane & (G - 1));
}
// Ascending sort of a bitonic sequence over groups of G lanes (the
// half-cleaner steps of the last stage only).
template <typename K, int J>
__device__ inline K bitonic_clean(K key, int l) {
  const K other = xor_lane<J>(key);
  key = (l & J) == 0 ? (other < key ? other : key) : (other > key ? other : key);
  if constexpr (J > 1)
    return bitonic_clean<K, J / 2>(key, l);
  else
    return key;
}
template <typename K, int G>
__device__ inline K lane_merge(K key, int lane) {
  return bitonic_clean<K, G / 2>(key, lane & (G - 1));
}

// Each wavefront takes one chunk of SUM_CHUNK consecutive rows (lane j
// holds the row pointers of rows 2j, 2j + 1 and 2j + 2 of the chunk, loaded
// once, read out with readlane) and sorts its row pairs in order with the
// entry loads issued two pairs ahead: loads are branch-free (a lane past its
// row's end reads row_ptrs[0] instead), so the wait before a pair's sort
// covers only its own loads.
constexpr int SUM_CHUNK = 128;  // rows per wavefront (64 pairs)
struct SumPair {
  int64_t a0[2], na[2], b0[2], o[2];
  int n[2];  // entries of each row; -1: past m or not this kernel's row
};
template <typename T>
struct SumEnt {
  uint32_t c[2];
  T v[2];  // the lane's entry in pass 0 / 1 (pass 1 only when the rows do not share the lanes)
};

template <typename T, bool WRITE, typename K>
__global__ __launch_bounds__(256) void csr_sum_wave_kernel(const T* __restrict__ av, const int64_t* __restrict__ ac,
                                                           const int64_t* __restrict__ ar, const T* __restrict__ bv,
                                                           const int64_t* __restrict__ bc,
                                                           const int64_t* __restrict__ br, int64_t m,
                                                           int64_t* __restrict__ ucount,
                                                           const int64_t* __restrict__ out_rp,
                                                           int64_t* __restrict__ out_col, T* __restrict__ out_val) {
  typedef typename tsp::Acc<T>::type AccT;
  const int lane = threadIdx.x & 63;
  const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * SUM_CHUNK;
  if (r0 >= m) return;
  const int npairs = (int)((m - r0 < SUM_CHUNK ? m - r0 : SUM_CHUNK) + 1) / 2;
  // row pointers of rows r0 + 2 lane + {0, 1, 2} (clamped to m)
  int64_t ra[3], rbp[3], ro[2];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int64_t i = r0 + 2 * lane + j < m ? r0 + 2 * lane + j : m;
    ra[j] = ar[i];
    rbp[j] = br[i];
    if (WRITE && j < 2) ro[j] = out_rp[i];
  }
  auto rl64 = [](int64_t v, int l) {
    const uint64_t u = (uint64_t)v;
    return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l) << 32) |
                     (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l));
  };
  auto pair_of = [&](int q, SumPair& p) {
    const int l = q < npairs ? q : npairs - 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      p.a0[i] = rl64(ra[i], l);
      p.na[i] = rl64(ra[i + 1], l) - p.a0[i];
      p.b0[i] = rl64(rbp[i], l);
      if (WRITE) p.o[i] = rl64(ro[i], l);
      const int64_t nn = p.na[i] + (rl64(rbp[i + 1], l) - p.b0[i]);
      p.n[i] = (q < npairs && r0 + 2 * q + i < m && nn <= WAVE_ROW) ? (int)nn : -1;
    }
  };
  auto halves_of = [](const SumPair& p) { return p.n[0] <= 32 && p.n[1] <= 32; };
  auto load_ent = [&](const SumPair& p, SumEnt<T>& e) {
    const bool halves = halves_of(p);
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int i = halves ? (lane >> 5) : pass;
      const int pos = halves ? (lane & 31) : lane;
      // (selects, not indexing: a lane-dependent index would put p in scratch)
      const int ni = i ? p.n[1] : p.n[0];
      const int64_t nai = i ? p.na[1] : p.na[0], a0i = i ? p.a0[1] : p.a0[0], b0i = i ? p.b0[1] : p.b0[0];
      // lane pos of the row's group holds A's entry pos (pos < na) or B's
      // entry G - 1 - pos (pos >= G - nb): A ascending, B reversed
      const int G = halves ? 32 : 64;
      const bool use = (!halves || pass == 0) && ni > 0;
      const bool in_a = use && pos < nai;
      const bool in_b = use && pos >= G - (ni - nai);
      const int jb = G - 1 - pos;
      const int64_t* cp = in_a ? ac + a0i + pos : (in_b ? bc + b0i + jb : ar);
      const T* vp = in_a ? av + a0i + pos : (in_b ? bv + b0i + jb : (const T*)ar);
      e.c[pass] = (uint32_t)*cp;
      e.v[pass] = *vp;
    }
  };
  auto process = [&](int64_t rb, const SumPair& p, const SumEnt<T>& e) {
    const bool halves = halves_of(p);
    // the rows: both at once in the halves, or one after the other
    // (unrolled: a runtime pass index would put e in scratch)
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      if (halves && pass == 1) break;
      const int i = halves ? (lane >> 5) : pass;  // this lane's row
      const int pos = halves ? (lane & 31) : lane;
      const int nr = i ? p.n[1] : p.n[0];
      if (!halves && nr < 0) continue;  // uniform: the whole wave serves row `pass`
      const int64_t r = rb + i;
      const int G = halves ? 32 : 64;
      const int na = (int)(i ? p.na[1] : p.na[0]), nb = nr - na;
      const bool in_a = nr > 0 && pos < na, in_b = nr > 0 && pos >= G - nb;
      // key: column and the entry's position in the row (A's then B's, in
      // input order), so equal columns keep input order
      K key = (K)~(K)0;  // padding sorts after every entry
      AccT v = 0;
      const uint32_t c = e.c[pass];
      if (in_a || in_b) {
        v = tsp::to_acc(e.v[pass]);
        key = sum_key<K>(c, in_a ? pos : na + (G - 1 - pos));
      }
      // A ascending from the group's first lane, B descending to its last
      // lane: a bitonic sequence when both rows are sorted by column, so the
      // last stage's half-cleaners sort it; any inversion: the full network
      const uint32_t cprev = __shfl_up(c, 1, 64);
      const bool inv = (in_a && pos > 0 && cprev > c) || (in_b && pos > G - nb && cprev < c);
      if (__builtin_amdgcn_ballot_w64(inv) == 0)
        key = halves ? lane_merge<K, 32>(key, lane) : lane_merge<K, 64>(key, lane);
      else
        key = halves ? lane_sort<K, 32>(key, lane) : lane_sort<K, 64>(key, lane);
      const int base = halves ? (lane & 32) : 0;  // first lane of this row's group
      const uint32_t col = key_col_of(key);
      const int kp = (int)(key & 63);             // the entry's position -> the lane holding its value
      const int src = kp < na ? kp : (G - 1 - (kp - na)) & (G - 1);
      const AccT sv = __shfl(v, base + src, 64);
      const uint32_t prev = __shfl_up(col, 1, 64);
      const bool head = pos < nr && (pos == 0 || prev != col);
      const uint64_t hb_all = __builtin_amdgcn_ballot_w64(head);
      const uint64_t hb = halves ? (hb_all >> base) & 0xffffffffull : hb_all;
      if (!WRITE) {
        if (pos == 0 && nr >= 0) ucount[r] = __popcll(hb);
        continue;
      }
      AccT sum = sv;
      bool open = head;
      for (int k = 1; k < WAVE_ROW; ++k) {
        if (__builtin_amdgcn_ballot_w64(open) == 0) break;
        const uint32_t c2 = __shfl_down(col, k, 64);
        const AccT v2 = __shfl_down(sv, k, 64);
        open = open && pos + k < nr && c2 == col;
        if (open) sum += v2;
      }
      if (head) {
        const int64_t o = (i ? p.o[1] : p.o[0]) + __popcll(hb & ((1ull << pos) - 1));
        out_col[o] = (int64_t)col;
        out_val[o] = tsp::from_acc<T>(sum);
      }
    }
  };
  // three (pair, entries) slots used round robin with constant indices, so no
  // register holding a load in flight is copied (a copy would wait for it);
  // the pair count is padded to a multiple of 3 with empty pairs (all rows
  // -1: no output, loads of row_ptrs[0]), so the loop body has no branch
  SumPair P0, P1, P2;
  SumEnt<T> E0, E1, E2;
  auto step = [&](int q, const SumPair& pc, const SumEnt<T>& ec, SumPair& pn, SumEnt<T>& en) {
    pair_of(q + 2, pn);
    load_ent(pn, en);
    process(r0 + 2 * q, pc, ec);
  };
  pair_of(0, P0);
  load_ent(P0, E0);
  pair_of(1, P1);
  load_ent(P1, E1);
  for (int q = 0; q < npairs; q += 3) {
    step(q, P0, E0, P2, E2);
    step(q + 1, P1, E1, P0, E0);
    step(q + 2, P2, E2, P1, E1);
  }
}

// rows with n <= SUM_CAP: a 256-thread workgroup per chunk of SUM_RPW
// consecutive rows, whose entries are staged in LDS at once (column with the
// head flag in bit 31, value, chunk-local row) when they fit SUM_CAP, else
// row by row; row offsets come from a wavefront scan of the row lengths
template <typename T, bool WRITE>
__global__ __launch_bounds__(256) void csr_sum_rows_kernel(const T* __restrict__ av, const int64_t* __restrict__ ac,
                                                           const int64_t* __restrict__ ar, const T* __restrict__ bv,
                                                           const int64_t* __restrict__ bc,
                                                           const int64_t* __restrict__ br, int64_t m,
                                                           int64_t* __restrict__ ucount,
                                                           const int64_t* __restrict__ out_rp,
                                                           int64_t* __restrict__ out_col, T* __restrict__ out_val) {
  typedef typename tsp::Acc<T>::type AccT;
  static_assert(SUM_RPW == 64, "one lane per row in the offset scan");
  __shared__ uint32_t scol[SUM_CAP];
  __shared__ uint8_t srow[SUM_CAP];  // chunk-local row of each staged entry
  __shared__ AccT sval[WRITE ? SUM_CAP : 1];
  __shared__ int64_t ua[SUM_RPW + 1], ub[SUM_RPW + 1];
  __shared__ int32_t off[SUM_RPW + 1];  // chunk-local entry offsets (long rows count 0)
  __shared__ int32_t cnt[SUM_RPW];
  __shared__ int64_t orp[WRITE ? SUM_RPW : 1];  // output row starts
  const int tid = threadIdx.x;
  if (!WRITE && blockIdx.x == 0 && tid == 0) ucount[m] = 0;
  for (int64_t r0 = (int64_t)blockIdx.x * SUM_RPW; r0 < m; r0 += (int64_t)gridDim.x * SUM_RPW) {
    const int nr = (int)(m - r0 < SUM_RPW ? m - r0 : SUM_RPW);
    __syncthreads();  // the previous chunk's LDS reads are done
    if (tid <= nr) {
      ua[tid] = ar[r0 + tid];
      ub[tid] = br[r0 + tid];
      if (WRITE && tid < nr) orp[tid] = out_rp[r0 + tid];
    }
    __syncthreads();
    if (tid < 64) {
      int32_t x = 0;
      if (tid < nr) {
        const int64_t l = (ua[tid + 1] - ua[tid]) + (ub[tid + 1] - ub[tid]);
        x = (l > SUM_CAP || l <= WAVE_ROW) ? 0 : (int32_t)l;  // the other kernels' rows
        cnt[tid] = 0;
      }
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int32_t y = __shfl_up(x, o, 64);
        if (tid >= o) x += y;
      }
      off[tid + 1] = x;
      if (tid == 0) off[0] = 0;
    }
    __syncthreads();
    const int32_t total = off[nr];
    // rows [rb, re) staged together: all rows when they fit, else one by one
    const bool whole = total <= SUM_CAP;
    for (int rb = 0; rb < nr; rb = whole ? nr : rb + 1) {
      const int re = whole ? nr : rb + 1;
      const int32_t base = off[rb], tot = off[re] - base;
      if (!whole) __syncthreads();  // the previous row's LDS reads are done
      for (int e = tid; e < tot; e += 256) {
        int lo = rb, hi = re;  // off[lo] - base <= e < off[hi] - base
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (off[mid] - base <= e)
            lo = mid;
          else
            hi = mid;
        }
        while (off[lo + 1] - base <= e) ++lo;  // skip rows without entries
        const int64_t j = e - (off[lo] - base);
        const int64_t na = ua[lo + 1] - ua[lo];
        const int64_t src = j < na ? ua[lo] + j : ub[lo] + (j - na);
        srow[e] = (uint8_t)lo;
        scol[e] = (uint32_t)(j < na ? ac[src] : bc[src]);
        if (WRITE) sval[e] = tsp::to_acc(j < na ? av[src] : bv[src]);
      }
      __syncthreads();
      for (int e = tid; e < tot; e += 256) {
        const int k = srow[e];
        const uint32_t ci = scol[e] & 0x7fffffffu;
        int dup = 0;
        for (int j = off[k] - base; j < e; ++j) dup += (scol[j] & 0x7fffffffu) == ci;
        if (dup == 0) {
          scol[e] = ci | 0x80000000u;
          if (!WRITE) atomicAdd(&cnt[k], 1);
        }
      }
      __syncthreads();
      if (WRITE) {
        for (int e = tid; e < tot; e += 256) {
          const uint32_t f = scol[e];
          if (!(f >> 31)) continue;
          const int k = srow[e];
          const uint32_t ci = f & 0x7fffffffu;
          int64_t rank = 0;
          AccT sum = sval[e];
          for (int j = off[k] - base; j < off[k + 1] - base; ++j) {
            const uint32_t g = scol[j];
            rank += (g >> 31) && (g & 0x7fffffffu) < ci;
            if (j > e && (g & 0x7fffffffu) == ci) sum += sval[j];
          }
          const int64_t o = orp[k] + rank;
          out_col[o] = (int64_t)ci;
          out_val[o] = tsp::from_acc<T>(sum);
        }
      }
    }
    if (!WRITE) {
      __syncthreads();
      // long rows keep the count the long-row kernel writes
      if (tid < nr) {
        const int64_t l = (ua[tid + 1] - ua[tid]) + (ub[tid + 1] - ub[tid]);
        if (l > WAVE_ROW && l <= SUM_CAP) ucount[r0 + tid] = cnt[tid];
      }
    }
  }
}

// rows with n > SUM_CAP, one 256-thread workgroup each; hflag: a byte per
// union entry (row r's entries at ar[r] + br[r] + j)
template <typename T, bool WRITE>
__global__ __launch_bounds__(256) void csr_sum_long_kernel(const T* __restrict__ av, const int64_t* __restrict__ ac,
                                                           const int64_t* __restrict__ ar, const T* __restrict__ bv,
                                                           const int64_t* __restrict__ bc,
                                                           const int64_t* __restrict__ br, int64_t m,
                                                           uint8_t* __restrict__ hflag, int64_t* __restrict__ ucount,
                                                           const int64_t* __restrict__ out_rp,
                                                           int64_t* __restrict__ out_col, T* __restrict__ out_val) {
  typedef typename tsp::Acc<T>::type AccT;
  __shared__ uint32_t tcol[LONG_TILE];
  __shared__ uint8_t thead[LONG_TILE];
  __shared__ AccT tval[LONG_TILE];
  __shared__ int64_t part[4];
  __shared__ int64_t longs[256];
  __shared__ int nlong;
  const int tid = threadIdx.x;
  // chunks of 256 rows: the long ones are listed, then taken one at a time
  for (int64_t c0 = (int64_t)blockIdx.x * 256; c0 < m; c0 += (int64_t)gridDim.x * 256) {
    __syncthreads();
    if (tid == 0) nlong = 0;
    __syncthreads();
    if (c0 + tid < m) {
      const int64_t rr = c0 + tid;
      if ((ar[rr + 1] - ar[rr]) + (br[rr + 1] - br[rr]) > SUM_CAP) longs[atomicAdd(&nlong, 1)] = rr;
    }
    __syncthreads();
    const int nl = nlong;
    for (int li = 0; li < nl; ++li) {
      const int64_t r = longs[li];
      const SumRow<T> R = sum_row(av, ac, ar, bv, bc, br, r);
      const int64_t n = R.n;
      uint8_t* hf = hflag + ar[r] + br[r];
      int64_t heads = 0;
      if (!WRITE) {
        // head flags: i heads its column when no j < i has it
        for (int64_t i0 = 0; i0 < n; i0 += 256) {
          const int64_t i = i0 + tid;
          const uint32_t ci = i < n ? R.col(i) : 0xffffffffu;
          bool h = i < n;
          for (int64_t t0 = 0; t0 < i0 + 256 && t0 < n; t0 += LONG_TILE) {
            __syncthreads();
            for (int64_t j = t0 + tid; j < t0 + LONG_TILE && j < n; j += 256) tcol[j - t0] = R.col(j);
            __syncthreads();
            const int64_t jend = i < t0 + LONG_TILE ? i : t0 + LONG_TILE;
            for (int64_t j = t0; j < jend && h; ++j) h = tcol[j - t0] != ci;
          }
          if (i < n) hf[i] = h ? 1 : 0;
          heads += h;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) heads += __shfl_xor(heads, o, 64);
        __syncthreads();
        if ((tid & 63) == 0) part[tid >> 6] = heads;
        __syncthreads();
        if (tid == 0) ucount[r] = part[0] + part[1] + part[2] + part[3];
        __syncthreads();
        continue;
      }
      // write: rank of each head among the heads (by column) and the sum of
      // its column's entries, tile by tile in input order
      for (int64_t i0 = 0; i0 < n; i0 += 256) {
        const int64_t i = i0 + tid;
        const bool h = i < n && hf[i];
        const uint32_t ci = i < n ? R.col(i) : 0;
        int64_t rank = 0;
        AccT sum = 0;
        for (int64_t t0 = 0; t0 < n; t0 += LONG_TILE) {
          __syncthreads();
          for (int64_t j = t0 + tid; j < t0 + LONG_TILE && j < n; j += 256) {
            tcol[j - t0] = R.col(j);
            thead[j - t0] = hf[j];
            tval[j - t0] = R.val(j);
          }
          __syncthreads();
          if (h) {
            const int64_t len = n - t0 < LONG_TILE ? n - t0 : LONG_TILE;
            for (int64_t j = 0; j < len; ++j) {
              const uint32_t cj = tcol[j];
              rank += thead[j] && cj < ci;
              if (cj == ci && t0 + j >= i) sum = t0 + j == i ? tval[j] : sum + tval[j];
            }
          }
        }
        if (h) {
          out_col[out_rp[r] + rank] = (int64_t)ci;
          out_val[out_rp[r] + rank] = tsp::from_acc<T>(sum);
        }
      }
    }
  }
}

// ------------------------------------------------------------- CSR transpose
//
// A (m x n) -> A^T: entries in CSR order are stably sorted by column alone
// (32-bit keys), carrying (row, value) as the sort's payload, so within a
// column the rows stay in increasing order and duplicates keep their input
// order: the order of the reference's COO swap + sort by (col, row).
template <typename T>
struct RowVal {
  uint32_t row;
  T val;
};

template <typename T>
struct TrKeys {
  const int64_t* cols;
  const T* vals;
  uint32_t* keys;
  RowVal<T>* payload;
  __device__ void operator()(int64_t k, int64_t r) const {
    keys[k] = (uint32_t)cols[k];
    payload[k] = RowVal<T>{(uint32_t)r, vals[k]};
  }
};

// The sort's last pass stores a transposed entry's (row, value) payload
// straight into the output arrays: the row as the int64 column index.
template <typename T>
struct TrOut {
  int64_t* col;
  T* val;
  __device__ void operator()(int64_t i, const RowVal<T>& p) const {
    col[i] = (int64_t)p.row;
    val[i] = p.val;
  }
};

// row_ptrs[c] = first k with sorted column key >= c (c = 0 .. n). A binary
// search per pointer: as fast as one pass over the keys that fills each
// gap (28 us on cfg2's 16.8 M keys either way), and unlike it independent of
// how the keys spread (a pass that fills gaps took 431 us with every key in
// 16 of 1 M columns).
__global__ __launch_bounds__(256) void tr_row_ptrs_kernel(const uint32_t* __restrict__ keys, int64_t nnz, int64_t n,
                                                          int64_t* __restrict__ row_ptrs) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c > n) return;
  int64_t lo = 0, hi = nnz;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)keys[mid] < c)
      lo = mid + 1;
    else
      hi = mid;
  }
  row_ptrs[c] = lo;
}


int key_bits(int64_t m, int64_t n) {
  const uint64_t maxkey = (uint64_t)(m * n);  // keys < m * n
  int bits = 1;
  while (bits < 64 && (maxkey >> bits) != 0) ++bits;
  return bits;
}

int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

// ------------------------------------------------------------- dispatch

int elem_size(int dtype) { return dtype == TSP_F64 ? 8 : (dtype == TSP_F32 ? 4 : 2); }

bool dtype_ok(int dtype) { return dtype == TSP_F32 || dtype == TSP_F64 || dtype == TSP_BF16; }

template <typename T>
int bsr_pattern_t(const void* A, int64_t lda, int64_t m, int64_t n, int64_t b, double threshold, uint8_t* keep,
                  int64_t* row_ptrs, int64_t* counts, hipStream_t st) {
  const int64_t mb = tsp::ceil_div(m, b), nbc = tsp::ceil_div(n, b);
  const auto thr = round_threshold<T>(threshold);
  const int64_t nblk = mb * nbc;
  if (nblk > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "bsr from_dense: too many blocks");
  if (nblk > 0) {
    const int V = 16 / (int)sizeof(T);
    if (vec_width<T>(A, lda) == V && b % V == 0)
      hipLaunchKernelGGL((bsr_keep_kernel<T, 16 / sizeof(T)>), dim3((unsigned)nblk), dim3(256), 0, st, (const T*)A,
                         lda, m, n, b, nbc, thr, keep);
    else
      hipLaunchKernelGGL((bsr_keep_kernel<T, 1>), dim3((unsigned)nblk), dim3(256), 0, st, (const T*)A, lda, m, n, b,
                         nbc, thr, keep);
    int rc = tsp::check_launch("bsr_keep launch");
    if (rc) return rc;
    hipLaunchKernelGGL(row_count_u8_kernel, dim3((unsigned)tsp::ceil_div(mb, 4)), dim3(256), 0, st, keep, mb, nbc,
                       counts);
    rc = tsp::check_launch("row_count launch");
    if (rc) return rc;
  }
  return scan_counts(counts, mb, row_ptrs, st);
}

template <typename T>
int bsr_fill_t(const void* A, int64_t lda, int64_t m, int64_t n, int64_t b, const uint8_t* keep,
               const int64_t* row_ptrs, int64_t n_blocks, int64_t* col_indices, void* blocks, hipStream_t st) {
  const int64_t mb = tsp::ceil_div(m, b), nbc = tsp::ceil_div(n, b);
  if (mb == 0 || n_blocks == 0) return TSP_OK;
  if (mb > INT32_MAX || n_blocks > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "bsr from_dense: too many blocks");
  hipLaunchKernelGGL(bsr_cols_kernel, dim3((unsigned)mb), dim3(256), 0, st, keep, nbc, row_ptrs, col_indices);
  int rc = tsp::check_launch("bsr_cols launch");
  if (rc) return rc;
  const int V = 16 / (int)sizeof(T);
  if (vec_width<T>(A, lda) == V && b % V == 0 && ((uintptr_t)blocks % 16) == 0)
    hipLaunchKernelGGL((bsr_gather_kernel<T, 16 / sizeof(T)>), dim3((unsigned)n_blocks), dim3(256), 0, st,
                       (const T*)A, lda, m, n, b, mb, row_ptrs, col_indices, (T*)blocks);
  else
    hipLaunchKernelGGL((bsr_gather_kernel<T, 1>), dim3((unsigned)n_blocks), dim3(256), 0, st, (const T*)A, lda, m,
                       n, b, mb, row_ptrs, col_indices, (T*)blocks);
  return tsp::check_launch("bsr_gather launch");
}

template <typename T>
int csr_pattern_t(const void* A, int64_t lda, int64_t m, int64_t n, double threshold, int64_t* row_ptrs,
                  int64_t* counts, hipStream_t st) {
  const auto thr = round_threshold<T>(threshold);
  if (m > 0) {
    const int64_t g = tsp::ceil_div(m, 4);
    if (g > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "csr from_dense: too many rows");
    if (vec_width<T>(A, lda) > 1)
      hipLaunchKernelGGL((csr_count_kernel<T, 16 / sizeof(T)>), dim3((unsigned)g), dim3(256), 0, st, (const T*)A, lda,
                         m, n, thr, counts);
    else
      hipLaunchKernelGGL((csr_count_kernel<T, 1>), dim3((unsigned)g), dim3(256), 0, st, (const T*)A, lda, m, n, thr,
                         counts);
    int rc = tsp::check_launch("csr_count launch");
    if (rc) return rc;
  }
  return scan_counts(counts, m, row_ptrs, st);
}

template <typename T>
int csr_fill_t(const void* A, int64_t lda, int64_t m, int64_t n, double threshold, const int64_t* row_ptrs,
               int64_t* col_indices, void* values, hipStream_t st) {
  const auto thr = round_threshold<T>(threshold);
  if (m == 0) return TSP_OK;
  const int64_t g = tsp::ceil_div(m, 4);
  if (g > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "csr from_dense: too many rows");
  if (vec_width<T>(A, lda) > 1)
    hipLaunchKernelGGL((csr_fill_kernel<T, 16 / sizeof(T)>), dim3((unsigned)g), dim3(256), 0, st, (const T*)A, lda, m,
                       n, thr, row_ptrs, col_indices, (T*)values);
  else
    hipLaunchKernelGGL((csr_fill_kernel<T, 1>), dim3((unsigned)g), dim3(256), 0, st, (const T*)A, lda, m, n, thr,
                       row_ptrs, col_indices, (T*)values);
  return tsp::check_launch("csr_fill launch");
}

}  // namespace

// Workspace of the from_dense pattern calls: block (or row) counts.
extern "C" int64_t tsp_format_workspace_size(int64_t rows) {
  if (rows < 0) return -1;
  return 8 * (rows + 1);
}

extern "C" int tsp_bsr_from_dense_pattern(const void* A, int dtype, int64_t lda, int64_t m, int64_t n,
                                          int64_t block_size, double threshold, uint8_t* keep, int64_t* row_ptrs,
                                          void* workspace, void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_from_dense_pattern: dtype %d", dtype);
  if (m < 0 || n < 0 || block_size <= 0 || lda < n) return tsp::fail(TSP_EINVAL, "tsp_bsr_from_dense_pattern: bad size");
  if (!row_ptrs || !workspace || (m > 0 && n > 0 && (!A || !keep)))
    return tsp::fail(TSP_EINVAL, "tsp_bsr_from_dense_pattern: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (n == 0) {  // no block columns: every block row is empty
    const int64_t mb = tsp::ceil_div(m, block_size);
    int rc = tsp::zero_fill(workspace, 8 * mb, st);
    if (rc) return rc;
    return scan_counts((const int64_t*)workspace, mb, row_ptrs, st);
  }
  if (dtype == TSP_F32)
    return bsr_pattern_t<float>(A, lda, m, n, block_size, threshold, keep, row_ptrs, (int64_t*)workspace, st);
  if (dtype == TSP_F64)
    return bsr_pattern_t<double>(A, lda, m, n, block_size, threshold, keep, row_ptrs, (int64_t*)workspace, st);
  return bsr_pattern_t<uint16_t>(A, lda, m, n, block_size, threshold, keep, row_ptrs, (int64_t*)workspace, st);
}

extern "C" int tsp_bsr_from_dense_fill(const void* A, int dtype, int64_t lda, int64_t m, int64_t n, int64_t block_size,
                                       const uint8_t* keep, const int64_t* row_ptrs, int64_t n_blocks,
                                       int64_t* col_indices, void* blocks, void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_from_dense_fill: dtype %d", dtype);
  if (m < 0 || n < 0 || block_size <= 0 || lda < n || n_blocks < 0)
    return tsp::fail(TSP_EINVAL, "tsp_bsr_from_dense_fill: bad size");
  if (n_blocks == 0) return TSP_OK;
  if (!A || !keep || !row_ptrs || !col_indices || !blocks) return tsp::fail(TSP_EINVAL, "tsp_bsr_from_dense_fill: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TSP_F32)
    return bsr_fill_t<float>(A, lda, m, n, block_size, keep, row_ptrs, n_blocks, col_indices, blocks, st);
  if (dtype == TSP_F64)
    return bsr_fill_t<double>(A, lda, m, n, block_size, keep, row_ptrs, n_blocks, col_indices, blocks, st);
  return bsr_fill_t<uint16_t>(A, lda, m, n, block_size, keep, row_ptrs, n_blocks, col_indices, blocks, st);
}

extern "C" int tsp_bsr_to_dense(const void* blocks, int dtype, const int64_t* row_ptrs, const int64_t* col_indices,
                                int64_t n_blocks, int64_t block_size, int64_t m, int64_t n, void* out, int64_t ldo,
                                void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_to_dense: dtype %d", dtype);
  if (m < 0 || n < 0 || block_size <= 0 || ldo < n || n_blocks < 0) return tsp::fail(TSP_EINVAL, "tsp_bsr_to_dense: bad size");
  if (m == 0 || n == 0) return TSP_OK;
  if (!row_ptrs || !out || (n_blocks > 0 && (!blocks || !col_indices)))
    return tsp::fail(TSP_EINVAL, "tsp_bsr_to_dense: null pointer");
  const int64_t mb = tsp::ceil_div(m, block_size), nbc = tsp::ceil_div(n, block_size);
  if (mb * nbc > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_to_dense: too many blocks");
  hipStream_t st = (hipStream_t)stream;
  const dim3 g((unsigned)(mb * nbc));
  if (dtype == TSP_F32)
    hipLaunchKernelGGL(bsr_to_dense_kernel<float>, g, dim3(256), 0, st, (const float*)blocks, row_ptrs, col_indices,
                       block_size, nbc, m, n, (float*)out, ldo);
  else if (dtype == TSP_F64)
    hipLaunchKernelGGL(bsr_to_dense_kernel<double>, g, dim3(256), 0, st, (const double*)blocks, row_ptrs, col_indices,
                       block_size, nbc, m, n, (double*)out, ldo);
  else
    hipLaunchKernelGGL(bsr_to_dense_kernel<uint16_t>, g, dim3(256), 0, st, (const uint16_t*)blocks, row_ptrs,
                       col_indices, block_size, nbc, m, n, (uint16_t*)out, ldo);
  return tsp::check_launch("bsr_to_dense launch");
}

extern "C" int tsp_csr_from_dense_pattern(const void* A, int dtype, int64_t lda, int64_t m, int64_t n, double threshold,
                                          int64_t* row_ptrs, void* workspace, void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_from_dense_pattern: dtype %d", dtype);
  if (m < 0 || n < 0 || lda < n) return tsp::fail(TSP_EINVAL, "tsp_csr_from_dense_pattern: bad size");
  if (!row_ptrs || !workspace || (m > 0 && n > 0 && !A)) return tsp::fail(TSP_EINVAL, "tsp_csr_from_dense_pattern: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (n == 0) {
    int rc = tsp::zero_fill(workspace, 8 * m, st);
    if (rc) return rc;
    return scan_counts((const int64_t*)workspace, m, row_ptrs, st);
  }
  if (dtype == TSP_F32) return csr_pattern_t<float>(A, lda, m, n, threshold, row_ptrs, (int64_t*)workspace, st);
  if (dtype == TSP_F64) return csr_pattern_t<double>(A, lda, m, n, threshold, row_ptrs, (int64_t*)workspace, st);
  return csr_pattern_t<uint16_t>(A, lda, m, n, threshold, row_ptrs, (int64_t*)workspace, st);
}

extern "C" int tsp_csr_from_dense_fill(const void* A, int dtype, int64_t lda, int64_t m, int64_t n, double threshold,
                                       const int64_t* row_ptrs, int64_t* col_indices, void* values, void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_from_dense_fill: dtype %d", dtype);
  if (m < 0 || n < 0 || lda < n) return tsp::fail(TSP_EINVAL, "tsp_csr_from_dense_fill: bad size");
  if (m == 0 || n == 0) return TSP_OK;
  // col_indices / values may be null when no entry passes (nothing is written)
  if (!A || !row_ptrs) return tsp::fail(TSP_EINVAL, "tsp_csr_from_dense_fill: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TSP_F32) return csr_fill_t<float>(A, lda, m, n, threshold, row_ptrs, col_indices, values, st);
  if (dtype == TSP_F64) return csr_fill_t<double>(A, lda, m, n, threshold, row_ptrs, col_indices, values, st);
  return csr_fill_t<uint16_t>(A, lda, m, n, threshold, row_ptrs, col_indices, values, st);
}

extern "C" int tsp_csr_to_dense(const void* values, int dtype, const int64_t* col_indices, const int64_t* row_ptrs,
                                int64_t m, int64_t n, void* out, int64_t ldo, void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_to_dense: dtype %d", dtype);
  if (m < 0 || n < 0 || ldo < n) return tsp::fail(TSP_EINVAL, "tsp_csr_to_dense: bad size");
  if (m == 0 || n == 0) return TSP_OK;
  if (!row_ptrs || !out) return tsp::fail(TSP_EINVAL, "tsp_csr_to_dense: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (ldo == n) {
    int rc = tsp::zero_fill(out, m * n * elem_size(dtype), st);
    if (rc) return rc;
  } else {
    const int64_t gz = tsp::ceil_div(m * n, 256) < 65536 ? tsp::ceil_div(m * n, 256) : 65536;
    if (dtype == TSP_F32)
      hipLaunchKernelGGL(zero_rows_kernel<float>, dim3((unsigned)gz), dim3(256), 0, st, (float*)out, m, n, ldo);
    else if (dtype == TSP_F64)
      hipLaunchKernelGGL(zero_rows_kernel<double>, dim3((unsigned)gz), dim3(256), 0, st, (double*)out, m, n, ldo);
    else
      hipLaunchKernelGGL(zero_rows_kernel<uint16_t>, dim3((unsigned)gz), dim3(256), 0, st, (uint16_t*)out, m, n, ldo);
    int rc = tsp::check_launch("zero_rows launch");
    if (rc) return rc;
  }
  const int64_t g = tsp::ceil_div(m, 256);
  if (g > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_to_dense: too many rows");
  if (dtype == TSP_F32)
    hipLaunchKernelGGL(csr_to_dense_kernel<float>, dim3((unsigned)g), dim3(256), 0, st, (const float*)values,
                       col_indices, row_ptrs, m, (float*)out, ldo);
  else if (dtype == TSP_F64)
    hipLaunchKernelGGL(csr_to_dense_kernel<double>, dim3((unsigned)g), dim3(256), 0, st, (const double*)values,
                       col_indices, row_ptrs, m, (double*)out, ldo);
  else
    hipLaunchKernelGGL(csr_to_dense_kernel<uint16_t>, dim3((unsigned)g), dim3(256), 0, st, (const uint16_t*)values,
                       col_indices, row_ptrs, m, (uint16_t*)out, ldo);
  return tsp::check_launch("csr_to_dense launch");
}

extern "C" int tsp_csr_row_indices(const int64_t* row_ptrs, int64_t m, int64_t nnz, int64_t* rows, void* stream) {
  if (m < 0 || nnz < 0 || (m == 0 && nnz > 0)) return tsp::fail(TSP_EINVAL, "tsp_csr_row_indices: bad size");
  if (nnz == 0) return TSP_OK;
  if (!row_ptrs || !rows) return tsp::fail(TSP_EINVAL, "tsp_csr_row_indices: null pointer");
  return launch_entry_rows(row_ptrs, m, nnz, RowsOut{rows}, (hipStream_t)stream, "tsp_csr_row_indices");
}

namespace {

// Stable radix sort of (key, value) pairs with the value type of `dtype`:
// the values move with their keys, so no permutation has to be gathered
// afterwards. tmp == nullptr queries the temporary size.
template <typename K, typename V>
hipError_t sort_pairs(void* tmp, size_t& tmp_bytes, const K* kin, K* kout, const V* vin, V* vout, int64_t nnz,
                      int bits, hipStream_t st) {
  return tsp::rsort::radix_sort_pairs(tmp, tmp_bytes, kin, kout, vin, vout, nnz, 0, bits, st);
}

template <typename K, typename F>
hipError_t sort_pairs_dtype(int dtype, void* tmp, size_t& tmp_bytes, const K* kin, K* kout, const void* vin,
                            void* vout, int64_t nnz, int bits, hipStream_t st) {
  if (dtype == TSP_F32)
    return sort_pairs(tmp, tmp_bytes, kin, kout, (const F*)vin, (F*)vout, nnz, bits, st);
  if (dtype == TSP_F64)
    return sort_pairs(tmp, tmp_bytes, kin, kout, (const double*)vin, (double*)vout, nnz, bits, st);
  return sort_pairs(tmp, tmp_bytes, kin, kout, (const uint16_t*)vin, (uint16_t*)vout, nnz, bits, st);
}

template <typename K = uint64_t>
int64_t coo_sort_tmp(int dtype, int64_t nnz, int bits) {
  size_t tmp = 0;
  if (nnz > 0 && sort_pairs_dtype<K, float>(dtype, nullptr, tmp, (const K*)nullptr, (K*)nullptr, nullptr, nullptr, nnz,
                                            bits, 0) != hipSuccess)
    return -1;
  return (int64_t)tmp;
}

// keys fit in 32 bits: every key and the bound m * n are <= UINT32_MAX
bool narrow_keys(int64_t m, int64_t n) { return m == 0 || n <= (int64_t)UINT32_MAX / m; }

template <typename K>
int coo_to_csr_keys(const void* values, int dtype, const int64_t* row_indices, const int64_t* col_indices, int64_t nnz,
                    int64_t m, int64_t n, int64_t* row_ptrs, int64_t* col_out, void* values_out, char* w,
                    int64_t workspace_bytes, hipStream_t st) {
  const int64_t g = tsp::ceil_div(nnz, 256);
  K* keys = (K*)w;
  K* keys_s = (K*)(w + align256(8 * nnz));
  void* tmp = w + 2 * align256(8 * nnz);
  size_t tmp_bytes = (size_t)(workspace_bytes - 2 * align256(8 * nnz));
  hipLaunchKernelGGL(coo_keys_kernel<K>, dim3((unsigned)g), dim3(256), 0, st, row_indices, col_indices, nnz, n, keys);
  int rc = tsp::check_launch("coo_keys launch");
  if (rc) return rc;
  const hipError_t se =
      sort_pairs_dtype<K, float>(dtype, tmp, tmp_bytes, keys, keys_s, values, values_out, nnz, key_bits(m, n), st);
  if (se != hipSuccess) return tsp::check_hip(se, "radix_sort_pairs");
  rc = tsp::check_launch("radix_sort_pairs");
  if (rc) return rc;
  hipLaunchKernelGGL(key_cols_kernel<K>, dim3((unsigned)g), dim3(256), 0, st, keys_s, nnz, n, col_out);
  rc = tsp::check_launch("key_cols launch");
  if (rc) return rc;
  hipLaunchKernelGGL(coo_row_ptrs_kernel<K>, dim3((unsigned)tsp::ceil_div(m + 1, 256)), dim3(256), 0, st, keys_s, nnz,
                     m, n, row_ptrs);
  return tsp::check_launch("coo_row_ptrs launch");
}

}  // namespace

extern "C" int64_t tsp_coo_to_csr_workspace_size(int64_t nnz, int64_t m, int64_t n) {
  if (nnz < 0 || m < 0 || n < 0) return -1;
  if (nnz > UINT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_to_csr: more than 2^32 - 1 entries"), -1;
  // sized for the widest value type (fp64), which also covers fp32 / bf16;
  // the two key arrays get 8 bytes an entry whichever key width runs
  const int bits = nnz > 0 ? key_bits(m, n) : 1;
  const int64_t tmp = narrow_keys(m, n) ? coo_sort_tmp<uint32_t>(TSP_F64, nnz, bits) : coo_sort_tmp(TSP_F64, nnz, bits);
  if (tmp < 0) return -1;
  return 2 * align256(8 * nnz) + align256(tmp);
}

extern "C" int tsp_coo_to_csr(const void* values, int dtype, const int64_t* row_indices, const int64_t* col_indices,
                              int64_t nnz, int64_t m, int64_t n, int64_t* row_ptrs, int64_t* col_out, void* values_out,
                              void* workspace, int64_t workspace_bytes, void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_to_csr: dtype %d", dtype);
  if (nnz < 0 || m < 0 || n < 0) return tsp::fail(TSP_EINVAL, "tsp_coo_to_csr: bad size");
  if (nnz > UINT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_to_csr: more than 2^32 - 1 entries");
  if (m > 0 && n > 0 && m > INT64_MAX / n) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_to_csr: m * n overflows");
  if (!row_ptrs) return tsp::fail(TSP_EINVAL, "tsp_coo_to_csr: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (nnz == 0) {
    int rc = tsp::zero_fill(row_ptrs, 8 * (m + 1), st);
    return rc;
  }
  if (!values || !row_indices || !col_indices || !col_out || !values_out || !workspace)
    return tsp::fail(TSP_EINVAL, "tsp_coo_to_csr: null pointer");
  if (workspace_bytes < tsp_coo_to_csr_workspace_size(nnz, m, n))
    return tsp::fail(TSP_EINVAL, "tsp_coo_to_csr: workspace too small");
  const int64_t g = tsp::ceil_div(nnz, 256);
  if (g > INT32_MAX || tsp::ceil_div(m + 1, 256) > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_to_csr: too large");
  if (narrow_keys(m, n))
    return coo_to_csr_keys<uint32_t>(values, dtype, row_indices, col_indices, nnz, m, n, row_ptrs, col_out, values_out,
                                     (char*)workspace, workspace_bytes, st);
  return coo_to_csr_keys<uint64_t>(values, dtype, row_indices, col_indices, nnz, m, n, row_ptrs, col_out, values_out,
                                   (char*)workspace, workspace_bytes, st);
}

extern "C" int64_t tsp_coo_sum_to_csr_workspace_size(int64_t nnz, int64_t m, int64_t n) {
  if (nnz < 0 || m < 0 || n < 0) return -1;
  if (nnz > UINT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_sum_to_csr: more than 2^32 - 1 entries"), -1;
  const int64_t sort_b = coo_sort_tmp(TSP_F64, nnz, nnz > 0 ? key_bits(m, n) : 1);
  if (sort_b < 0) return -1;
  size_t scan_b = 0;
  if (nnz > 0 && tsp::rsort::inclusive_scan<int64_t>(nullptr, scan_b, nullptr, nullptr, nnz) != hipSuccess) return -1;
  const int64_t tmp = sort_b > (int64_t)scan_b ? sort_b : (int64_t)scan_b;
  return 6 * align256(8 * nnz) + align256(tmp);
}

extern "C" int tsp_coo_sum_to_csr(const void* values, int dtype, const int64_t* row_indices,
                                  const int64_t* col_indices, int64_t nnz, int64_t m, int64_t n, int64_t* row_ptrs,
                                  int64_t* col_out, void* values_out, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_sum_to_csr: dtype %d", dtype);
  if (nnz < 0 || m < 0 || n < 0) return tsp::fail(TSP_EINVAL, "tsp_coo_sum_to_csr: bad size");
  if (nnz > UINT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_sum_to_csr: more than 2^32 - 1 entries");
  if (m > 0 && n > 0 && m > INT64_MAX / n) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_sum_to_csr: m * n overflows");
  if (!row_ptrs) return tsp::fail(TSP_EINVAL, "tsp_coo_sum_to_csr: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (nnz == 0) return tsp::zero_fill(row_ptrs, 8 * (m + 1), st);
  if (!values || !row_indices || !col_indices || !col_out || !values_out || !workspace)
    return tsp::fail(TSP_EINVAL, "tsp_coo_sum_to_csr: null pointer");
  if (workspace_bytes < tsp_coo_sum_to_csr_workspace_size(nnz, m, n))
    return tsp::fail(TSP_EINVAL, "tsp_coo_sum_to_csr: workspace too small");
  const int64_t g = tsp::ceil_div(nnz, 256);
  if (g > INT32_MAX || tsp::ceil_div(m + 1, 256) > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_coo_sum_to_csr: too large");
  char* w = (char*)workspace;
  const int64_t a = align256(8 * nnz);
  uint64_t* keys = (uint64_t*)w;
  uint64_t* keys_s = (uint64_t*)(w + a);
  void* vals_s = w + 2 * a;  // values sorted with their keys (at most 8 bytes each)
  int64_t* head = (int64_t*)(w + 3 * a);
  int64_t* seg = (int64_t*)(w + 4 * a);
  uint64_t* ukeys = (uint64_t*)(w + 5 * a);
  void* tmp = w + 6 * a;
  size_t tmp_bytes = (size_t)(workspace_bytes - 6 * a);
  hipLaunchKernelGGL(coo_keys_kernel<uint64_t>, dim3((unsigned)g), dim3(256), 0, st, row_indices, col_indices, nnz, n, keys);
  int rc = tsp::check_launch("coo_keys launch");
  if (rc) return rc;
  const hipError_t sse =
      sort_pairs_dtype<uint64_t, float>(dtype, tmp, tmp_bytes, keys, keys_s, values, vals_s, nnz, key_bits(m, n), st);
  if (sse != hipSuccess) return tsp::check_hip(sse, "radix_sort_pairs");
  hipLaunchKernelGGL(run_heads_kernel, dim3((unsigned)g), dim3(256), 0, st, keys_s, nnz, head);
  rc = tsp::check_launch("run_heads launch");
  if (rc) return rc;
  tmp_bytes = (size_t)(workspace_bytes - 6 * a);
  hipError_t se = tsp::rsort::inclusive_scan(tmp, tmp_bytes, (const int64_t*)head, seg, nnz, st);
  if (se != hipSuccess) return tsp::check_hip(se, "inclusive_scan");
  if (dtype == TSP_F32)
    hipLaunchKernelGGL(run_sum_kernel<float>, dim3((unsigned)g), dim3(256), 0, st, keys_s, seg, head,
                       (const float*)vals_s, nnz, n, ukeys, col_out, (float*)values_out);
  else if (dtype == TSP_F64)
    hipLaunchKernelGGL(run_sum_kernel<double>, dim3((unsigned)g), dim3(256), 0, st, keys_s, seg, head,
                       (const double*)vals_s, nnz, n, ukeys, col_out, (double*)values_out);
  else
    hipLaunchKernelGGL(run_sum_kernel<uint16_t>, dim3((unsigned)g), dim3(256), 0, st, keys_s, seg, head,
                       (const uint16_t*)vals_s, nnz, n, ukeys, col_out, (uint16_t*)values_out);
  rc = tsp::check_launch("run_sum launch");
  if (rc) return rc;
  hipLaunchKernelGGL(run_row_ptrs_kernel<false>, dim3((unsigned)tsp::ceil_div(m + 1, 256)), dim3(256), 0, st, ukeys, seg, nnz,
                     m, n, row_ptrs);
  return tsp::check_launch("run_row_ptrs launch");
}

namespace {

template <typename T>
int64_t tr_sort_tmp(int64_t nnz, int bits) {
  size_t tmp = 0;
  if (nnz > 0 && sort_pairs(nullptr, tmp, (const uint32_t*)nullptr, (uint32_t*)nullptr, (const RowVal<T>*)nullptr,
                            (RowVal<T>*)nullptr, nnz, bits, 0) != hipSuccess)
    return -1;
  return (int64_t)tmp;
}

int col_bits(int64_t n) {  // bits of the largest column index n - 1
  int bits = 1;
  while (bits < 32 && ((uint64_t)(n > 0 ? n - 1 : 0) >> bits) != 0) ++bits;
  return bits;
}

template <typename T>
int csr_transpose_t(const T* values, const int64_t* col_indices, const int64_t* row_ptrs, int64_t m, int64_t n,
                    int64_t nnz, int64_t* out_row_ptrs, int64_t* out_col, T* out_values, char* w,
                    int64_t workspace_bytes, hipStream_t st) {
  const int64_t ka = align256(4 * nnz), pa = align256((int64_t)sizeof(RowVal<T>) * nnz);
  uint32_t* keys = (uint32_t*)w;
  uint32_t* keys_s = (uint32_t*)(w + ka);
  RowVal<T>* pay = (RowVal<T>*)(w + 2 * ka);
  RowVal<T>* pay_s = (RowVal<T>*)(w + 2 * ka + pa);
  void* tmp = w + 2 * ka + 2 * pa;
  size_t tmp_bytes = (size_t)(workspace_bytes - (2 * ka + 2 * pa));
  int rc = launch_entry_rows(row_ptrs, m, nnz, TrKeys<T>{col_indices, values, keys, pay}, st, "tr_keys launch");
  if (rc) return rc;
  // (pay_s: scratch between passes; the last pass writes out_col / out_values)
  const hipError_t se = tsp::rsort::radix_sort_pairs_to(tmp, tmp_bytes, (const uint32_t*)keys, keys_s,
                                                        (const RowVal<T>*)pay, pay_s, nnz, 0, col_bits(n),
                                                        TrOut<T>{out_col, out_values}, st);
  if (se != hipSuccess) return tsp::check_hip(se, "radix_sort_pairs");
  hipLaunchKernelGGL(tr_row_ptrs_kernel, dim3((unsigned)tsp::ceil_div(n + 1, 256)), dim3(256), 0, st,
                     (const uint32_t*)keys_s, nnz, n, out_row_ptrs);
  return tsp::check_launch("tr_row_ptrs launch");
}

}  // namespace

extern "C" int64_t tsp_csr_transpose_workspace_size(int64_t nnz, int64_t m, int64_t n, int dtype) {
  if (nnz < 0 || m < 0 || n < 0 || !dtype_ok(dtype)) return -1;
  if (nnz > UINT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_transpose: more than 2^32 - 1 entries"), -1;
  const int bits = col_bits(n);
  int64_t tmp, pay;
  if (dtype == TSP_F32) {
    tmp = tr_sort_tmp<float>(nnz, bits);
    pay = (int64_t)sizeof(RowVal<float>);
  } else if (dtype == TSP_F64) {
    tmp = tr_sort_tmp<double>(nnz, bits);
    pay = (int64_t)sizeof(RowVal<double>);
  } else {
    tmp = tr_sort_tmp<uint16_t>(nnz, bits);
    pay = (int64_t)sizeof(RowVal<uint16_t>);
  }
  if (tmp < 0) return -1;
  return 2 * align256(4 * nnz) + 2 * align256(pay * nnz) + align256(tmp);
}

extern "C" int tsp_csr_transpose(const void* values, int dtype, const int64_t* col_indices, const int64_t* row_ptrs,
                                 int64_t m, int64_t n, int64_t nnz, int64_t* out_row_ptrs, int64_t* out_col,
                                 void* out_values, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_transpose: dtype %d", dtype);
  if (nnz < 0 || m < 0 || n < 0 || (m == 0 && nnz > 0)) return tsp::fail(TSP_EINVAL, "tsp_csr_transpose: bad size");
  if (m > UINT32_MAX || n > (int64_t)UINT32_MAX + 1 || nnz > UINT32_MAX)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_transpose: dimensions or entries past 2^32");
  if (!out_row_ptrs) return tsp::fail(TSP_EINVAL, "tsp_csr_transpose: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (nnz == 0) return tsp::zero_fill(out_row_ptrs, 8 * (n + 1), st);
  if (!values || !col_indices || !row_ptrs || !out_col || !out_values || !workspace)
    return tsp::fail(TSP_EINVAL, "tsp_csr_transpose: null pointer");
  if (workspace_bytes < tsp_csr_transpose_workspace_size(nnz, m, n, dtype))
    return tsp::fail(TSP_EINVAL, "tsp_csr_transpose: workspace too small");
  if (tsp::ceil_div(nnz, 256) > INT32_MAX || tsp::ceil_div(n + 1, 256) > INT32_MAX)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_transpose: too large");
  char* w = (char*)workspace;
  if (dtype == TSP_F32)
    return csr_transpose_t((const float*)values, col_indices, row_ptrs, m, n, nnz, out_row_ptrs, out_col,
                           (float*)out_values, w, workspace_bytes, st);
  if (dtype == TSP_F64)
    return csr_transpose_t((const double*)values, col_indices, row_ptrs, m, n, nnz, out_row_ptrs, out_col,
                           (double*)out_values, w, workspace_bytes, st);
  return csr_transpose_t((const uint16_t*)values, col_indices, row_ptrs, m, n, nnz, out_row_ptrs, out_col,
                         (uint16_t*)out_values, w, workspace_bytes, st);
}

// ------------------------------------------------ BSR block-column view

namespace {

// entry k (block k of block row r): sort key = its block column; payload = (r, k)
struct BlkKeys {
  const int64_t* cols;
  uint32_t* keys;
  RowVal<uint32_t>* payload;
  int64_t* block_rows;
  __device__ void operator()(int64_t k, int64_t r) const {
    keys[k] = (uint32_t)cols[k];
    payload[k] = RowVal<uint32_t>{(uint32_t)r, (uint32_t)k};
    block_rows[k] = r;
  }
};

__global__ __launch_bounds__(256) void blk_unpack_kernel(const RowVal<uint32_t>* __restrict__ payload, int64_t nnzb,
                                                         int64_t* __restrict__ col_block_rows,
                                                         int64_t* __restrict__ col_block_ids) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= nnzb) return;
  const RowVal<uint32_t> p = payload[k];
  col_block_rows[k] = (int64_t)p.row;
  col_block_ids[k] = (int64_t)p.val;
}

}  // namespace

extern "C" int64_t tsp_bsr_col_view_workspace_size(int64_t nnzb, int64_t n_block_cols) {
  if (nnzb < 0 || n_block_cols < 0) return -1;
  if (nnzb > UINT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_col_view: more than 2^32 - 1 blocks"), -1;
  size_t tmp = 0;
  if (nnzb > 0 && tsp::rsort::radix_sort_pairs(nullptr, tmp, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                               (const RowVal<uint32_t>*)nullptr, (RowVal<uint32_t>*)nullptr, nnzb, 0,
                                               col_bits(n_block_cols)) != hipSuccess)
    return -1;
  return 2 * align256(4 * nnzb) + 2 * align256(8 * nnzb) + align256((int64_t)tmp);
}

extern "C" int tsp_bsr_col_view(const int64_t* block_row_ptrs, const int64_t* block_col_indices, int64_t n_block_rows,
                                int64_t n_block_cols, int64_t nnzb, int64_t* block_rows, int64_t* col_ptrs,
                                int64_t* col_block_ids, int64_t* col_block_rows, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  if (nnzb < 0 || n_block_rows < 0 || n_block_cols < 0 || (n_block_rows == 0 && nnzb > 0))
    return tsp::fail(TSP_EINVAL, "tsp_bsr_col_view: bad size");
  if (nnzb > UINT32_MAX || n_block_rows > UINT32_MAX || n_block_cols > (int64_t)UINT32_MAX + 1)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_col_view: sizes past 2^32");
  if (!col_ptrs) return tsp::fail(TSP_EINVAL, "tsp_bsr_col_view: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (nnzb == 0) return tsp::zero_fill(col_ptrs, 8 * (n_block_cols + 1), st);
  if (!block_row_ptrs || !block_col_indices || !block_rows || !col_block_ids || !col_block_rows || !workspace)
    return tsp::fail(TSP_EINVAL, "tsp_bsr_col_view: null pointer");
  if (workspace_bytes < tsp_bsr_col_view_workspace_size(nnzb, n_block_cols))
    return tsp::fail(TSP_EINVAL, "tsp_bsr_col_view: workspace too small");
  if (tsp::ceil_div(n_block_cols + 1, 256) > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_col_view: too large");
  char* w = (char*)workspace;
  const int64_t ka = align256(4 * nnzb), pa = align256(8 * nnzb);
  uint32_t* keys = (uint32_t*)w;
  uint32_t* keys_s = (uint32_t*)(w + ka);
  RowVal<uint32_t>* pay = (RowVal<uint32_t>*)(w + 2 * ka);
  RowVal<uint32_t>* pay_s = (RowVal<uint32_t>*)(w + 2 * ka + pa);
  void* tmp = w + 2 * ka + 2 * pa;
  size_t tmp_bytes = (size_t)(workspace_bytes - (2 * ka + 2 * pa));
  int rc = launch_entry_rows(block_row_ptrs, n_block_rows, nnzb, BlkKeys{block_col_indices, keys, pay, block_rows}, st,
                             "bsr_col_view keys launch");
  if (rc) return rc;
  // stable: within a block column, blocks keep their CSR order, i.e. increasing block row
  const hipError_t se = tsp::rsort::radix_sort_pairs(tmp, tmp_bytes, (const uint32_t*)keys, keys_s,
                                                     (const RowVal<uint32_t>*)pay, pay_s, nnzb, 0,
                                                     col_bits(n_block_cols), st);
  if (se != hipSuccess) return tsp::check_hip(se, "radix_sort_pairs");
  hipLaunchKernelGGL(blk_unpack_kernel, dim3((unsigned)tsp::ceil_div(nnzb, 256)), dim3(256), 0, st,
                     (const RowVal<uint32_t>*)pay_s, nnzb, col_block_rows, col_block_ids);
  rc = tsp::check_launch("bsr_col_view unpack launch");
  if (rc) return rc;
  hipLaunchKernelGGL(tr_row_ptrs_kernel, dim3((unsigned)tsp::ceil_div(n_block_cols + 1, 256)), dim3(256), 0, st,
                     (const uint32_t*)keys_s, nnzb, n_block_cols, col_ptrs);
  return tsp::check_launch("bsr_col_view col_ptrs launch");
}

namespace {

int64_t sum_scan_tmp(int64_t m) {
  size_t b = 0;
  if (tsp::rsort::exclusive_scan<int64_t>(nullptr, b, nullptr, nullptr, 0, m + 1) != hipSuccess) return -1;
  return (int64_t)b;
}

template <typename T>
int csr_sum_t(const T* av, const int64_t* ac, const int64_t* ar, const T* bv, const int64_t* bc, const int64_t* br,
              int64_t N, int64_t m, int64_t n, int64_t* row_ptrs, int64_t* col_out, T* values_out, char* w,
              int64_t workspace_bytes, hipStream_t st) {
  int64_t* ucount = (int64_t*)w;
  uint8_t* hflag = (uint8_t*)(w + align256(8 * (m + 1)));
  void* tmp = w + align256(8 * (m + 1)) + align256(N);
  size_t tb = (size_t)(workspace_bytes - align256(8 * (m + 1)) - align256(N));
  const int64_t chunks = tsp::ceil_div(m, SUM_RPW);
  const unsigned g = (unsigned)(chunks < 65536 ? chunks : 65536);
  const unsigned gl = (unsigned)(m < 1024 ? m : 1024);
  // csr_sum_wave: a wavefront per SUM_CHUNK rows
  const int64_t gw64 = tsp::ceil_div(m, 4 * SUM_CHUNK);
  if (gw64 > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_sum: too many rows");
  const unsigned gw = (unsigned)gw64;
  const bool key32 = col_bits(n) <= 26;
  if (key32)
    hipLaunchKernelGGL((csr_sum_wave_kernel<T, false, uint32_t>), dim3(gw), dim3(256), 0, st, av, ac, ar, bv, bc, br,
                       m, ucount, (const int64_t*)nullptr, (int64_t*)nullptr, (T*)nullptr);
  else
    hipLaunchKernelGGL((csr_sum_wave_kernel<T, false, uint64_t>), dim3(gw), dim3(256), 0, st, av, ac, ar, bv, bc, br,
                       m, ucount, (const int64_t*)nullptr, (int64_t*)nullptr, (T*)nullptr);
  int rc0 = tsp::check_launch("csr_sum_wave (count) launch");
  if (rc0) return rc0;
  hipLaunchKernelGGL((csr_sum_rows_kernel<T, false>), dim3(g), dim3(256), 0, st, av, ac, ar, bv, bc, br, m, ucount,
                     (const int64_t*)nullptr, (int64_t*)nullptr, (T*)nullptr);
  int rc = tsp::check_launch("csr_sum_rows (count) launch");
  if (rc) return rc;
  hipLaunchKernelGGL((csr_sum_long_kernel<T, false>), dim3(gl), dim3(256), 0, st, av, ac, ar, bv, bc, br, m, hflag,
                     ucount, (const int64_t*)nullptr, (int64_t*)nullptr, (T*)nullptr);
  rc = tsp::check_launch("csr_sum_long (count) launch");
  if (rc) return rc;
  hipError_t se = tsp::rsort::exclusive_scan(tmp, tb, (const int64_t*)ucount, row_ptrs, (int64_t)0, m + 1, st);
  if (se != hipSuccess) return tsp::check_hip(se, "exclusive_scan");
  if (key32)
    hipLaunchKernelGGL((csr_sum_wave_kernel<T, true, uint32_t>), dim3(gw), dim3(256), 0, st, av, ac, ar, bv, bc, br, m,
                       (int64_t*)nullptr, (const int64_t*)row_ptrs, col_out, values_out);
  else
    hipLaunchKernelGGL((csr_sum_wave_kernel<T, true, uint64_t>), dim3(gw), dim3(256), 0, st, av, ac, ar, bv, bc, br, m,
                       (int64_t*)nullptr, (const int64_t*)row_ptrs, col_out, values_out);
  rc = tsp::check_launch("csr_sum_wave (write) launch");
  if (rc) return rc;
  hipLaunchKernelGGL((csr_sum_rows_kernel<T, true>), dim3(g), dim3(256), 0, st, av, ac, ar, bv, bc, br, m,
                     (int64_t*)nullptr, (const int64_t*)row_ptrs, col_out, values_out);
  rc = tsp::check_launch("csr_sum_rows (write) launch");
  if (rc) return rc;
  hipLaunchKernelGGL((csr_sum_long_kernel<T, true>), dim3(gl), dim3(256), 0, st, av, ac, ar, bv, bc, br, m, hflag,
                     (int64_t*)nullptr, (const int64_t*)row_ptrs, col_out, values_out);
  return tsp::check_launch("csr_sum_long (write) launch");
}

}  // namespace

extern "C" int64_t tsp_csr_sum_workspace_size(int64_t nnz_a, int64_t nnz_b, int64_t m, int64_t n, int dtype) {
  if (nnz_a < 0 || nnz_b < 0 || m < 0 || n < 0 || !dtype_ok(dtype)) return -1;
  const int64_t tmp = sum_scan_tmp(m);
  if (tmp < 0) return -1;
  return align256(8 * (m + 1)) + align256(nnz_a + nnz_b) + align256(tmp);
}

extern "C" int tsp_csr_sum(const void* a_values, const int64_t* a_cols, const int64_t* a_row_ptrs, int64_t nnz_a,
                           const void* b_values, const int64_t* b_cols, const int64_t* b_row_ptrs, int64_t nnz_b,
                           int dtype, int64_t m, int64_t n, int64_t* row_ptrs, int64_t* col_out, void* values_out,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  if (!dtype_ok(dtype)) return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_sum: dtype %d", dtype);
  if (nnz_a < 0 || nnz_b < 0 || m < 0 || n < 0 || (m == 0 && nnz_a + nnz_b > 0))
    return tsp::fail(TSP_EINVAL, "tsp_csr_sum: bad size");
  if (m > UINT32_MAX || n > (int64_t)UINT32_MAX + 1 || nnz_a + nnz_b > UINT32_MAX)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_csr_sum: sizes past 2^32");
  if (!row_ptrs) return tsp::fail(TSP_EINVAL, "tsp_csr_sum: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (nnz_a + nnz_b == 0) return tsp::zero_fill(row_ptrs, 8 * (m + 1), st);
  if (!a_row_ptrs || !b_row_ptrs || !col_out || !values_out || !workspace ||
      (nnz_a > 0 && (!a_values || !a_cols)) || (nnz_b > 0 && (!b_values || !b_cols)))
    return tsp::fail(TSP_EINVAL, "tsp_csr_sum: null pointer");
  if (workspace_bytes < tsp_csr_sum_workspace_size(nnz_a, nnz_b, m, n, dtype))
    return tsp::fail(TSP_EINVAL, "tsp_csr_sum: workspace too small");
  char* w = (char*)workspace;
  if (dtype == TSP_F32)
    return csr_sum_t((const float*)a_values, a_cols, a_row_ptrs, (const float*)b_values, b_cols, b_row_ptrs, nnz_a + nnz_b, m, n,
                     row_ptrs, col_out, (float*)values_out, w, workspace_bytes, st);
  if (dtype == TSP_F64)
    return csr_sum_t((const double*)a_values, a_cols, a_row_ptrs, (const double*)b_values, b_cols, b_row_ptrs, nnz_a + nnz_b, m, n,
                     row_ptrs, col_out, (double*)values_out, w, workspace_bytes, st);
  return csr_sum_t((const uint16_t*)a_values, a_cols, a_row_ptrs, (const uint16_t*)b_values, b_cols, b_row_ptrs, nnz_a + nnz_b, m, n,
                   row_ptrs, col_out, (uint16_t*)values_out, w, workspace_bytes, st);
}
