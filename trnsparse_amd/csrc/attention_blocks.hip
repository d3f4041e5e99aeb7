// Block-sparse attention as block-sparse products, gfx950: the softmax over
// block scores and the per-block softmax gradient.
//
// The one-pass attention kernels (attention.hip, attention_bwd.hip) hold a
// query block's scores, weights and output rows in registers, which caps
// the head_dim they serve. For larger head_dims the same semantics
// (reference trnsparse/ops.py:280-473) run as block-sparse products over the
// mask stacked over heads (stacked block row h * Mt + i holds mask block row
// i shifted by h * Mt block columns; Q, K, V, O, dO are its (heads * seq,
// head_dim) operands):
//   forward   S  = Q K^T on the pattern (tsp_bsr_sddmm_ex, fp32 blocks)
//             P, row stats  (tsp_bsa_block_softmax, below)
//             O  = P V      (tsp_bsr_spmm)
//   backward  S  = Q K^T, dP = dO V^T (tsp_bsr_sddmm_ex)
//             Drow = rowsum(dO * O)    (tsp_bsa_rowdot, below)
//             P, dS = scale P (dP - Drow) (tsp_bsa_block_grad, below)
//             dV = P^T dO, dK = dS^T Q (tsp_bsr_spmm_t), dQ = dS K (tsp_bsr_spmm)
// Every product runs on the MFMA kernels of the BSR path and is exact in its
// order; the kernels here are elementwise passes over the fp32 blocks.
#include "common.h"

namespace {

constexpr int BS = 128;       // block size of the stacked pattern
constexpr int BB = BS * BS;   // entries per block

__device__ inline void put(float* p, float v) { *p = v; }
__device__ inline void put(uint16_t* p, float v) { *p = tsp::f32_to_bf16_bits(v); }

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// One 256-thread workgroup per stacked block row; wavefront w takes rows w,
// w + 4, ...; lane l holds columns 2l and 2l + 1 of the row in every block
// (512 contiguous bytes per wave load). Each lane keeps an online max and sum
// of its columns over the row's blocks; one max and one sum over the lanes
// give the row's stats, and a second pass writes the weights.
template <typename OutT>
__global__ __launch_bounds__(256) void bsa_block_softmax_kernel(const float* __restrict__ S,
                                                                const int64_t* __restrict__ rp, float scale,
                                                                OutT* __restrict__ P, float* __restrict__ row_max,
                                                                float* __restrict__ row_denom) {
  const int64_t R = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t k0 = rp[R], k1 = rp[R + 1];
  for (int r = w; r < BS; r += 4) {
    float m = -INFINITY, l = 0.f;
    for (int64_t k = k0; k < k1; ++k) {
      const f32x2 v = *reinterpret_cast<const f32x2*>(S + k * BB + r * BS + 2 * lane);
      const float a = scale * v.x, b = scale * v.y;
      const float mn = fmaxf(m, fmaxf(a, b));
      l = l * __expf(m - mn) + __expf(a - mn) + __expf(b - mn);
      m = mn;
    }
    const float M = wave_max(m);
    const float L = tsp::wave_sum(k1 > k0 ? l * __expf(m - M) : 0.f);
    const float mx = k1 > k0 ? M : 0.f;
    const float den = L > 1e-12f ? L : 1e-12f;
    if (lane == 0) {
      row_max[R * BS + r] = mx;
      row_denom[R * BS + r] = den;
    }
    for (int64_t k = k0; k < k1; ++k) {
      const int64_t e = k * BB + r * BS + 2 * lane;
      const f32x2 v = *reinterpret_cast<const f32x2*>(S + e);
      put(P + e, __expf(scale * v.x - mx) / den);
      put(P + e + 1, __expf(scale * v.y - mx) / den);
    }
  }
}

// One workgroup per stored block, rows as in the softmax kernel.
template <typename OutT>
__global__ __launch_bounds__(256) void bsa_block_grad_kernel(const float* __restrict__ S, const float* __restrict__ dP,
                                                             const int64_t* __restrict__ brow, float scale,
                                                             const float* __restrict__ row_max,
                                                             const float* __restrict__ row_denom,
                                                             const float* __restrict__ Drow, OutT* __restrict__ P,
                                                             OutT* __restrict__ dS) {
  const int64_t k = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row0 = brow[k] * BS;
  for (int r = w; r < BS; r += 4) {
    const float mx = row_max[row0 + r], den = row_denom[row0 + r], dd = Drow[row0 + r];
    const int64_t e = k * BB + r * BS + 2 * lane;
    const f32x2 s = *reinterpret_cast<const f32x2*>(S + e);
    const f32x2 g = *reinterpret_cast<const f32x2*>(dP + e);
    const float p0 = __expf(scale * s.x - mx) / den, p1 = __expf(scale * s.y - mx) / den;
    const float d0 = scale * (p0 * (g.x - dd)), d1 = scale * (p1 * (g.y - dd));
    put(P + e, p0);
    put(P + e + 1, p1);
    put(dS + e, d0);
    put(dS + e + 1, d1);
  }
}

template <typename T> __device__ inline float ldf(const T* p) { return (float)*p; }
template <> __device__ inline float ldf<uint16_t>(const uint16_t* p) { return tsp::bf16_bits_to_f32(*p); }
__device__ inline float cvf(float v) { return v; }
__device__ inline float cvf(uint16_t v) { return tsp::bf16_bits_to_f32(v); }

// Drow[r] = sum_d dO[r][d] O[r][d], one wavefront per row; VEC: head_dim a
// multiple of 4 with 8-byte (bf16) / 16-byte (fp32) aligned rows, four
// elements per lane and load.
template <typename T> struct Vec4;
template <> struct Vec4<float> { typedef f32x4 type; };
template <> struct Vec4<uint16_t> { typedef uint16_t type __attribute__((ext_vector_type(4))); };

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void bsa_rowdot_kernel(const T* __restrict__ O, const T* __restrict__ dO,
                                                         int64_t rows, int64_t D, float* __restrict__ Drow) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  float s = 0.f;
  if (VEC) {
    typedef typename Vec4<T>::type V4;
    const V4* o4 = reinterpret_cast<const V4*>(O + r * D);
    const V4* g4 = reinterpret_cast<const V4*>(dO + r * D);
    for (int64_t d = lane; d < D / 4; d += 64) {
      const V4 a = o4[d], b = g4[d];
      s += cvf((T)a.x) * cvf((T)b.x) + cvf((T)a.y) * cvf((T)b.y) + cvf((T)a.z) * cvf((T)b.z) + cvf((T)a.w) * cvf((T)b.w);
    }
  } else {
    for (int64_t d = lane; d < D; d += 64) s += ldf(O + r * D + d) * ldf(dO + r * D + d);
  }
  s = tsp::wave_sum(s);
  if (lane == 0) Drow[r] = s;
}

bool aligned8(const void* p) { return ((uintptr_t)p & 7) == 0; }

}  // namespace

extern "C" int tsp_bsa_block_softmax(const float* S, const int64_t* block_row_ptrs, int64_t n_block_rows,
                                     int64_t block_size, double scale, void* P, int out_dtype, float* row_max,
                                     float* row_denom, void* stream) {
  if (block_size != BS) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_block_softmax: block_size %lld (128 only)", (long long)block_size);
  if (out_dtype != TSP_F32 && out_dtype != TSP_BF16)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_block_softmax: out_dtype %d (f32 or bf16)", out_dtype);
  if (n_block_rows < 0) return tsp::fail(TSP_EINVAL, "tsp_bsa_block_softmax: bad size");
  if (n_block_rows == 0) return TSP_OK;
  if (n_block_rows > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_block_softmax: too many block rows");
  if (!block_row_ptrs || !row_max || !row_denom) return tsp::fail(TSP_EINVAL, "tsp_bsa_block_softmax: null pointer");
  if (!aligned8(S)) return tsp::fail(TSP_EINVAL, "tsp_bsa_block_softmax: S must be 8-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (out_dtype == TSP_F32)
    hipLaunchKernelGGL(bsa_block_softmax_kernel<float>, dim3((unsigned)n_block_rows), dim3(256), 0, st, S,
                       block_row_ptrs, (float)scale, (float*)P, row_max, row_denom);
  else
    hipLaunchKernelGGL(bsa_block_softmax_kernel<uint16_t>, dim3((unsigned)n_block_rows), dim3(256), 0, st, S,
                       block_row_ptrs, (float)scale, (uint16_t*)P, row_max, row_denom);
  return tsp::check_launch("bsa_block_softmax launch");
}

extern "C" int tsp_bsa_block_grad(const float* S, const float* dP, const int64_t* block_rows, int64_t n_blocks,
                                  int64_t block_size, double scale, const float* row_max, const float* row_denom,
                                  const float* Drow, void* P, void* dS, int out_dtype, void* stream) {
  if (block_size != BS) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_block_grad: block_size %lld (128 only)", (long long)block_size);
  if (out_dtype != TSP_F32 && out_dtype != TSP_BF16)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_block_grad: out_dtype %d (f32 or bf16)", out_dtype);
  if (n_blocks < 0) return tsp::fail(TSP_EINVAL, "tsp_bsa_block_grad: bad size");
  if (n_blocks == 0) return TSP_OK;
  if (n_blocks > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_block_grad: too many blocks");
  if (!S || !dP || !block_rows || !row_max || !row_denom || !Drow || !P || !dS)
    return tsp::fail(TSP_EINVAL, "tsp_bsa_block_grad: null pointer");
  if (!aligned8(S) || !aligned8(dP)) return tsp::fail(TSP_EINVAL, "tsp_bsa_block_grad: S and dP must be 8-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (out_dtype == TSP_F32)
    hipLaunchKernelGGL(bsa_block_grad_kernel<float>, dim3((unsigned)n_blocks), dim3(256), 0, st, S, dP, block_rows,
                       (float)scale, row_max, row_denom, Drow, (float*)P, (float*)dS);
  else
    hipLaunchKernelGGL(bsa_block_grad_kernel<uint16_t>, dim3((unsigned)n_blocks), dim3(256), 0, st, S, dP, block_rows,
                       (float)scale, row_max, row_denom, Drow, (uint16_t*)P, (uint16_t*)dS);
  return tsp::check_launch("bsa_block_grad launch");
}

extern "C" int tsp_bsa_rowdot(const void* O, const void* dO, int dtype, int64_t rows, int64_t head_dim, float* Drow,
                              void* stream) {
  if (dtype != TSP_F32 && dtype != TSP_BF16) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_rowdot: dtype %d", dtype);
  if (rows < 0 || head_dim < 0) return tsp::fail(TSP_EINVAL, "tsp_bsa_rowdot: bad size");
  if (rows == 0) return TSP_OK;
  if (!O || !dO || !Drow) return tsp::fail(TSP_EINVAL, "tsp_bsa_rowdot: null pointer");
  const int64_t grid = tsp::ceil_div(rows, 4);
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_rowdot: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const int64_t esz = dtype == TSP_F32 ? 4 : 2;
  const bool vec = head_dim % 4 == 0 && ((uintptr_t)O % (4 * esz)) == 0 && ((uintptr_t)dO % (4 * esz)) == 0;
  if (dtype == TSP_F32) {
    if (vec)
      hipLaunchKernelGGL((bsa_rowdot_kernel<float, true>), dim3((unsigned)grid), dim3(256), 0, st, (const float*)O,
                         (const float*)dO, rows, head_dim, Drow);
    else
      hipLaunchKernelGGL((bsa_rowdot_kernel<float, false>), dim3((unsigned)grid), dim3(256), 0, st, (const float*)O,
                         (const float*)dO, rows, head_dim, Drow);
  } else {
    if (vec)
      hipLaunchKernelGGL((bsa_rowdot_kernel<uint16_t, true>), dim3((unsigned)grid), dim3(256), 0, st,
                         (const uint16_t*)O, (const uint16_t*)dO, rows, head_dim, Drow);
    else
      hipLaunchKernelGGL((bsa_rowdot_kernel<uint16_t, false>), dim3((unsigned)grid), dim3(256), 0, st,
                         (const uint16_t*)O, (const uint16_t*)dO, rows, head_dim, Drow);
  }
  return tsp::check_launch("bsa_rowdot launch");
}
