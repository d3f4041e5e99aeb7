// Block-sparse attention backward for gfx950.
//
// Semantics follow the reference tiled backward (trnsparse/ops.py:360-473),
// per head, with the forward's row stats (row_max in natural-log units of the
// scaled scores, row_denom):
//   D[q]      = sum_d dO[q][d] * O[q][d]
//   P[q][k]   = exp(scale * Q[q].K[k] - row_max[q]) / row_denom[q]
//   dS[q][k]  = P[q][k] * (dO[q].V[k] - D[q])
//   dQ[q]    += scale * sum_k dS[q][k] K[k]      (k over q's stored blocks)
//   dK[k]    += scale * sum_q dS[q][k] Q[q]      (q over the query blocks that
//   dV[k]    += sum_q P[q][k] dO[q]               store k's block)
// Rows of Q past the last full block row, and keys that no stored block
// covers, get zero gradient. The reference's NKI kernels split this the same
// way (row-first dQ, column-first dK/dV over a BSC view,
// trnsparse/nki/kernels.py:295-524); its host gathers are not needed here.
//
// Kernels
//   bsa_bwd_d             D in the accumulation type (f32; f64 for f64).
//   bsa_bwd_dq_bf16_d128  bf16, b = 128, d = 128: workgroup per (head, query
//       block row), wavefront per 32 queries; per 64-key half
//       S^T = K Q^T and dP^T = V dO^T on v_mfma_f32_32x32x16_bf16 with the
//       wave's Q and dO rows in registers, P and dS in registers, then
//       dQ^T += K^T dS^T with K read through ds_read_b64_tr_b16. K/V halves
//       stream through a 4-stage LDS ring by direct buffer loads three
//       halves ahead.
//   bsa_bwd_dkdv_bf16_d128  same shapes: workgroup per (head, key block
//       column) over the block-column view of the mask, wavefront per 32 keys;
//       per 64-query half S = Q K^T and dP = dO V^T with the wave's K and V
//       rows in registers, then dV^T += dO^T P and dK^T += Q^T dS with Q and
//       dO read through transpose reads. Q/dO halves and their stats stream
//       through a 3-stage LDS ring, two halves ahead, as one stream across
//       the items of a persistent workgroup.
//   bsa_bwd_dq_f32<D> / bsa_bwd_dkdv_f32<D> / bsa_bwd_reduce_f32<D>  fp32,
//       b = 128, D in {64, 128}: the same passes on v_mfma_f32_32x32x2_f32
//       (operand forms at the kernels); D = 256 runs the row and column
//       passes of attention_bwd_d256.hip (16-row tiles) and the reduce here.
//   bsa_bwd_dq_generic / bsa_bwd_dkdv_generic  any dtype / block size /
//       head_dim: one thread per (row, 32-wide slice of head_dim).
// Swizzle: K (row pass) and Q, dO (column pass) are read both as 16-byte rows
// (16 consecutive keys of one chunk) and through transpose reads (4
// consecutive keys, 4 chunks); slot = chunk ^ (((key % 4) << 2) | ((key / 4) %
// 4)) is conflict-free for both on the 64-bank LDS. V in the row pass is only
// read as rows: slot = chunk ^ (key % 16).
#include <new>

#include "common.h"

#include "lds_dma.h"
#include "slots.h"

namespace tsp {
// attention_bwd_d256.hip: the fp32 head_dim-256 row and column passes
int bsa_bwd_f32_d256_rows(const float* Q, const float* K, const float* V, const float* O, const float* dO, int64_t S,
                        int64_t H, const int64_t* rp, const int64_t* ci, int64_t Mt, float scale_log2, float scale,
                        const float* rmax, const float* rden, float* qstat, float* dQ, hipStream_t st);
int bsa_bwd_f32_d256_cols(const float* Q, const float* K, const float* V, const float* dO, int64_t S, int64_t H,
                          const int64_t* crow, const int32_t* items, int64_t n_items, int n_partials, int64_t Mt,
                          float scale_log2, float scale, const float* qstat, float* dK, float* dV, float* partial,
                          hipStream_t st);
}  // namespace tsp

namespace {

constexpr float LOG2E = 1.4426950408889634f;

template <typename T> struct AAcc { typedef float type; };
template <> struct AAcc<double> { typedef double type; };
template <typename T> __device__ inline typename AAcc<T>::type ld(const T* p) { return (typename AAcc<T>::type)*p; }
template <> __device__ inline float ld<uint16_t>(const uint16_t* p) { return tsp::bf16_bits_to_f32(*p); }
template <typename T> __device__ inline T st(typename AAcc<T>::type v) { return (T)v; }
template <> __device__ inline uint16_t st<uint16_t>(float v) { return tsp::f32_to_bf16_bits(v); }
__device__ inline float aexp(float v) { return __expf(v); }
__device__ inline double aexp(double v) { return exp(v); }

// ------------------------------------------------------------------ D

template <typename T>
__global__ __launch_bounds__(256) void bsa_bwd_d(const T* __restrict__ O, const T* __restrict__ dO, int64_t rows,
                                                 int64_t D, typename AAcc<T>::type* __restrict__ Dout) {
  typedef typename AAcc<T>::type AccT;
  // one wavefront per row
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  AccT s = 0;
  for (int64_t d = lane; d < D; d += 64) s += ld(O + r * D + d) * ld(dO + r * D + d);
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if (lane == 0) Dout[r] = s;
}

// -------------------------------------------------------------- generic

constexpr int GEN_DC = 32;

// dQ: thread per (query, head_dim slice), walking the query's stored blocks.
// Stats are (head, Mt * b); D is (head, S).
template <typename T>
__global__ __launch_bounds__(128) void bsa_bwd_dq_generic(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V, const T* __restrict__ dO, int64_t S,
    int64_t D, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci, int64_t b, int64_t Mt,
    typename AAcc<T>::type scale, const typename AAcc<T>::type* __restrict__ rmax,
    const typename AAcc<T>::type* __restrict__ rden, const typename AAcc<T>::type* __restrict__ Dv, T* __restrict__ dQ) {
  typedef typename AAcc<T>::type AccT;
  const int64_t head = blockIdx.z;
  const int64_t q = (int64_t)blockIdx.x * 128 + threadIdx.x;
  if (q >= S) return;
  const int64_t d0 = (int64_t)blockIdx.y * GEN_DC;
  const int64_t hs = head * S * D;
  AccT acc[GEN_DC];
#pragma unroll
  for (int i = 0; i < GEN_DC; ++i) acc[i] = 0;
  const int64_t m = q / b;
  if (m < Mt) {
    const AccT mx = rmax[head * Mt * b + q], den = rden[head * Mt * b + q], Dq = Dv[head * S + q];
    for (int64_t idx = rp[m]; idx < rp[m + 1]; ++idx) {
      const int64_t key0 = ci[idx] * b;
      for (int64_t key = key0; key < key0 + b && key < S; ++key) {
        AccT s = 0, dp = 0;
        for (int64_t d = 0; d < D; ++d) {
          s += ld(Q + hs + q * D + d) * ld(K + hs + key * D + d);
          dp += ld(dO + hs + q * D + d) * ld(V + hs + key * D + d);
        }
        const AccT p = aexp(s * scale - mx) / den;
        const AccT ds = p * (dp - Dq) * scale;
#pragma unroll
        for (int i = 0; i < GEN_DC; ++i)
          if (d0 + i < D) acc[i] += ds * ld(K + hs + key * D + d0 + i);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < GEN_DC; ++i)
    if (d0 + i < D) dQ[hs + q * D + d0 + i] = st<T>(acc[i]);
}

// dK, dV: thread per (key, head_dim slice), walking the block rows that store
// the key's block column (block-column view: cp[ncols + 1] / crow). Block
// rows at or past Mt hold no queries of the forward and are skipped.
template <typename T>
__global__ __launch_bounds__(128) void bsa_bwd_dkdv_generic(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V, const T* __restrict__ dO, int64_t S,
    int64_t D, const int64_t* __restrict__ cp, const int64_t* __restrict__ crow, int64_t ncols, int64_t b, int64_t Mt,
    typename AAcc<T>::type scale, const typename AAcc<T>::type* __restrict__ rmax,
    const typename AAcc<T>::type* __restrict__ rden, const typename AAcc<T>::type* __restrict__ Dv, T* __restrict__ dK,
    T* __restrict__ dV) {
  typedef typename AAcc<T>::type AccT;
  const int64_t head = blockIdx.z;
  const int64_t key = (int64_t)blockIdx.x * 128 + threadIdx.x;
  if (key >= S) return;
  const int64_t d0 = (int64_t)blockIdx.y * GEN_DC;
  const int64_t hs = head * S * D;
  AccT ak[GEN_DC], av[GEN_DC];
#pragma unroll
  for (int i = 0; i < GEN_DC; ++i) ak[i] = av[i] = 0;
  const int64_t c = key / b;
  if (c < ncols) {
    for (int64_t p0 = cp[c]; p0 < cp[c + 1]; ++p0) {
      const int64_t m = crow[p0];
      if (m >= Mt) continue;
      for (int64_t q = m * b; q < m * b + b; ++q) {
        AccT s = 0, dp = 0;
        for (int64_t d = 0; d < D; ++d) {
          s += ld(Q + hs + q * D + d) * ld(K + hs + key * D + d);
          dp += ld(dO + hs + q * D + d) * ld(V + hs + key * D + d);
        }
        const AccT p = aexp(s * scale - rmax[head * Mt * b + q]) / rden[head * Mt * b + q];
        const AccT ds = p * (dp - Dv[head * S + q]) * scale;
#pragma unroll
        for (int i = 0; i < GEN_DC; ++i) {
          if (d0 + i < D) {
            av[i] += p * ld(dO + hs + q * D + d0 + i);
            ak[i] += ds * ld(Q + hs + q * D + d0 + i);
          }
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < GEN_DC; ++i) {
    if (d0 + i < D) {
      dK[hs + key * D + d0 + i] = st<T>(ak[i]);
      dV[hs + key * D + d0 + i] = st<T>(av[i]);
    }
  }
}

template <typename T>
int launch_generic(const void* Q, const void* K, const void* V, const void* dO, int64_t H, int64_t S, int64_t D,
                   const int64_t* rp, const int64_t* ci, const int64_t* cp, const int64_t* crow, int64_t ncols, int64_t b,
                   int64_t Mt, double scale, const void* rmax, const void* rden, const void* Dv, void* dQ, void* dK, void* dV,
                   hipStream_t stream) {
  typedef typename AAcc<T>::type AccT;
  const int64_t gx = tsp::ceil_div(S, 128), gy = tsp::ceil_div(D, GEN_DC);
  if (gx > INT32_MAX || gy > 65535 || H > 65535) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_bwd: problem too large for the generic kernels");
  hipLaunchKernelGGL((bsa_bwd_dq_generic<T>), dim3((unsigned)gx, (unsigned)gy, (unsigned)H), dim3(128), 0, stream,
                     (const T*)Q, (const T*)K, (const T*)V, (const T*)dO, S, D, rp, ci, b, Mt, (AccT)scale,
                     (const AccT*)rmax, (const AccT*)rden, (const AccT*)Dv, (T*)dQ);
  int rc = tsp::check_launch("bsa_bwd_dq_generic launch");
  if (rc) return rc;
  hipLaunchKernelGGL((bsa_bwd_dkdv_generic<T>), dim3((unsigned)gx, (unsigned)gy, (unsigned)H), dim3(128), 0, stream,
                     (const T*)Q, (const T*)K, (const T*)V, (const T*)dO, S, D, cp, crow, ncols, b, Mt, (AccT)scale,
                     (const AccT*)rmax, (const AccT*)rden, (const AccT*)Dv, (T*)dK, (T*)dV);
  return tsp::check_launch("bsa_bwd_dkdv_generic launch");
}

// ------------------------------------------------------- bf16 MFMA, d = 128

namespace abw {
constexpr int D = 128;
constexpr int BS = 128;             // block size served by the MFMA kernels
constexpr int HR = 64;              // rows (keys in the row pass, queries in the column pass) per ring stage
constexpr int ROWB = D * 2;         // bytes per row
constexpr int HBYTES = HR * ROWB;   // 16 KiB
constexpr int KS = D / 16;          // k-steps over head_dim
constexpr int NU = D / 32;          // 32-wide head_dim subtiles
constexpr int SEG_MAX = 64;         // most block rows one column-pass item walks
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

// The 16-byte chunk c of stage row r sits in slot c ^ swz(r). Rows are read
// as 16-byte pieces of 16 consecutive rows (one chunk) and through transpose
// reads of 4 consecutive rows (4 chunks); swz is a bijection on r % 16 whose
// low two bits follow r / 4 and high two bits r % 4, so both access forms hit
// 16 (resp. 4 x 4) distinct slots.
__host__ __device__ constexpr int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// One wave's share (rows [16w, 16w + 16)) of a 64-row half starting at global
// row row0 of the buffer `rs`, into the stage at LDS address dst.
__device__ inline void dma_half(tsp::dma::i32x4 rs, int64_t row0, uint32_t dst, int w, int lane) {
#pragma unroll
  for (int qq = 0; qq < 4; ++qq) {
    const int j = 4 * w + qq;
    const int rr = 4 * j + (lane >> 4);
    const int p = lane & 15;
    tsp::dma::buffer16(rs, (uint32_t)((row0 + rr) * ROWB + ((p ^ swz(rr)) << 4)), dst + j * 1024);
  }
}

// A operand of v_mfma_f32_32x32x16_bf16 from stage rows r0 + [0, 32) (lane
// row r0 + l32), head_dim chunk 2 ks + h: lane offset l32 * ROWB, kx = swz(l32) ^ h.
__device__ inline bf16x8 row_read(const uint8_t* base, int loff, int kx, int r0, int ks) {
  return *(const bf16x8*)(base + loff + r0 * ROWB + (((2 * ks) ^ kx) << 4));
}

// A operand holding the transpose: rows (MFMA i) are head_dim 32u + l32 and
// the 8 k values are stage rows r0 + 4h + {0..3} and r0 + 8 + 4h + {0..3}
// (the k order of the lane's own accumulator rows), from two
// ds_read_b64_tr_b16: lane j of 16-lane group gq points at row
// r0 + 8 rr + 4 (gq / 2) + j / 4, column 32u + 16 (gq % 2) + 4 (j % 4).
struct TrLane {
  int off[2];
  int xu;
};
__device__ inline TrLane tr_lane(int lane) {
  const int gq = lane >> 4, jq = lane & 15;
  const int c0 = 2 * (gq & 1) + ((jq & 3) >> 1);
  TrLane t;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int row = 8 * rr + 4 * (gq >> 1) + (jq >> 2);
    t.off[rr] = row * ROWB + ((c0 ^ (swz(row) & 3)) << 4) + 8 * (jq & 1);
  }
  t.xu = jq >> 2;  // swz(row) >> 2
  return t;
}
__device__ inline bf16x8 tr_read(const uint8_t* base, const TrLane& t, int r0, int u) {
  s16x4 r[2];
#pragma unroll
  for (int rr = 0; rr < 2; ++rr)
    r[rr] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + t.off[rr] + r0 * ROWB + ((u ^ t.xu) << 6)));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7));
}
// Address form of the two reads for the slot kernels. A stage starts at an
// LDS address that is a multiple of 256 and rows are 256 bytes, so the
// swizzled chunk bits (4-7) of a lane's address are free in the stage base:
// per step one base per access kind is formed (row reads: stage + l32 * ROWB
// + swz(l32)^h in bits 4-7; transpose reads: stage + off[rr] + xu in bits
// 6-7) and each read is base ^ (k-step or subtile bits) plus a constant row
// offset that the ds_read immediate absorbs.
// Round 4 floats to bf16 (round to nearest even, v_cvt_pk_bf16_f32) as 4 halfwords.
__device__ inline u16x4 bf16x4_rne(f32x4 v) {
  return __builtin_bit_cast(u16x4, __builtin_convertvector(v, bf16x4));
}


typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
__device__ inline bf16x8 lds_row(uint32_t rb, int ks, uint32_t off) {
  return *(const lds_bf16x8*)(uintptr_t)((rb ^ (uint32_t)(ks << 5)) + off);
}
__device__ inline bf16x8 lds_trp(uint32_t tb0, uint32_t tb1, int u, uint32_t off) {
  const s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)((tb0 ^ (uint32_t)(u << 6)) + off));
  const s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)((tb1 ^ (uint32_t)(u << 6)) + off));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7));
}
}  // namespace abw

// Both passes run one wavefront per SIMD (a 256-thread workgroup per CU)
// and issue their work in a fixed slot order: slot k is one MFMA whose LDS
// operand was read PF slots earlier (a register ring, so LDS latency hides
// behind the MFMAs of the same wave), plus a slice of the softmax-gradient
// VALU work of the previous 32-row tile, so that the VALU runs while the
// matrix core is busy. sched_barrier keeps the compiler from regrouping
// the slots.
constexpr int PF = 4;  // operand reads in flight


// Row pass: workgroup per (head, query block row m < Mt), XCD-aware order as
// the forward (XCD x walks heads x, x + 8, ...; block rows of one head side by
// side share its K/V in L2). Wavefront w owns queries m * 128 + 32 w + [0, 32)
// with their Q and dO rows in registers; 64-key halves of K and V stream
// through a 4-stage LDS ring by direct buffer loads issued three halves ahead.
// Per half, slots 0-31: S^T and dP^T tiles of the two 32-key tiles tt (16
// MFMAs each, K / V rows as A, Q / dO as B); slots 16-39 also form P^T and
// dS^T of tile 0 (slots 16-31) and tile 1 (32-39); slots 32-47: dQ^T += K^T
// dS^T (K through transpose reads). Also computes D and leaves per-query
// stats for the column pass: plane 0 r = log2e * row_max + log2 row_denom
// (P = exp2(log2e * scale * s - r)), plane 1 D.
__global__ __launch_bounds__(256, 1) void bsa_bwd_dq_bf16_d128(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ O, const uint16_t* __restrict__ dO, int64_t S, int64_t H,
    const int64_t* __restrict__ rp, const int64_t* __restrict__ ci, int64_t Mt, float scale_log2, float scale,
    const float* __restrict__ rmax, const float* __restrict__ rden, float* __restrict__ qstat,
    uint16_t* __restrict__ dQ) {
  using namespace abw;
  constexpr int STAGE = 2 * HBYTES;  // K half, V half
  constexpr int NST = 4;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];

  const int64_t g = blockIdx.x;
  const int64_t xcd = g & 7, slot = g >> 3;
  const int64_t head = xcd + 8 * (slot / Mt);
  const int64_t m = slot % Mt;
  if (head >= H) return;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t hs = head * S * D;
  const int64_t q = m * BS + w * 32 + l32;  // < S since m < Mt

  bf16x8 qf[KS], dof[KS];  // the lane's Q and dO rows (B operands), loaded below
  float Dq = 0.f, rq = 0.f;

  f32x16 acc[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) acc[u] = f32x16{};

  const int64_t start = rp[m];
  const int nblk = (int)(rp[m + 1] - start);
  const int nsteps = 2 * nblk;
  const tsp::dma::i32x4 krs = tsp::dma::make_rsrc(K + hs, (uint32_t)(S * ROWB));
  const tsp::dma::i32x4 vrs = tsp::dma::make_rsrc(V + hs, (uint32_t)(S * ROWB));
  const uint32_t lds0 = tsp::dma::lds_addr(lds);

  // key-block indices of the row, 64 at a time in one VGPR, read with readlane;
  // the load side (three halves ahead) and the compute side keep their own copy
  auto load_cols = [&](int base) {
    const int i = base + lane < nblk ? base + lane : nblk - 1;
    return tsp::dma::load_lo32_sync(ci + start + i);
  };
  int cb_i = 0, cv_i = 0, cb_c = 0, cv_c = 0;
  if (nblk > 0) cv_i = cv_c = load_cols(0);
  auto key_of = [&](int s, int& cb, int& cv) {
    const int blk = s >> 1;
    if (blk - cb >= 64) {
      cb = blk & ~63;
      cv = load_cols(cb);
    }
    return (int64_t)__builtin_amdgcn_readlane(cv, blk - cb) * BS + HR * (s & 1);
  };
  auto issue = [&](int s) {
    const int64_t key0 = key_of(s, cb_i, cv_i);
    const uint32_t st = lds0 + (s % NST) * STAGE;
    dma_half(krs, key0, st, w, lane);
    dma_half(vrs, key0, st + HBYTES, w, lane);
  };

  const int loff = l32 * ROWB;
  const int kx = swz(l32) ^ h;
  const TrLane trl = tr_lane(lane);
  float nr = 0.f;

  auto compute = [&](uint32_t st, int64_t key0) {
    const bool tail = key0 + HR > S;
    const uint32_t rb = st + (uint32_t)(loff + (kx << 4));
    const uint32_t tb0 = st + (uint32_t)(trl.off[0] + (trl.xu << 6));
    const uint32_t tb1 = st + (uint32_t)(trl.off[1] + (trl.xu << 6));
    // slot -> LDS operand: 0-31 S^T / dP^T of tile k / 16 (even: K row, odd:
    // V row, k-step (k % 16) / 2); 32-47 K^T for dQ of tile (k - 32) / 8,
    // k-step a = (k / 4) % 2, head_dim subtile u = k % 4
    auto fetch = [&](int k) -> bf16x8 {
      if (k < 32) return lds_row(rb, (k & 15) >> 1, (k & 1) * HBYTES + 32 * (k >> 4) * ROWB);
      const int j = k - 32;
      return lds_trp(tb0, tb1, j & 3, (32 * (j >> 3) + 16 * ((j >> 2) & 1)) * ROWB);
    };
    f32x16 sc[2], dp[2];
    float pd[2][16];
    bf16x8 db[2][2];
    bf16x8 ring[PF];
    tsp::static_for<PF>([&](auto kc) __attribute__((always_inline)) { ring[decltype(kc)::value] = fetch(decltype(kc)::value); });
    // dS^T element v of tile tt (key 32 tt + 8 (v / 4) + 4 h + v % 4)
    auto ds_elem = [&](int tt, int v) {
      float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[tt][v], scale_log2, nr));
      if (tail && key0 + 32 * tt + 8 * (v >> 2) + 4 * h + (v & 3) >= S) p = 0.f;
      pd[tt][v] = p * (dp[tt][v] - Dq);
      if ((v & 7) == 7) {
        typedef float f32x8_ __attribute__((ext_vector_type(8)));
        f32x8_ t;
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = pd[tt][(v & 8) + i];
        db[tt][v >> 3] = __builtin_convertvector(t, bf16x8);
      }
    };
    tsp::static_for<48>([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      const bf16x8 op = ring[k % PF];
      if constexpr (k + PF < 48) ring[k % PF] = fetch(k + PF);
      if constexpr (k < 32) {
        constexpr int tt = k >> 4, ks = (k & 15) >> 1;
        if constexpr (k & 1)
          dp[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op, dof[ks], ks ? dp[tt] : f32x16{}, 0, 0, 0);
        else
          sc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op, qf[ks], ks ? sc[tt] : f32x16{}, 0, 0, 0);
      } else {
        constexpr int j = k - 32;
        acc[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op, db[j >> 3][(j >> 2) & 1], acc[j & 3], 0, 0, 0);
      }
      if constexpr (k >= 16 && k < 32) ds_elem(0, k - 16);
      if constexpr (k >= 32 && k < 40) {
        ds_elem(1, 2 * (k - 32));
        ds_elem(1, 2 * (k - 32) + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

#pragma unroll
  for (int s = 0; s < NST - 1; ++s)
    if (s < nsteps) issue(s);
  // Q, dO and O rows of the lane's query ([16 ks + 8 h, +8)) load behind the
  // first halves; D and the stats for the column pass
  float dsum = 0.f;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    qf[s] = *(const bf16x8*)(Q + hs + q * D + 16 * s + 8 * h);
    dof[s] = *(const bf16x8*)(dO + hs + q * D + 16 * s + 8 * h);
    const bf16x8 of = *(const bf16x8*)(O + hs + q * D + 16 * s + 8 * h);
#pragma unroll
    for (int i = 0; i < 8; ++i) dsum += (float)dof[s][i] * (float)of[i];
  }
  Dq = dsum + __shfl_xor(dsum, 32, 64);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    tsp::pin_agpr(qf[s]);
    tsp::pin_agpr(dof[s]);
  }
  rq = rmax[head * Mt * BS + q] * LOG2E + __builtin_amdgcn_logf(rden[head * Mt * BS + q]);
  nr = -rq;
  if (h == 0) {
    const int64_t HS = H * S;
    qstat[head * S + q] = rq;
    qstat[HS + head * S + q] = Dq;
  }
  for (int s = 0; s < nsteps; ++s) {
    const int64_t key0 = key_of(s, cb_c, cv_c);
    // this wave's loads of half s are done once only the later halves (8
    // loads each) are outstanding
    const int ahead = nsteps - 1 - s < NST - 2 ? nsteps - 1 - s : NST - 2;
    if (ahead >= 2)
      tsp::dma::wait_vm<16>();
    else if (ahead == 1)
      tsp::dma::wait_vm<8>();
    else
      tsp::dma::wait_vm<0>();
    tsp::dma::barrier();  // every wave's part is in LDS; stage (s - 1) % NST is free
    if (s + NST - 1 < nsteps) issue(s + NST - 1);
    compute(lds0 + (s % NST) * STAGE, key0);
  }

  // dQ[q][32 u + 8 g4 + 4 h + i] = scale * acc[u][4 g4 + i]
  uint16_t* dq = dQ + hs + q * D;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4 t = {acc[u][4 * g4], acc[u][4 * g4 + 1], acc[u][4 * g4 + 2], acc[u][4 * g4 + 3]};
      *(u16x4*)(dq + 32 * u + 8 * g4 + 4 * h) = bf16x4_rne(t * scale);
    }
  }
}

// Column pass, persistent: 8 * G8 workgroups (G8 <= 32 per XCD, one per
// CU); workgroup j of XCD x takes the slots j, j + G8, j + 2 G8, ... of its
// XCD's slot list, slot s = (item s / nh, head x + 8 (s % nh)); an item is
// (block column, range [p0, p1) of its column view, partial slot or -1) and
// items are sorted heaviest first, so the round robin spreads the work. The
// item records and their block rows (gathered from the column view) are
// staged in LDS RCAP at a time; the 64-query halves of all items of a batch
// form one stream through a 3-stage LDS ring (Q half, dO half and their
// stats, direct buffer loads two halves ahead), so the loads of an item's
// first halves overlap the previous item's last ones, and the next item's K
// and V rows load during the current item's last half.
// Wavefront w owns keys col * 128 + 32 w + [0, 32) with the K and V rows in
// registers. Per half, slots 0-31: S and dP tiles of the two 32-query tiles
// qt (Q / dO rows as A, K / V as B); slots 16-47 also form P and dS of tile 0
// (16-31) and tile 1 (32-47), one element per slot; slots 32-63: dV^T +=
// dO^T P and dK^T += Q^T dS (dO, Q through transpose reads). An item covering
// a whole column writes bf16 dK / dV, a segment of a split column writes
// fp32 partials that bsa_bwd_reduce sums in segment order.
constexpr int RCAP = 64;  // item records staged per batch
__global__ __launch_bounds__(256, 1) void bsa_bwd_dkdv_bf16_d128(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ dO, int64_t S, int64_t H, int nh, const int64_t* __restrict__ crow,
    const int32_t* __restrict__ items, int n_items, int n_partials, float scale_log2, float scale,
    const float* __restrict__ qstat, uint16_t* __restrict__ dK, uint16_t* __restrict__ dV,
    float* __restrict__ partial) {
  using namespace abw;
  constexpr int STAGE = 2 * HBYTES + 1024;  // Q half, dO half, stats [4][64] floats (r, D, D, D)
  constexpr int NST = 3;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];
  __shared__ int32_t rhdr[RCAP][4];        // col, partial slot, n block rows (-1: no such head), head
  __shared__ int32_t rrow[RCAP][SEG_MAX];  // block rows of the item

  const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3, G8 = gridDim.x >> 3;
  const int64_t nslots = (int64_t)n_items * nh;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t HS = H * S;
  const uint32_t lds0 = tsp::dma::lds_addr(lds);
  // per-item state (the compute lambda reads it)
  f32x16 dk[NU], dv[NU];
  bf16x8 kf[KS], vf[KS];  // the wave's K and V rows (B operands)
  bf16x8 kn[KS], vn[KS];  // the next item's, loaded during the current item's last half

  const int loff = l32 * ROWB;
  const int kx = swz(l32) ^ h;
  const TrLane trl = tr_lane(lane);

  auto compute = [&](uint32_t st) {
    const uint32_t rb = st + (uint32_t)(loff + (kx << 4));
    const uint32_t tb0 = st + (uint32_t)(trl.off[0] + (trl.xu << 6));
    const uint32_t tb1 = st + (uint32_t)(trl.off[1] + (trl.xu << 6));
    const uint32_t sb = st + 2 * HBYTES + 16 * h;
    // slot -> LDS operand: 0-31 S / dP of tile k / 16 (even: Q row, odd: dO
    // row, k-step (k % 16) / 2); 32-63 of tile (k - 32) / 16, k-step
    // a = (k / 8) % 2, subtile u = (k / 2) % 4 (even: dO^T for dV, odd: Q^T for dK)
    auto fetch = [&](int k) -> bf16x8 {
      if (k < 32) return lds_row(rb, (k & 15) >> 1, (k & 1) * HBYTES + 32 * (k >> 4) * ROWB);
      const int j = k - 32;
      return lds_trp(tb0, tb1, (j >> 1) & 3, ((j & 1) ? 0 : HBYTES) + (32 * (j >> 4) + 16 * ((j >> 3) & 1)) * ROWB);
    };
    f32x16 sc[2], dp[2];
    u32x4 pw[2][2], dw[2][2];  // bf16 pairs of P and dS, k order of the B operand
    f32x4 rc, dc, rn, dn;      // stats of the current / next group of 4 queries
    bf16x8 ring[PF];
    tsp::static_for<PF>([&](auto kc) __attribute__((always_inline)) { ring[decltype(kc)::value] = fetch(decltype(kc)::value); });
    // stats (r, D) of the queries 32 qt + 8 g + 4 h + [0, 4)
    typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
    auto stats = [&](int qt, int gg) {
      rn = *(const lds_f32x4*)(uintptr_t)(sb + 4 * (32 * qt + 8 * gg));
      dn = *(const lds_f32x4*)(uintptr_t)(sb + 4 * (64 + 32 * qt + 8 * gg));
    };
    // P and dS elements v, v + 1 of tile qt (query 32 qt + 8 (v / 4) + 4 h + v % 4)
    auto ds_pair = [&](int qt, int v) {
      if ((v & 3) == 0) {
        rc = rn;
        dc = dn;
        if (v < 12)
          stats(qt, (v >> 2) + 1);
        else if (qt == 0)
          stats(1, 0);
      }
      typedef float f32x2 __attribute__((ext_vector_type(2)));
      typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
      f32x2 p, d;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = v + i;
        p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[qt][e], scale_log2, -rc[e & 3]));
        d[i] = p[i] * (dp[qt][e] - dc[e & 3]);
      }
      pw[qt][v >> 3][(v & 7) >> 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2));
      dw[qt][v >> 3][(v & 7) >> 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(d, bf16x2));
    };
    tsp::static_for<64>([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      const bf16x8 op = ring[k % PF];
      if constexpr (k + PF < 64) ring[k % PF] = fetch(k + PF);
      if constexpr (k == 12) stats(0, 0);
      if constexpr (k < 32) {
        constexpr int qt = k >> 4, ks = (k & 15) >> 1;
        if constexpr (k & 1)
          dp[qt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op, vf[ks], ks ? dp[qt] : f32x16{}, 0, 0, 0);
        else
          sc[qt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op, kf[ks], ks ? sc[qt] : f32x16{}, 0, 0, 0);
      } else {
        constexpr int j = k - 32, qt = j >> 4, a = (j >> 3) & 1, u = (j >> 1) & 3;
        if constexpr (j & 1)
          dk[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op, __builtin_bit_cast(bf16x8, dw[qt][a]), dk[u], 0, 0, 0);
        else
          dv[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op, __builtin_bit_cast(bf16x8, pw[qt][a]), dv[u], 0, 0, 0);
      }
      if constexpr (k >= 16 && k < 48 && (k & 1) == 0) ds_pair((k - 16) >> 4, (k - 16) & 15);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  auto load_kv = [&](int col, int head, bf16x8* kr, bf16x8* vr) {
    const int64_t key = (int64_t)col * BS + w * 32 + l32;
    const bool kvalid = key < S;
    const int64_t off = head * S * D + key * D + 8 * h;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      kr[s] = kvalid ? *(const bf16x8*)(K + off + 16 * s) : bf16x8{};
      vr[s] = kvalid ? *(const bf16x8*)(V + off + 16 * s) : bf16x8{};
    }
  };

  for (int64_t r0 = 0; j + r0 * G8 < nslots; r0 += RCAP) {
    // ---- stage the batch's item records and block rows
    const int64_t left = (nslots - j + G8 - 1) / G8 - r0;
    const int R = (int)(left < RCAP ? left : RCAP);
    __syncthreads();  // the previous batch's records and ring are no longer read
    if (tid < R) {
      const int64_t sl = j + (r0 + tid) * G8;
      const int64_t it = sl / nh, head = xcd + 8 * (sl % nh);
      rhdr[tid][0] = items[4 * it];
      rhdr[tid][1] = items[4 * it + 3];
      rhdr[tid][2] = head < H ? items[4 * it + 2] - items[4 * it + 1] : -1;
      rhdr[tid][3] = (int32_t)head;
    }
    for (int e = tid; e < R * SEG_MAX; e += 256) {
      const int r = e / SEG_MAX, i = e % SEG_MAX;
      const int64_t sl = j + (r0 + r) * G8;
      const int64_t it = sl / nh;
      const int p0 = items[4 * it + 1], n = items[4 * it + 2] - p0;
      if (i < n) rrow[r][i] = (int32_t)crow[p0 + i];
    }
    __syncthreads();

    // ---- one stream of halves over the batch's items
    auto nsteps_of = [&](int r) {
      const int n = __builtin_amdgcn_readfirstlane(rhdr[r][2]);
      return n > 0 ? 2 * n : 0;
    };
    int pr = 0, pt = 0, pc = 0;  // producer: item, half within it, halves issued
    auto p_skip = [&]() {
      while (pr < R && pt >= nsteps_of(pr)) {
        ++pr;
        pt = 0;
      }
    };
    auto issue_next = [&]() {
      if (pr >= R) return;
      const int head = __builtin_amdgcn_readfirstlane(rhdr[pr][3]);
      const int64_t q0 = (int64_t)__builtin_amdgcn_readfirstlane(rrow[pr][pt >> 1]) * BS + HR * (pt & 1);
      const int64_t hs = (int64_t)head * S * D;
      const uint32_t st = lds0 + (pc % NST) * STAGE;
      dma_half(tsp::dma::make_rsrc(Q + hs, (uint32_t)(S * ROWB)), q0, st, w, lane);
      dma_half(tsp::dma::make_rsrc(dO + hs, (uint32_t)(S * ROWB)), q0, st + HBYTES, w, lane);
      if (w == 0)
        tsp::dma::global16(qstat + ((lane >> 4) ? HS : 0) + (int64_t)head * S + 4 * (lane & 15) + q0,
                           st + 2 * HBYTES);
      ++pt;
      ++pc;
      p_skip();
    };
    p_skip();
    issue_next();
    issue_next();
    int cc = 0;  // halves consumed
    bool have_next = false;
    for (int r = 0; r < R; ++r) {
      const int nst = nsteps_of(r);
      if (__builtin_amdgcn_readfirstlane(rhdr[r][2]) < 0) continue;  // head past H
      const int col = __builtin_amdgcn_readfirstlane(rhdr[r][0]);
      const int pslot = __builtin_amdgcn_readfirstlane(rhdr[r][1]);
      const int head = __builtin_amdgcn_readfirstlane(rhdr[r][3]);
      if (have_next) {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          kf[s] = kn[s];
          vf[s] = vn[s];
        }
      } else {
        load_kv(col, head, kf, vf);
      }
      have_next = false;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        tsp::pin_agpr(kf[s]);
        tsp::pin_agpr(vf[s]);
      }
#pragma unroll
      for (int u = 0; u < NU; ++u) dk[u] = dv[u] = f32x16{};
      for (int t = 0; t < nst; ++t) {
        // loads of half cc are done once only the next half's (8 or 9
        // loads) may be outstanding
        if (pc > cc + 1)
          tsp::dma::wait_vm<8>();
        else
          tsp::dma::wait_vm<0>();
        tsp::dma::barrier();  // every wave's part is in LDS; stage (cc + 2) % 3 is free
        issue_next();
        if (t == nst - 1) {  // the next item's K and V rows
          int rn = r + 1;
          while (rn < R && __builtin_amdgcn_readfirstlane(rhdr[rn][2]) < 0) ++rn;
          if (rn < R) {
            load_kv(__builtin_amdgcn_readfirstlane(rhdr[rn][0]), __builtin_amdgcn_readfirstlane(rhdr[rn][3]), kn, vn);
            have_next = true;
          }
        }
        compute(lds0 + (cc % NST) * STAGE);
        ++cc;
      }

      // lane holds dK^T / dV^T [32 u + 8 g4 + 4 h + i][key]
      const int64_t key = (int64_t)col * BS + w * 32 + l32;
      const int64_t hs = (int64_t)head * S * D;
      if (pslot < 0) {
        if (key < S) {
          uint16_t* pk = dK + hs + key * D;
          uint16_t* pv = dV + hs + key * D;
#pragma unroll
          for (int u = 0; u < NU; ++u) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              const f32x4 tk = {dk[u][4 * g4], dk[u][4 * g4 + 1], dk[u][4 * g4 + 2], dk[u][4 * g4 + 3]};
              const f32x4 tv = {dv[u][4 * g4], dv[u][4 * g4 + 1], dv[u][4 * g4 + 2], dv[u][4 * g4 + 3]};
              *(u16x4*)(pk + 32 * u + 8 * g4 + 4 * h) = bf16x4_rne(tk * scale);
              *(u16x4*)(pv + 32 * u + 8 * g4 + 4 * h) = bf16x4_rne(tv);
            }
          }
        }
      } else {
        float* pk = partial + (((int64_t)head * n_partials + pslot) * 2) * (BS * D) + (w * 32 + l32) * D;
        float* pv = pk + BS * D;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const f32x4 tk = {dk[u][4 * g4], dk[u][4 * g4 + 1], dk[u][4 * g4 + 2], dk[u][4 * g4 + 3]};
            const f32x4 tv = {dv[u][4 * g4], dv[u][4 * g4 + 1], dv[u][4 * g4 + 2], dv[u][4 * g4 + 3]};
            *(f32x4*)(pk + 32 * u + 8 * g4 + 4 * h) = tk * scale;
            *(f32x4*)(pv + 32 * u + 8 * g4 + 4 * h) = tv;
          }
        }
      }
    }
    tsp::dma::wait_vm<0>();
  }
}

// dK / dV of the split columns: sum of the segments' partials in segment
// order (deterministic), rounded to bf16. Workgroup per (split, 16-key chunk
// of the column, head); thread per 4 consecutive head_dim values of one key
// of dK or dV.
__global__ __launch_bounds__(256) void bsa_bwd_reduce(const int32_t* __restrict__ splits, int n_partials, int64_t S,
                                                      const float* __restrict__ partial, uint16_t* __restrict__ dK,
                                                      uint16_t* __restrict__ dV) {
  using namespace abw;
  const int sp = blockIdx.x >> 3, chunk = blockIdx.x & 7;
  const int64_t head = blockIdx.y;
  const int col = splits[4 * sp], slot0 = splits[4 * sp + 1], nseg = splits[4 * sp + 2];
  const float* base = partial + (head * n_partials + slot0) * 2 * (BS * D);
#pragma unroll
  for (int e0 = 0; e0 < 2 * 16 * (D / 4); e0 += 256) {
    const int e = e0 + threadIdx.x;
    const int which = e / (16 * (D / 4));
    const int r = chunk * 16 + (e / (D / 4)) % 16, d4 = e % (D / 4);
    const int64_t key = (int64_t)col * BS + r;
    if (key >= S) continue;
    f32x4 sum = f32x4{};
    for (int j = 0; j < nseg; ++j) sum += *(const f32x4*)(base + (j * 2 + which) * (BS * D) + r * D + 4 * d4);
    *(u16x4*)((which ? dV : dK) + (head * S + key) * D + 4 * d4) = bf16x4_rne(sum);
  }
}

// ------------------------------------------------------------- fp32 MFMA
//
// fp32, b = 128, head_dim D in {64, 128}, on v_mfma_f32_32x32x2_f32. Same
// split as the bf16 kernels (a row pass for dQ that also leaves the query
// stats, a column pass for dK / dV over the column plan, a reduce for split
// columns), with one ring stage per 4096 / D rows (K and V rows in the row
// pass, Q and dO rows plus their stats in the column pass) streamed by direct
// buffer loads one stage ahead. Operand forms, as in the fp32 forward:
//   * products over head_dim (S, dP): lane half h supplies d = 8t + 4h + c
//     at step 4t + c, one b128 read per four MFMAs from 32 rows of a stage
//     (chunk read) against the wave's own rows held in registers;
//   * products over rows (dQ, dK, dV): the output's MFMA row r is head_dim
//     NU*r + u, so one contiguous read of NU floats of a stage row (row
//     read) feeds all NU subtiles, and the k index follows the accumulator
//     row order of the S / dP tiles, whose elements are the B operand in
//     place.
// Stage rows are stored 16-byte chunk ^ (row % 16): chunk reads of one chunk
// from 32 rows hit distinct banks, and a row read is a permutation of one
// row.
namespace abf {
template <int D>
struct Cfg {
  static constexpr int BS = 128;
  static constexpr int HR = 4096 / D;       // rows per ring stage
  static constexpr int ROWB = D * 4;        // bytes per row
  static constexpr int HBYTES = HR * ROWB;  // 16 KiB
  static constexpr int NT = HR / 32;        // 32-row tiles per stage
  static constexpr int NU = D / 32;         // head_dim subtiles of row products
  static constexpr int KT = D / 8;          // b128 chunk reads per 32-row tile
  static constexpr int SPB = BS / HR;       // stages per block
};
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <int NU> struct VRow;
template <> struct VRow<4> { typedef f32x4 type; };
template <> struct VRow<2> { typedef f32x2 type; };

// One wave's share of a stage: rows [row0, row0 + HR) of the buffer rs into
// LDS dst, 16 instructions of 1 KiB, 4 per wave.
template <int D>
__device__ inline void dma_rows(tsp::dma::i32x4 rs, int64_t row0, uint32_t dst, int w, int lane) {
  constexpr int LPR = D / 4, RPI = 64 / LPR, ROWB = D * 4;
#pragma unroll
  for (int qq = 0; qq < 4; ++qq) {
    const int j = 4 * w + qq;
    const int rr = RPI * j + lane / LPR;
    const int p = lane % LPR;
    tsp::dma::buffer16(rs, (uint32_t)((row0 + rr) * ROWB + ((p ^ (rr & 15)) << 4)), dst + j * 1024);
  }
}
// chunk read: logical chunk c of stage row `row` (row % 16 == kx)
template <int D>
__device__ inline f32x4 chunk_read(const uint8_t* base, int row, int c, int kx) {
  return *(const f32x4*)(base + row * (D * 4) + ((c ^ kx) << 4));
}
// row read: floats [NU * l32, NU * l32 + NU) of stage row `row`
template <int D>
__device__ inline typename VRow<D / 32>::type row_read(const uint8_t* base, int row, int l32) {
  constexpr int NU = D / 32;
  const int byte = NU * 4 * l32;
  return *(const typename VRow<NU>::type*)(base + row * (D * 4) + ((((byte >> 4) ^ (row & 15))) << 4) + (byte & 15));
}
// Store a 32-row x D tile held as NU accumulators (element v of subtile u is
// head_dim NU * (8 (v / 4) + 4 h + v % 4) + u of the lane's row) to dst, times f.
template <int D>
__device__ inline void store_rows(float* dst, const f32x16* acc, int h, float f) {
  constexpr int NU = D / 32;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    float* d = dst + NU * (8 * a + 4 * h);
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      f32x4 t;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int idx = 4 * k + e;
        t[e] = acc[idx % NU][4 * a + idx / NU] * f;
      }
      *(f32x4*)(d + 4 * k) = t;
    }
  }
}
}  // namespace abf

// Row pass: workgroup per (head, query block row m < Mt), XCD-aware order as
// the forward; wavefront w owns queries m * 128 + 32 w + [0, 32) with their Q
// and dO rows in registers. Per 32-key tile: S^T = K Q^T and dP^T = V dO^T
// (K, V chunk reads), dS^T = P^T (dP^T - D) in place, dQ^T += K^T dS^T (K row
// reads). Writes the column pass's query stats: plane 0 r = log2e * row_max
// + log2 row_denom (P = exp2(log2e * scale * s - r)), plane 1 D.
template <int D>
__global__ __launch_bounds__(256, 1) void bsa_bwd_dq_f32(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V, const float* __restrict__ O,
    const float* __restrict__ dO, int64_t S, int64_t H, const int64_t* __restrict__ rp,
    const int64_t* __restrict__ ci, int64_t Mt, float scale_log2, float scale, const float* __restrict__ rmax,
    const float* __restrict__ rden, float* __restrict__ qstat, float* __restrict__ dQ) {
  typedef abf::Cfg<D> C;
  constexpr int BS = C::BS, HR = C::HR, ROWB = C::ROWB, HBYTES = C::HBYTES, NT = C::NT, NU = C::NU, KT = C::KT;
  constexpr int SPB = C::SPB, STAGE = 2 * HBYTES, NST = 2;
  typedef typename abf::VRow<NU>::type vrow_t;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];

  const int64_t g = blockIdx.x;
  const int64_t xcd = g & 7, slot = g >> 3;
  const int64_t head = xcd + 8 * (slot / Mt);
  const int64_t m = slot % Mt;
  if (head >= H) return;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t hs = head * S * D;
  const int64_t q = m * BS + w * 32 + l32;  // < S since m < Mt

  f32x4 qf[KT], dof[KT];
  float dsum = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    qf[t] = *(const f32x4*)(Q + hs + q * D + 8 * t + 4 * h);
    dof[t] = *(const f32x4*)(dO + hs + q * D + 8 * t + 4 * h);
    const f32x4 of = *(const f32x4*)(O + hs + q * D + 8 * t + 4 * h);
#pragma unroll
    for (int c = 0; c < 4; ++c) dsum += dof[t][c] * of[c];
  }
  const float Dq = dsum + __shfl_xor(dsum, 32, 64);
  const float rq = rmax[head * Mt * BS + q] * LOG2E + __builtin_amdgcn_logf(rden[head * Mt * BS + q]);
  const float nr = -rq;
  if (h == 0) {
    qstat[head * S + q] = rq;
    qstat[H * S + head * S + q] = Dq;
  }

  f32x16 acc[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) acc[u] = f32x16{};

  const int64_t start = rp[m];
  const int nblk = (int)(rp[m + 1] - start);
  const int nsteps = SPB * nblk;
  const tsp::dma::i32x4 krs = tsp::dma::make_rsrc(K + hs, (uint32_t)(S * ROWB));
  const tsp::dma::i32x4 vrs = tsp::dma::make_rsrc(V + hs, (uint32_t)(S * ROWB));
  const uint32_t lds0 = tsp::dma::lds_addr(lds);

  int cbase = 0, cv = 0;
  auto load_cols = [&](int base) {
    const int i = base + lane < nblk ? base + lane : nblk - 1;
    return tsp::dma::load_lo32_sync(ci + start + i);
  };
  if (nblk > 0) cv = load_cols(0);
  auto colblk = [&](int blk) {
    if (blk - cbase >= 64) {
      cbase = blk & ~63;
      cv = load_cols(cbase);
    }
    return __builtin_amdgcn_readlane(cv, blk - cbase);
  };
  auto first_key = [&](int s) { return (int64_t)colblk(s / SPB) * BS + HR * (s % SPB); };
  auto issue = [&](int s) {
    const int64_t key0 = first_key(s);
    const uint32_t st = lds0 + (s % NST) * STAGE;
    abf::dma_rows<D>(krs, key0, st, w, lane);
    abf::dma_rows<D>(vrs, key0, st + HBYTES, w, lane);
  };

  const int kx = l32 & 15;
  auto compute = [&](const uint8_t* st, int64_t key0) {
    const uint8_t* Ks = st;
    const uint8_t* Vs = st + HBYTES;
    f32x16 sc[NT], dp[NT];
    f32x4 ka[2][NT], va[2][NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      ka[0][tt] = abf::chunk_read<D>(Ks, 32 * tt + l32, h, kx);
      va[0][tt] = abf::chunk_read<D>(Vs, 32 * tt + l32, h, kx);
    }
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      if (t + 1 < KT) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
          ka[(t + 1) & 1][tt] = abf::chunk_read<D>(Ks, 32 * tt + l32, 2 * (t + 1) + h, kx);
          va[(t + 1) & 1][tt] = abf::chunk_read<D>(Vs, 32 * tt + l32, 2 * (t + 1) + h, kx);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
          const bool first = t == 0 && c == 0;
          sc[tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[t & 1][tt][c], qf[t][c], first ? f32x16{} : sc[tt], 0, 0, 0);
          dp[tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[t & 1][tt][c], dof[t][c], first ? f32x16{} : dp[tt], 0, 0, 0);
        }
    }
    // dS^T element v of tile tt: key key0 + 32 tt + 8 (v / 4) + 4 h + v % 4
    const bool tail = key0 + HR > S;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[tt][v], scale_log2, nr));
        if (tail && key0 + 32 * tt + 8 * (v >> 2) + 4 * h + (v & 3) >= S) p = 0.f;
        sc[tt][v] = p * (dp[tt][v] - Dq);
      }
    // dQ^T += K^T dS^T
    vrow_t kb[2];
    auto krow = [&](int i) { return abf::row_read<D>(Ks, 32 * (i >> 4) + 8 * ((i & 15) >> 2) + 4 * h + (i & 3), l32); };
    kb[0] = krow(0);
#pragma unroll
    for (int i = 0; i < 16 * NT; ++i) {
      if (i + 1 < 16 * NT) kb[(i + 1) & 1] = krow(i + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < NU; ++u)
        acc[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(kb[i & 1][u], sc[i >> 4][i & 15], acc[u], 0, 0, 0);
    }
  };

  if (nsteps > 0) issue(0);
  for (int s = 0; s < nsteps; ++s) {
    const int64_t key0 = first_key(s);
    tsp::dma::wait_vm<0>();
    tsp::dma::barrier();
    if (s + 1 < nsteps) issue(s + 1);
    compute(lds + (s % NST) * STAGE, key0);
  }
  abf::store_rows<D>(dQ + hs + q * D, acc, h, scale);
}

// Column pass: workgroup per (plan item, head), items heaviest first; an
// item is (key block column, range [p0, p1) of its column view, partial slot
// or -1). Wavefront w owns keys col * 128 + 32 w + [0, 32) with the K and V
// rows in registers. Per 32-query tile of a stored block row m < Mt: S =
// Q K^T and dP = dO V^T (Q, dO chunk reads), P and dS = P (dP - D) in place
// with the stats staged beside the rows, dV^T += dO^T P and dK^T += Q^T dS
// (dO, Q row reads). An item covering a whole column writes dK / dV, a
// segment of a split column writes fp32 partials summed by the reduce.
template <int D>
__global__ __launch_bounds__(256, 1) void bsa_bwd_dkdv_f32(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, int64_t S, int64_t H, const int64_t* __restrict__ crow,
    const int32_t* __restrict__ items, int n_partials, int64_t Mt, float scale_log2, float scale,
    const float* __restrict__ qstat, float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ partial) {
  typedef abf::Cfg<D> C;
  constexpr int BS = C::BS, HR = C::HR, ROWB = C::ROWB, HBYTES = C::HBYTES, NT = C::NT, NU = C::NU, KT = C::KT;
  constexpr int SPB = C::SPB, STAGE = 2 * HBYTES + 1024, NST = 2;  // Q rows, dO rows, stats (r[HR], D[HR])
  typedef typename abf::VRow<NU>::type vrow_t;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];

  const int64_t it = blockIdx.x / H, head = blockIdx.x % H;
  const int col = items[4 * it], p0 = items[4 * it + 1], p1 = items[4 * it + 2], pslot = items[4 * it + 3];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t hs = head * S * D, HS = H * S;
  const int64_t key = (int64_t)col * BS + w * 32 + l32;
  const bool kvalid = key < S;

  f32x4 kf[KT], vf[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    kf[t] = kvalid ? *(const f32x4*)(K + hs + key * D + 8 * t + 4 * h) : f32x4{};
    vf[t] = kvalid ? *(const f32x4*)(V + hs + key * D + 8 * t + 4 * h) : f32x4{};
  }
  f32x16 dk[NU], dv[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) dk[u] = dv[u] = f32x16{};

  const int nblk = p1 - p0;
  const int nsteps = SPB * nblk;
  const tsp::dma::i32x4 qrs = tsp::dma::make_rsrc(Q + hs, (uint32_t)(S * ROWB));
  const tsp::dma::i32x4 ors = tsp::dma::make_rsrc(dO + hs, (uint32_t)(S * ROWB));
  const uint32_t lds0 = tsp::dma::lds_addr(lds);

  // block rows of the item, 64 at a time in one VGPR, read with readlane
  int rbase = 0, rv = 0;
  auto load_rows = [&](int base) {
    const int i = base + lane < nblk ? base + lane : nblk - 1;
    return tsp::dma::load_lo32_sync(crow + p0 + i);
  };
  if (nblk > 0) rv = load_rows(0);
  auto rowblk = [&](int i) {
    if (i - rbase >= 64) {
      rbase = i & ~63;
      rv = load_rows(rbase);
    }
    return (int64_t)__builtin_amdgcn_readlane(rv, i - rbase);
  };
  // stage s: block row rowblk(s / SPB) (skipped when >= Mt: no forward
  // queries), queries from m * 128 + HR * (s % SPB)
  auto issue = [&](int s, int64_t mrow) {
    if (mrow >= Mt) return;
    const int64_t q0 = mrow * BS + HR * (s % SPB);
    const uint32_t st = lds0 + (s % NST) * STAGE;
    abf::dma_rows<D>(qrs, q0, st, w, lane);
    abf::dma_rows<D>(ors, q0, st + HBYTES, w, lane);
    if (w == 0) {  // lanes [0, HR/4): r, the rest D (the lanes past 2 HR / 4 repeat D)
      constexpr int LPP = HR / 4;
      const int plane = lane >= LPP ? 1 : 0;
      tsp::dma::global16(qstat + plane * HS + head * S + q0 + 4 * (lane % LPP), st + 2 * HBYTES);
    }
  };

  const int kx = l32 & 15;
  auto compute = [&](const uint8_t* st) {
    const uint8_t* Qs = st;
    const uint8_t* Os = st + HBYTES;
    const float* stats = (const float*)(st + 2 * HBYTES);
    f32x16 sc[NT], dp[NT];
    f32x4 qa[2][NT], oa[2][NT];
#pragma unroll
    for (int qt = 0; qt < NT; ++qt) {
      qa[0][qt] = abf::chunk_read<D>(Qs, 32 * qt + l32, h, kx);
      oa[0][qt] = abf::chunk_read<D>(Os, 32 * qt + l32, h, kx);
    }
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      if (t + 1 < KT) {
#pragma unroll
        for (int qt = 0; qt < NT; ++qt) {
          qa[(t + 1) & 1][qt] = abf::chunk_read<D>(Qs, 32 * qt + l32, 2 * (t + 1) + h, kx);
          oa[(t + 1) & 1][qt] = abf::chunk_read<D>(Os, 32 * qt + l32, 2 * (t + 1) + h, kx);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int qt = 0; qt < NT; ++qt) {
          const bool first = t == 0 && c == 0;
          sc[qt] = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[t & 1][qt][c], kf[t][c], first ? f32x16{} : sc[qt], 0, 0, 0);
          dp[qt] = __builtin_amdgcn_mfma_f32_32x32x2f32(oa[t & 1][qt][c], vf[t][c], first ? f32x16{} : dp[qt], 0, 0, 0);
        }
    }
    // P and dS element v of tile qt: query 32 qt + 8 (v / 4) + 4 h + v % 4 of the stage
#pragma unroll
    for (int qt = 0; qt < NT; ++qt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const f32x4 r4 = *(const f32x4*)(stats + 32 * qt + 8 * a + 4 * h);
        const f32x4 d4 = *(const f32x4*)(stats + HR + 32 * qt + 8 * a + 4 * h);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int v = 4 * a + c;
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[qt][v], scale_log2, -r4[c]));
          sc[qt][v] = p;
          dp[qt][v] = p * (dp[qt][v] - d4[c]);
        }
      }
    // dV^T += dO^T P, dK^T += Q^T dS
    vrow_t ob[2], qb[2];
    auto rowof = [&](int i) { return 32 * (i >> 4) + 8 * ((i & 15) >> 2) + 4 * h + (i & 3); };
    ob[0] = abf::row_read<D>(Os, rowof(0), l32);
    qb[0] = abf::row_read<D>(Qs, rowof(0), l32);
#pragma unroll
    for (int i = 0; i < 16 * NT; ++i) {
      if (i + 1 < 16 * NT) {
        ob[(i + 1) & 1] = abf::row_read<D>(Os, rowof(i + 1), l32);
        qb[(i + 1) & 1] = abf::row_read<D>(Qs, rowof(i + 1), l32);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        dv[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(ob[i & 1][u], sc[i >> 4][i & 15], dv[u], 0, 0, 0);
        dk[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(qb[i & 1][u], dp[i >> 4][i & 15], dk[u], 0, 0, 0);
      }
    }
  };

  if (nsteps > 0) issue(0, rowblk(0));
  for (int s = 0; s < nsteps; ++s) {
    const int64_t mrow = rowblk(s / SPB);
    tsp::dma::wait_vm<0>();
    tsp::dma::barrier();
    if (s + 1 < nsteps) issue(s + 1, rowblk((s + 1) / SPB));
    if (mrow < Mt) compute(lds + (s % NST) * STAGE);
  }

  if (pslot < 0) {
    if (kvalid) {
      abf::store_rows<D>(dK + hs + key * D, dk, h, scale);
      abf::store_rows<D>(dV + hs + key * D, dv, h, 1.f);
    }
  } else {
    float* pk = partial + (((int64_t)head * n_partials + pslot) * 2) * (BS * D) + (w * 32 + l32) * D;
    abf::store_rows<D>(pk, dk, h, scale);
    abf::store_rows<D>(pk + BS * D, dv, h, 1.f);
  }
}

// dK / dV of the split columns in fp32: sum of the segments' partials in
// segment order (deterministic). Workgroup per (split, 16-key chunk, head);
// thread per 4 consecutive head_dim values of one key of dK or dV.
template <int D>
__global__ __launch_bounds__(256) void bsa_bwd_reduce_f32(const int32_t* __restrict__ splits, int n_partials, int64_t S,
                                                          const float* __restrict__ partial, float* __restrict__ dK,
                                                          float* __restrict__ dV) {
  constexpr int BS = 128;
  const int sp = blockIdx.x >> 3, chunk = blockIdx.x & 7;
  const int64_t head = blockIdx.y;
  const int col = splits[4 * sp], slot0 = splits[4 * sp + 1], nseg = splits[4 * sp + 2];
  const float* base = partial + (head * n_partials + slot0) * 2 * (BS * D);
#pragma unroll
  for (int e0 = 0; e0 < 2 * 16 * (D / 4); e0 += 256) {
    const int e = e0 + threadIdx.x;
    const int which = e / (16 * (D / 4));
    const int r = chunk * 16 + (e / (D / 4)) % 16, d4 = e % (D / 4);
    const int64_t key = (int64_t)col * BS + r;
    if (key >= S) continue;
    f32x4 sum = f32x4{};
    for (int j = 0; j < nseg; ++j) sum += *(const f32x4*)(base + (j * 2 + which) * (BS * D) + r * D + 4 * d4);
    *(f32x4*)((which ? dV : dK) + (head * S + key) * D + 4 * d4) = sum;
  }
}

template <int D>
int launch_f32(const void* Q, const void* K, const void* V, const void* O, const void* dO, int64_t H, int64_t S,
               const int64_t* rp, const int64_t* ci, const int64_t* crow, int64_t Mt, double scale,
               const void* rmax, const void* rden, void* dQ, void* dK, void* dV, const int32_t* plan, int64_t n_items,
               int64_t n_splits, int64_t n_partials, void* workspace, hipStream_t st) {
  const int64_t nh = tsp::ceil_div(H, 8);
  const int64_t grid_a = nh * Mt * 8 * (D == 256 ? 2 : 1), grid_b = n_items * H * (D == 256 ? 2 : 1);
  if (grid_a > INT32_MAX || grid_b > INT32_MAX || 8 * n_splits > INT32_MAX || H > 65535)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_bwd: problem too large");
  const float sl2 = (float)(scale * 1.4426950408889634);
  float* qstat = (float*)workspace;
  float* partial = (float*)((char*)workspace + 16 * H * S);
  if (Mt * 128 < S) {  // rows without a block row: zero dQ
    const int64_t tail = (S - Mt * 128) * D * 4;
    for (int64_t hh = 0; hh < H; ++hh) {
      int rc = tsp::zero_fill((char*)dQ + (hh * S + Mt * 128) * D * 4, tail, st);
      if (rc) return rc;
    }
  }
  if constexpr (D == 256) {  // 16-row tiles, half a block per workgroup (attention_bwd_d256.hip)
    int rc = tsp::bsa_bwd_f32_d256_rows((const float*)Q, (const float*)K, (const float*)V, (const float*)O,
                                      (const float*)dO, S, H, rp, ci, Mt, sl2, (float)scale, (const float*)rmax,
                                      (const float*)rden, qstat, (float*)dQ, st);
    if (rc) return rc;
    rc = tsp::bsa_bwd_f32_d256_cols((const float*)Q, (const float*)K, (const float*)V, (const float*)dO, S, H, crow,
                                    plan + 4, n_items, (int)n_partials, Mt, sl2, (float)scale, (const float*)qstat,
                                    (float*)dK, (float*)dV, partial, st);
    if (rc) return rc;
  } else {
    if (grid_a > 0) {
      hipLaunchKernelGGL((bsa_bwd_dq_f32<D>), dim3((unsigned)grid_a), dim3(256), 0, st, (const float*)Q,
                         (const float*)K, (const float*)V, (const float*)O, (const float*)dO, S, H, rp, ci, Mt, sl2,
                         (float)scale, (const float*)rmax, (const float*)rden, qstat, (float*)dQ);
      int rc = tsp::check_launch("bsa_bwd_dq_f32 launch");
      if (rc) return rc;
    }
    if (grid_b > 0) {
      hipLaunchKernelGGL((bsa_bwd_dkdv_f32<D>), dim3((unsigned)grid_b), dim3(256), 0, st, (const float*)Q,
                         (const float*)K, (const float*)V, (const float*)dO, S, H, crow, plan + 4, (int)n_partials, Mt,
                         sl2, (float)scale, (const float*)qstat, (float*)dK, (float*)dV, partial);
      int rc = tsp::check_launch("bsa_bwd_dkdv_f32 launch");
      if (rc) return rc;
    }
  }
  if (n_splits > 0) {
    hipLaunchKernelGGL((bsa_bwd_reduce_f32<D>), dim3((unsigned)(8 * n_splits), (unsigned)H), dim3(256), 0, st,
                       plan + 4 + 4 * n_items, (int)n_partials, S, (const float*)partial, (float*)dK, (float*)dV);
    int rc = tsp::check_launch("bsa_bwd_reduce_f32 launch");
    if (rc) return rc;
  }
  return TSP_OK;
}

}  // namespace

// Host-side plan of the column pass. Items cover every key block column
// c < ceil(seq_len / block_size) (columns without stored blocks write zeros);
// a column with more than L stored block rows is cut into ceil(n / L) nearly
// equal segments with partial slots 0, 1, ... in column order. L follows the
// work per CU (n_heads * blocks / 256 CUs, halved, clamped to [4, 64]) so
// that no single item dominates. Items are sorted heaviest first (ties by
// column). Layout (int32): n_items, n_splits, n_partials, L; items
// (col, p_begin, p_end, slot or -1) x n_items; splits (col, slot0, n_seg, 0)
// x n_splits.
extern "C" int64_t tsp_bsa_bwd_plan(const int64_t* col_ptrs, int64_t n_block_cols, int64_t n_heads, int64_t seq_len,
                                    int64_t block_size, int32_t* plan, int64_t capacity) {
  if (n_block_cols < 0 || n_heads < 0 || seq_len < 0 || block_size <= 0 || (n_block_cols > 0 && !col_ptrs)) {
    tsp::fail(TSP_EINVAL, "tsp_bsa_bwd_plan: bad argument");
    return -1;
  }
  const int64_t ncols = tsp::ceil_div(seq_len, block_size);
  int64_t nnzb = 0;
  for (int64_t c = 0; c < ncols && c < n_block_cols; ++c) nnzb += col_ptrs[c + 1] - col_ptrs[c];
  if (n_block_cols > 0 && col_ptrs[n_block_cols] > INT32_MAX) {
    tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_bwd_plan: too many blocks");
    return -1;
  }
  int64_t L = (int64_t)((double)n_heads * (double)nnzb / 256.0 / 2.0 + 0.999);
  L = L < 4 ? 4 : (L > abw::SEG_MAX ? abw::SEG_MAX : L);
  struct Item { int32_t col, p0, p1, slot, weight; };
  // no exception crosses the C ABI: allocation failure is a status
  Item* items = new (std::nothrow) Item[ncols + nnzb / L + 1];
  int32_t* splits = new (std::nothrow) int32_t[4 * (nnzb / (L + 1) + 1)];
  if (!items || !splits) {
    delete[] items;
    delete[] splits;
    tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_bwd_plan: host memory for %lld items", (long long)(ncols + nnzb / L + 1));
    return -1;
  }
  int64_t ni = 0, ns = 0, np = 0;
  for (int64_t c = 0; c < ncols; ++c) {
    const int64_t b0 = c < n_block_cols ? col_ptrs[c] : 0;
    const int64_t n = c < n_block_cols ? col_ptrs[c + 1] - b0 : 0;
    if (n <= L) {
      items[ni++] = Item{(int32_t)c, (int32_t)b0, (int32_t)(b0 + n), -1, (int32_t)n};
      continue;
    }
    const int64_t nseg = (n + L - 1) / L, base = n / nseg, rem = n % nseg;
    splits[4 * ns] = (int32_t)c;
    splits[4 * ns + 1] = (int32_t)np;
    splits[4 * ns + 2] = (int32_t)nseg;
    splits[4 * ns + 3] = 0;
    ++ns;
    int64_t p = b0;
    for (int64_t j = 0; j < nseg; ++j) {
      const int64_t len = base + (j < rem ? 1 : 0);
      items[ni++] = Item{(int32_t)c, (int32_t)p, (int32_t)(p + len), (int32_t)(np + j), (int32_t)len};
      p += len;
    }
    np += nseg;
  }
  // heaviest first, stable in column order (insertion into weight buckets)
  const int64_t need = 4 + 4 * ni + 4 * ns;
  if (plan && capacity >= need) {
    plan[0] = (int32_t)ni;
    plan[1] = (int32_t)ns;
    plan[2] = (int32_t)np;
    plan[3] = (int32_t)L;
    int64_t o = 4;
    for (int64_t wgt = L; wgt >= 0; --wgt)
      for (int64_t i = 0; i < ni; ++i)
        if (items[i].weight == wgt) {
          plan[o++] = items[i].col;
          plan[o++] = items[i].p0;
          plan[o++] = items[i].p1;
          plan[o++] = items[i].slot;
        }
    for (int64_t i = 0; i < 4 * ns; ++i) plan[o++] = splits[i];
  }
  delete[] items;
  delete[] splits;
  return need;
}

extern "C" int64_t tsp_bsa_bwd_workspace_size(int64_t n_heads, int64_t seq_len, int64_t head_dim, int64_t n_partials) {
  if (n_heads < 0 || seq_len < 0 || head_dim < 0 || n_partials < 0) return -1;
  const int64_t pd = head_dim > abw::D ? head_dim : abw::D;  // fp32 partial rows of dK and dV
  return 16 * n_heads * seq_len + n_heads * n_partials * 2 * abw::BS * pd * 4;
}

extern "C" int tsp_bsa_bwd(const void* Q, const void* K, const void* V, const void* O, const void* dO, int dtype,
                           int64_t n_heads, int64_t seq_len, int64_t head_dim, const int64_t* block_row_ptrs,
                           const int64_t* block_col_indices, const int64_t* col_ptrs, const int64_t* col_block_rows,
                           int64_t n_block_cols, int64_t block_size, double scale, const void* row_max,
                           const void* row_denom, void* dQ, void* dK, void* dV, const int32_t* plan, int64_t n_items,
                           int64_t n_splits, int64_t n_partials, void* workspace, void* stream) {
  if (dtype != TSP_F32 && dtype != TSP_F64 && dtype != TSP_BF16)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_bwd: dtype %d not supported", dtype);
  if (n_heads < 0 || seq_len < 0 || head_dim < 0 || block_size <= 0 || n_block_cols < 0 || n_items < 0 ||
      n_splits < 0 || n_partials < 0)
    return tsp::fail(TSP_EINVAL, "tsp_bsa_bwd: bad size");
  if (n_heads == 0 || seq_len == 0 || head_dim == 0) return TSP_OK;
  if (!Q || !K || !V || !O || !dO || !block_row_ptrs || !block_col_indices || !col_ptrs || !col_block_rows || !row_max ||
      !row_denom || !dQ || !dK || !dV || !workspace)
    return tsp::fail(TSP_EINVAL, "tsp_bsa_bwd: null pointer");
  hipStream_t stream_ = (hipStream_t)stream;
  const int64_t Mt = seq_len / block_size;
  const int64_t rows = n_heads * seq_len;

  const bool aligned = ((uintptr_t)Q % 16) == 0 && ((uintptr_t)K % 16) == 0 && ((uintptr_t)V % 16) == 0 &&
                       ((uintptr_t)O % 16) == 0 && ((uintptr_t)dO % 16) == 0 && ((uintptr_t)dQ % 8) == 0 &&
                       ((uintptr_t)dK % 8) == 0 && ((uintptr_t)dV % 8) == 0 && ((uintptr_t)workspace % 16) == 0;
  if (dtype == TSP_BF16 && block_size == abw::BS && head_dim == abw::D && scale > 0 && plan && aligned &&
      (seq_len + abw::BS) * abw::ROWB <= (int64_t)UINT32_MAX) {
    if (n_items < tsp::ceil_div(seq_len, block_size))
      return tsp::fail(TSP_EINVAL, "tsp_bsa_bwd: plan has %lld items for %lld key block columns", (long long)n_items,
                       (long long)tsp::ceil_div(seq_len, block_size));
    const int64_t nh = tsp::ceil_div(n_heads, 8);
    const int64_t grid_a = nh * Mt * 8;
    if (grid_a > INT32_MAX || n_items * nh > INT32_MAX || 8 * n_splits > INT32_MAX || n_heads > 65535)
      return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_bwd: problem too large");
    const float sl2 = (float)(scale * 1.4426950408889634);
    float* qstat = (float*)workspace;
    float* partial = (float*)((char*)workspace + 16 * rows);
    if (Mt * block_size < seq_len) {  // rows without a block row: zero dQ
      const int64_t tail = (seq_len - Mt * block_size) * head_dim * 2;
      for (int64_t hh = 0; hh < n_heads; ++hh) {
        int rc = tsp::zero_fill((char*)dQ + (hh * seq_len + Mt * block_size) * head_dim * 2, tail, stream_);
        if (rc) return rc;
      }
    }
    if (grid_a > 0) {
      hipLaunchKernelGGL(bsa_bwd_dq_bf16_d128, dim3((unsigned)grid_a), dim3(256), 0, stream_, (const uint16_t*)Q,
                         (const uint16_t*)K, (const uint16_t*)V, (const uint16_t*)O, (const uint16_t*)dO, seq_len,
                         n_heads, block_row_ptrs, block_col_indices, Mt, sl2, (float)scale, (const float*)row_max,
                         (const float*)row_denom, qstat, (uint16_t*)dQ);
      int rc = tsp::check_launch("bsa_bwd_dq_bf16_d128 launch");
      if (rc) return rc;
    }
    if (n_items > 0) {
      const int64_t nslots = n_items * nh;
      const int64_t g8 = nslots < 32 ? nslots : 32;
      hipLaunchKernelGGL(bsa_bwd_dkdv_bf16_d128, dim3((unsigned)(8 * g8)), dim3(256), 0, stream_, (const uint16_t*)Q,
                         (const uint16_t*)K, (const uint16_t*)V, (const uint16_t*)dO, seq_len, n_heads, (int)nh,
                         col_block_rows, plan + 4, (int)n_items, (int)n_partials, sl2, (float)scale,
                         (const float*)qstat, (uint16_t*)dK, (uint16_t*)dV, partial);
      int rc = tsp::check_launch("bsa_bwd_dkdv_bf16_d128 launch");
      if (rc) return rc;
    }
    if (n_splits > 0) {
      hipLaunchKernelGGL(bsa_bwd_reduce, dim3((unsigned)(8 * n_splits), (unsigned)n_heads), dim3(256), 0, stream_,
                         plan + 4 + 4 * n_items, (int)n_partials, seq_len, (const float*)partial, (uint16_t*)dK,
                         (uint16_t*)dV);
      int rc = tsp::check_launch("bsa_bwd_reduce launch");
      if (rc) return rc;
    }
    return TSP_OK;
  }

  const bool aligned16 = aligned && ((uintptr_t)dQ % 16) == 0 && ((uintptr_t)dK % 16) == 0 && ((uintptr_t)dV % 16) == 0;
  if (dtype == TSP_F32 && block_size == 128 && (head_dim == 64 || head_dim == 128 || head_dim == 256) && scale > 0 &&
      plan && aligned16 &&
      (seq_len + 128) * head_dim * 4 <= (int64_t)UINT32_MAX) {
    if (n_items < tsp::ceil_div(seq_len, block_size))
      return tsp::fail(TSP_EINVAL, "tsp_bsa_bwd: plan has %lld items for %lld key block columns", (long long)n_items,
                       (long long)tsp::ceil_div(seq_len, block_size));
    if (head_dim == 256)
      return launch_f32<256>(Q, K, V, O, dO, n_heads, seq_len, block_row_ptrs, block_col_indices, col_block_rows, Mt,
                             scale, row_max, row_denom, dQ, dK, dV, plan, n_items, n_splits, n_partials, workspace,
                             stream_);
    if (head_dim == 128)
      return launch_f32<128>(Q, K, V, O, dO, n_heads, seq_len, block_row_ptrs, block_col_indices, col_block_rows, Mt,
                             scale, row_max, row_denom, dQ, dK, dV, plan, n_items, n_splits, n_partials, workspace,
                             stream_);
    return launch_f32<64>(Q, K, V, O, dO, n_heads, seq_len, block_row_ptrs, block_col_indices, col_block_rows, Mt, scale,
                          row_max, row_denom, dQ, dK, dV, plan, n_items, n_splits, n_partials, workspace, stream_);
  }

  // D = rowsum(dO * O) into the workspace
  {
    const int64_t grid = tsp::ceil_div(rows, 4);
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_bwd: too many rows");
    if (dtype == TSP_F32)
      hipLaunchKernelGGL(bsa_bwd_d<float>, dim3((unsigned)grid), dim3(256), 0, stream_, (const float*)O, (const float*)dO,
                         rows, head_dim, (float*)workspace);
    else if (dtype == TSP_F64)
      hipLaunchKernelGGL(bsa_bwd_d<double>, dim3((unsigned)grid), dim3(256), 0, stream_, (const double*)O,
                         (const double*)dO, rows, head_dim, (double*)workspace);
    else
      hipLaunchKernelGGL(bsa_bwd_d<uint16_t>, dim3((unsigned)grid), dim3(256), 0, stream_, (const uint16_t*)O,
                         (const uint16_t*)dO, rows, head_dim, (float*)workspace);
    int rc = tsp::check_launch("bsa_bwd_d launch");
    if (rc) return rc;
  }
  if (dtype == TSP_F64)
    return launch_generic<double>(Q, K, V, dO, n_heads, seq_len, head_dim, block_row_ptrs, block_col_indices, col_ptrs,
                                  col_block_rows, n_block_cols, block_size, Mt, scale, row_max, row_denom, workspace, dQ, dK, dV,
                                  stream_);
  if (dtype == TSP_F32)
    return launch_generic<float>(Q, K, V, dO, n_heads, seq_len, head_dim, block_row_ptrs, block_col_indices, col_ptrs,
                                 col_block_rows, n_block_cols, block_size, Mt, scale, row_max, row_denom, workspace, dQ, dK, dV, stream_);
  return launch_generic<uint16_t>(Q, K, V, dO, n_heads, seq_len, head_dim, block_row_ptrs, block_col_indices, col_ptrs,
                                  col_block_rows, n_block_cols, block_size, Mt, scale, row_max, row_denom, workspace, dQ, dK, dV,
                                  stream_);
}
