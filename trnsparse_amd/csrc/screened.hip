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
//   screened_f32_dma    fp32, 128x128 C tile per workgroup, streamed MFMA
//                       structure (direct-to-LDS slab ring, 64x64 wave
//                       tiles); the mask multiplies the A fragments after
//                       their LDS read; the K loop visits active k-tiles.
//   screened_f32_mfma   the register-staged variant on the shared MFMA core
//                       (mfma_f32.h), for operands past 4 GiB.
//   screened_f64_dma    fp64 (even m and strides): the same structure on
//                       v_mfma_f64_16x16x4_f64 (mfma_f64.h operand tiles).
//   screened_generic    other or unaligned operands: one thread per output.
//   screened_bwd_a_f32 / screened_bwd_b_f32 / screened_bwd_*_generic
//                       the backward (below).
#include <atomic>

#include "lds_dma.h"
#include "mfma_f32.h"
#include "mfma_f64.h"
#include "f32_pair_tiles.h"

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
  if (i < m) q = qsqrt<QT>(diag[i]);
  Q[i] = q;  // rows past m (the last tile's tail) hold 0: every workspace word is written
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

// screened_f32_dma<QT>: fp32 A and B, the streamed MFMA structure of
// bsr_spmm_f32_dma (4 waves of 64x64 with four 32x32x2 accumulators each,
// 64-wide k-slabs of A [128][64] and B [64][128] through a 2-stage LDS ring
// by direct global->LDS buffer loads, one slab ahead; rows and columns past
// m read as zero). The mask cannot be applied while staging, so it is
// applied to the A fragments after their LDS read: a * (Q_i*Q_k > thr ? 1 : 0)
// in diag's precision, with Q_k of the slab staged in LDS next to the ring.
// As there, a wave's two column subtiles interleave (columns 2j + u) so one
// 8-byte B read feeds both and C is stored in 8-byte pairs.
namespace sdma {
constexpr int KROWB = TILE * 4;        // B tile rows: 512 B
constexpr uint32_t OOB = 0xFFFFFFF0u;
}  // namespace sdma

template <typename QT, int SKC>
__global__ __launch_bounds__(256) void screened_f32_dma(
    const float* __restrict__ A, int64_t lda, const QT* __restrict__ Q, const QT* __restrict__ qmax, QT thr,
    int64_t m, const float* __restrict__ B, int64_t ldb, int64_t ncols, float* __restrict__ C, int64_t ldc, int nmt,
    int nnt) {
  using sdma::KROWB;
  using sdma::OOB;
  constexpr int TROWB = SKC * 4;         // A tile rows
  constexpr int CPR = TROWB / 16;        // 16-byte chunks per A row
  constexpr int TBYTES = TILE * TROWB;   // A tile == B tile bytes
  constexpr int STAGE = 2 * TBYTES;
  constexpr int INS = TBYTES / 1024 / 4; // 1-KiB load instructions per wave per tile
  constexpr int ARPI = 1024 / TROWB;     // A rows per instruction
  // slot of logical chunk c in A row r: 16 consecutive rows of one b128 read
  // cover all 64 banks
  auto aswz = [](int c, int r) { return CPR == 16 ? (c ^ (r & 15)) : (c ^ ((r >> 1) & 7)); };
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];
  __shared__ __attribute__((aligned(16))) QT qs[2][SKC];
  int64_t mt64;
  int ntile;
  if (!T32::tile_item(blockIdx.x, nmt, nnt, nullptr, mt64, ntile)) return;
  const int mt = (int)mt64;
  const int64_t row0 = (int64_t)mt * TILE, n0 = (int64_t)ntile * TILE;
  const QT qI = qmax[mt];
  const int nkt = (int)tsp::ceil_div(m, TILE);
  auto active = [&](int t) { return qI * qmax[t] > thr; };
  int nact = 0;
  for (int t = 0; t < nkt; ++t) nact += active(t) ? 1 : 0;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;
  f32x16 acc[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) acc[t][u] = f32x16{};

  if (nact > 0) {
    const tsp::dma::i32x4 rsa = tsp::dma::make_rsrc(A, (uint32_t)(m * lda * 4));
    const tsp::dma::i32x4 rsb = tsp::dma::make_rsrc(B, (uint32_t)(m * ldb * 4));
    const uint32_t lds0 = tsp::dma::lds_addr(lds);
    const int arow = wm * 64 + l32;
    QT qrow[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) qrow[t] = row0 + arow + 32 * t < m ? Q[row0 + arow + 32 * t] : (QT)0;

    constexpr int SPT = TILE / SKC;  // slabs per k tile
    int kt_issue = -1;               // k tile of the slabs being issued (advanced in order)
    QT qnext = 0;
    auto issue = [&](int s) {
      if ((s % SPT) == 0) {
        ++kt_issue;
        while (!active(kt_issue)) ++kt_issue;
      }
      const int64_t k0 = (int64_t)kt_issue * TILE + (s % SPT) * SKC;
      const uint32_t st = lds0 + (s & 1) * STAGE;
#pragma unroll
      for (int q = 0; q < INS; ++q) {
        const int i = INS * w + q;
        const int r = ARPI * i + lane / CPR;
        const int c = aswz(lane % CPR, r);
        const int64_t col = k0 + c * 4;
        tsp::dma::buffer16(rsa, col < m ? (uint32_t)(((row0 + r) * lda + col) * 4) : OOB, st + i * 1024);
      }
#pragma unroll
      for (int q = 0; q < INS; ++q) {
        const int j = INS * w + q;
        const int rr = 2 * j + (lane >> 5);
        const int c = (lane & 31) ^ (8 * ((rr >> 2) & 1));
        tsp::dma::buffer16(rsb, (uint32_t)(((k0 + rr) * ldb + n0 + c * 4) * 4), st + TBYTES + j * 1024);
      }
      if (w == 0 && lane < SKC) qnext = k0 + lane < m ? Q[k0 + lane] : (QT)0;  // into qs before its barrier
    };
    // column subtile u holds columns wn*64 + 2*l32 + u: one 8-byte read of a
    // B row feeds both subtiles
    const int bc2 = wn * 64 + 2 * l32;
    const int boff2 = (((bc2 >> 2) ^ (8 * h)) * 16) + (bc2 & 3) * 4 + 4 * h * KROWB;
    struct Ops {
      float a[2][4];
      float b[2][4];
    };
    auto fetch = [&](const uint8_t* st, const QT* qk, int g, Ops& o) {
      QT kq[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) kq[s] = qk[8 * g + 4 * h + s];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int r = arow + 32 * t;
        const f32x4 v = *(const f32x4*)(st + r * TROWB + aswz(2 * g + h, r) * 16);
#pragma unroll
        for (int s = 0; s < 4; ++s) o.a[t][s] = v[s] * ((qrow[t] * kq[s] > thr) ? 1.0f : 0.0f);
      }
      const uint8_t* Bs = st + TBYTES + 8 * g * KROWB;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const f32x2 bb = *(const f32x2*)(Bs + s * KROWB + boff2);
        o.b[0][s] = bb[0];
        o.b[1][s] = bb[1];
      }
    };
    auto mma = [&](const Ops& o) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int u = 0; u < 2; ++u)
            acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.a[t][s], o.b[u][s], acc[t][u], 0, 0, 0);
    };

    const int nsteps = nact * SPT;
    issue(0);
    if (w == 0 && lane < SKC) qs[0][lane] = qnext;
    for (int s = 0; s < nsteps; ++s) {
      tsp::dma::wait_vm<0>();  // this wave's loads of slab s are done
      tsp::dma::barrier();     // slab s and its Q_k are visible; stage (s+1) % 2 is free
      if (s + 1 < nsteps) issue(s + 1);
      const uint8_t* st = lds + (s & 1) * STAGE;
      const QT* qk = qs[s & 1];
      Ops o[2];
      fetch(st, qk, 0, o[0]);
#pragma unroll
      for (int g = 0; g < SKC / 8; ++g) {
        if (g + 1 < SKC / 8) fetch(st, qk, g + 1, o[(g + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        mma(o[g & 1]);
      }
      if (w == 0 && lane < SKC && s + 1 < nsteps) qs[(s + 1) & 1][lane] = qnext;
    }
  }
  // lane holds rows 8*(v/4) + 4*h + v%4 of columns wn*64 + 2*l32 + u
  const int64_t c = n0 + wn * 64 + 2 * l32;
  const bool pair = c + 1 < ncols && (ldc & 1) == 0 && ((uintptr_t)C & 7) == 0;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t r0 = row0 + wm * 64 + 32 * t + 4 * h;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t r = r0 + 8 * (v >> 2) + (v & 3);
      if (r < m) {
        if (pair) {
          *(f32x2*)(C + r * ldc + c) = f32x2{acc[t][0][v], acc[t][1][v]};
        } else {
          if (c < ncols) C[r * ldc + c] = acc[t][0][v];
          if (c + 1 < ncols) C[r * ldc + c + 1] = acc[t][1][v];
        }
      }
    }
  }
}

// screened_f64_dma<QT>: fp64 A and B on v_mfma_f64_16x16x4_f64 with the
// operand tiles of mfma_f64.h (4 waves of 64x64; A as a ROW tile [128][32]
// of the C tile's rows, B as a COL tile [32][128]; 32-wide k-slabs through a
// 2-stage direct-load ring, four per active k tile; A columns and B rows at
// or past m read as zero). As in the fp32 kernel the mask multiplies the A
// fragments after their LDS read, with Q_k of each slab staged in LDS.
template <typename QT>
__global__ __launch_bounds__(256) void screened_f64_dma(
    const double* __restrict__ A, int64_t lda, const QT* __restrict__ Q, const QT* __restrict__ qmax, QT thr,
    int64_t m, const double* __restrict__ B, int64_t ldb, int64_t ncols, double* __restrict__ C, int64_t ldc, int nmt,
    int nnt) {
  namespace F = tsp::f64tile;
  constexpr int STAGE = 2 * F::TILE;
  constexpr int SPT = TILE / F::KC;  // slabs per k tile
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];
  __shared__ __attribute__((aligned(16))) QT qs[2][F::KC];
  int64_t mt64;
  int ntile;
  if (!T32::tile_item(blockIdx.x, nmt, nnt, nullptr, mt64, ntile)) return;
  const int mt = (int)mt64;
  const int64_t row0 = (int64_t)mt * TILE, n0 = (int64_t)ntile * TILE;
  const QT qI = qmax[mt];
  const int nkt = (int)tsp::ceil_div(m, TILE);
  auto active = [&](int t) { return qI * qmax[t] > thr; };
  int nact = 0;
  for (int t = 0; t < nkt; ++t) nact += active(t) ? 1 : 0;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, g = lane >> 4, l16 = lane & 15;
  F::f64x4 acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = F::f64x4{};

  if (nact > 0) {
    const tsp::dma::i32x4 rsa = tsp::dma::make_rsrc(A, (uint32_t)(m * lda * 8));
    const tsp::dma::i32x4 rsb = tsp::dma::make_rsrc(B, (uint32_t)(m * ldb * 8));
    const uint32_t lds0 = tsp::dma::lds_addr(lds);
    QT qrow[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int64_t r = row0 + wm * 64 + 16 * t + l16;
      qrow[t] = r < m ? Q[r] : (QT)0;
    }
    int kt_issue = -1;  // k tile of the slabs being issued (advanced in order)
    QT qnext = 0;
    auto issue = [&](int s) {
      if ((s % SPT) == 0) {
        ++kt_issue;
        while (!active(kt_issue)) ++kt_issue;
      }
      const int64_t k0 = (int64_t)kt_issue * TILE + (s % SPT) * F::KC;
      const uint32_t st = lds0 + (s & 1) * STAGE;
      F::dma_row(rsa, row0, lda, k0, m, st, w, lane);
      F::dma_col(rsb, k0, ldb, n0, st + F::TILE, w, lane);
      if (w == 0 && lane < F::KC) qnext = k0 + lane < m ? Q[k0 + lane] : (QT)0;  // into qs before its barrier
    };
    const int nsteps = nact * SPT;
    issue(0);
    if (w == 0 && lane < F::KC) qs[0][lane] = qnext;
    for (int s = 0; s < nsteps; ++s) {
      tsp::dma::wait_vm<0>();  // this wave's loads of slab s are done
      tsp::dma::barrier();     // slab s and its Q_k are visible; stage (s+1) % 2 is free
      if (s + 1 < nsteps) issue(s + 1);
      const uint8_t* st = lds + (s & 1) * STAGE;
      const QT* qk = qs[s & 1];
      struct Ops {
        double a[4][2], b[4][2];
      };
      auto get = [&](int p, Ops& o) {
        F::fetch<true>(st, wm * 64, p, lane, o.a);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const QT q = qk[8 * g + 2 * p + k];
#pragma unroll
          for (int t = 0; t < 4; ++t) o.a[t][k] *= (qrow[t] * q > thr) ? 1.0 : 0.0;
        }
        F::fetch<false>(st + F::TILE, wn * 64, p, lane, o.b);
      };
      Ops o[2];
      get(0, o[0]);
#pragma unroll
      for (int p = 0; p < F::KC / 8; ++p) {
        if (p + 1 < F::KC / 8) get(p + 1, o[(p + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        F::mma(o[p & 1].a, o[p & 1].b, acc);
      }
      if (w == 0 && lane < F::KC && s + 1 < nsteps) qs[(s + 1) & 1][lane] = qnext;
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t c = n0 + wn * 64 + 16 * u + l16;
      if (c < ncols) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t r = row0 + wm * 64 + 16 * t + g + 4 * v;
          if (r < m) C[r * ldc + c] = acc[t][u][v];
        }
      }
    }
}

#ifndef SCREENED_KC
#define SCREENED_KC 32
#endif

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

// ---------------------------------------------------------------- backward
//
// The reference backward (trnsparse/nki/dispatch.py:478-484) materialises
// the mask and runs two dense products:
//   dA = (dC @ B^T) * mask            dB = (A * mask)^T @ dC
// Neither the mask nor A * mask is formed here; both products skip the
// 128x128 tile pairs (I, J) with fl(Qmax_I * Qmax_J) <= thr, where every
// pair is masked (the forward's tile skip, with the same caveat for
// non-finite entries inside such a tile):
//   screened_bwd_a_f32   dA tile (I, J) per workgroup. A masked pair writes
//       zeros; the others run the BSR backward's SDDMM engine (row tiles of
//       dC and B, k = the N columns, f32_pair_tiles.h) and the mask
//       multiplies each result in the epilogue (v * 1 or v * 0, the
//       reference's product with the float mask).
//   screened_bwd_b_f32   dB tile (rows J = columns of A, a 128-column tile
//       of N) per workgroup, walking the row tiles I of A active with J: the
//       A tile [k = rows i][columns] is the A^T operand (k tile reads),
//       masked after its LDS read with Q_i of the slab staged beside the
//       ring; dC rows of I are the [k][n] operand.
//   screened_bwd_a_generic / screened_bwd_b_generic   fp64 and operands the
//       streamed kernels do not take: one thread per output.
namespace P = tsp::f32pair;

template <typename QT>
__global__ __launch_bounds__(256) void screened_bwd_a_f32(const float* __restrict__ G, int64_t ldg,
                                                          const float* __restrict__ B, int64_t ldb, int64_t ncols,
                                                          const QT* __restrict__ Q, const QT* __restrict__ qmax,
                                                          QT thr, int64_t m, int nmt, float* __restrict__ dA,
                                                          int64_t ldda) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[P::NST * P::STAGE];
  // XCD-aware: XCD x takes a contiguous range of tiles, so the tiles of one
  // row tile I share its dC panel in that XCD's L2
  const int64_t ntiles = (int64_t)nmt * nmt;
  const int64_t gid = blockIdx.x, xcd = gid & 7, slot = gid >> 3;
  const int64_t per = tsp::ceil_div(ntiles, 8);
  const int64_t tix = xcd * per + slot;
  if (slot >= per || tix >= ntiles) return;
  const int I = (int)(tix / nmt), J = (int)(tix % nmt);
  const int64_t r0 = (int64_t)I * TILE, c0 = (int64_t)J * TILE;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

  if (!(qmax[I] * qmax[J] > thr)) {
    // every pair of the tile is masked: zeros, 4 columns per thread, 8 rows per pass
    const int64_t c = c0 + 4 * (tid & 31);
    for (int rr = tid >> 5; rr < TILE; rr += 8) {
      const int64_t r = r0 + rr;
      if (r >= m) break;
      float* p = dA + r * ldda + c;
      if (c + 3 < m && ((uintptr_t)p & 15) == 0) {
        *(f32x4*)p = f32x4{};
      } else {
        for (int e = 0; e < 4; ++e)
          if (c + e < m) p[e] = 0.f;
      }
    }
    return;
  }

  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;
  const P::i32x4 rsg = tsp::dma::make_rsrc(G, (uint32_t)(m * ldg * 4));
  const P::i32x4 rsb = tsp::dma::make_rsrc(B, (uint32_t)(m * ldb * 4));
  const uint32_t lds0 = tsp::dma::lds_addr(lds);
  auto issue = [&](int s) {
    const uint32_t st = lds0 + (s % P::NST) * P::STAGE;
    P::dma_row_tile(rsg, r0, ldg, (int64_t)s * P::KC, ncols, st, w, lane);
    P::dma_row_tile(rsb, c0, ldb, (int64_t)s * P::KC, ncols, st + P::TILE, w, lane);
  };
  P::Acc4 acc;
  acc.zero();
  const int ar = wm * 64 + l32, br = wn * 64 + l32;
  struct Ops {
    float x[2][4], y[2][4];
  };
  auto fetch = [&](const uint8_t* st, int gg, Ops& o) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const f32x4 a = P::frag_row(st, ar + 32 * t, gg, h);
      const f32x4 b = P::frag_row(st + P::TILE, br + 32 * t, gg, h);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        o.x[t][s] = a[s];
        o.y[t][s] = b[s];
      }
    }
  };
  const int nsteps = (int)tsp::ceil_div(ncols, P::KC);
  if (nsteps > 0) issue(0);
  for (int s = 0; s < nsteps; ++s) {
    tsp::dma::wait_vm<0>();
    tsp::dma::barrier();
    if (s + 1 < nsteps) issue(s + 1);
    const uint8_t* st = lds + (s % P::NST) * P::STAGE;
    Ops o[2];
    fetch(st, 0, o[0]);
#pragma unroll
    for (int gg = 0; gg < P::KC / 8; ++gg) {
      if (gg + 1 < P::KC / 8) fetch(st, gg + 1, o[(gg + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      acc.mma(o[gg & 1].x, o[gg & 1].y);
    }
  }
  // lane holds column l32 of subtile u and rows 8*(v/4) + 4h + v%4 of subtile t;
  // Q is padded with zeros to whole tiles
  QT qc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) qc[u] = Q[c0 + wn * 64 + 32 * u + l32];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t r = r0 + wm * 64 + 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
      if (r >= m) continue;
      const QT qr = Q[r];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int64_t c = c0 + wn * 64 + 32 * u + l32;
        if (c < m) dA[r * ldda + c] = acc.a[t][u][v] * ((qr * qc[u] > thr) ? 1.0f : 0.0f);
      }
    }
}

template <typename QT>
__global__ __launch_bounds__(256) void screened_bwd_b_f32(const float* __restrict__ A, int64_t lda,
                                                          const float* __restrict__ G, int64_t ldg, int64_t ncols,
                                                          const QT* __restrict__ Q, const QT* __restrict__ qmax,
                                                          QT thr, int64_t m, int nmt, int nnt, float* __restrict__ dB,
                                                          int64_t lddb) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[P::NST * P::STAGE];
  __shared__ __attribute__((aligned(16))) QT qs[2][P::KC];
  // XCD-aware: the column tiles of one row tile J share an XCD (and A's panel in its L2)
  int64_t jt64;
  int ntile;
  if (!T32::tile_item(blockIdx.x, nmt, nnt, nullptr, jt64, ntile)) return;
  const int J = (int)jt64;
  const int64_t k0 = (int64_t)J * TILE, n0 = (int64_t)ntile * TILE;
  const QT qJ = qmax[J];
  auto active = [&](int t) { return qmax[t] * qJ > thr; };
  int nact = 0;
  for (int t = 0; t < nmt; ++t) nact += active(t) ? 1 : 0;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;
  P::Acc4 acc;
  acc.zero();
  // A^T operand: output rows (columns of A) ac2 + t; row subtile t holds rows wm*64 + 2i + t
  const int ac2 = wm * 64 + 2 * l32, bc2 = wn * 64 + 2 * l32;
  if (nact > 0) {
    const P::i32x4 rsa = tsp::dma::make_rsrc(A, (uint32_t)(m * lda * 4));
    const P::i32x4 rsg = tsp::dma::make_rsrc(G, (uint32_t)(m * ldg * 4));
    const uint32_t lds0 = tsp::dma::lds_addr(lds);
    QT qk[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) qk[t] = Q[k0 + ac2 + t];  // padded with zeros to whole tiles
    constexpr int SPT = TILE / P::KC;  // slabs per row tile
    int it_issue = -1;                 // row tile of the slabs being issued (advanced in order)
    QT qnext = 0;
    auto issue = [&](int s) {
      if ((s % SPT) == 0) {
        ++it_issue;
        while (!active(it_issue)) ++it_issue;
      }
      const int64_t i0 = (int64_t)it_issue * TILE + (s % SPT) * P::KC;
      const uint32_t st = lds0 + (s % P::NST) * P::STAGE;
      // rows i0 .. i0+64 of A (past m: zero) as [k][columns k0 .. k0+128]
      P::dma_k_tile(rsa, i0, lda, k0, st, w, lane);
      P::dma_k_tile(rsg, i0, ldg, n0, st + P::TILE, w, lane);
      if (w == 0) qnext = Q[i0 + lane];  // into qs before its barrier
    };
    struct Ops {
      float x[2][4], y[2][4];
    };
    auto fetch = [&](const uint8_t* st, const QT* qi, int gg, Ops& o) {
      P::frag_k2(st, ac2, gg, h, o.x);
      P::frag_k2(st + P::TILE, bc2, gg, h, o.y);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const QT q = qi[8 * gg + 4 * h + s];
#pragma unroll
        for (int t = 0; t < 2; ++t) o.x[t][s] *= (q * qk[t] > thr) ? 1.0f : 0.0f;
      }
    };
    const int nsteps = nact * SPT;
    issue(0);
    if (w == 0) qs[0][lane] = qnext;
    for (int s = 0; s < nsteps; ++s) {
      tsp::dma::wait_vm<0>();  // this wave's loads of slab s are done
      tsp::dma::barrier();     // slab s and its Q_i are visible; stage (s+1) % 2 is free
      if (s + 1 < nsteps) issue(s + 1);
      const uint8_t* st = lds + (s % P::NST) * P::STAGE;
      const QT* qi = qs[s & 1];
      Ops o[2];
      fetch(st, qi, 0, o[0]);
#pragma unroll
      for (int gg = 0; gg < P::KC / 8; ++gg) {
        if (gg + 1 < P::KC / 8) fetch(st, qi, gg + 1, o[(gg + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        acc.mma(o[gg & 1].x, o[gg & 1].y);
      }
      if (w == 0 && s + 1 < nsteps) qs[(s + 1) & 1][lane] = qnext;
    }
  }
  // accumulator (t, u) element v of lane (h, l32): output row k0 + wm*64 +
  // 2(8(v/4) + 4h + v%4) + t, column n0 + wn*64 + 2 l32 + u; (u = 0, 1) is
  // one 8-byte store
  const int64_t c = n0 + bc2;
  const bool pair = c + 1 < ncols && (lddb & 1) == 0 && ((uintptr_t)dB & 7) == 0;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t rb = k0 + wm * 64 + 2 * (8 * (v >> 2) + 4 * h + (v & 3));
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int64_t r = rb + t;
      if (r < m) {
        if (pair) {
          *(f32x2*)(dB + r * lddb + c) = f32x2{acc.a[t][0][v], acc.a[t][1][v]};
        } else {
          if (c < ncols) dB[r * lddb + c] = acc.a[t][0][v];
          if (c + 1 < ncols) dB[r * lddb + c + 1] = acc.a[t][1][v];
        }
      }
    }
  }
}

// dA[r][c] = (sum_n G[r][n] B[c][n]) * mask(r, c)
template <typename T, typename QT>
__global__ __launch_bounds__(256) void screened_bwd_a_generic(const T* __restrict__ G, int64_t ldg,
                                                              const T* __restrict__ B, int64_t ldb, int64_t ncols,
                                                              const QT* __restrict__ Q, QT thr, int64_t m,
                                                              T* __restrict__ dA, int64_t ldda) {
  typedef typename tsp::Acc<T>::type AccT;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= m * m) return;
  const int64_t r = t / m, c = t - r * m;
  AccT acc = 0;
  for (int64_t k = 0; k < ncols; ++k) acc += (AccT)G[r * ldg + k] * (AccT)B[c * ldb + k];
  dA[r * ldda + c] = (T)acc * ((Q[r] * Q[c] > thr) ? (T)1 : (T)0);
}

// dB[k][n] = sum_i (A[i][k] * mask(i, k)) G[i][n]
template <typename T, typename QT>
__global__ __launch_bounds__(256) void screened_bwd_b_generic(const T* __restrict__ A, int64_t lda,
                                                              const T* __restrict__ G, int64_t ldg, int64_t ncols,
                                                              const QT* __restrict__ Q, QT thr, int64_t m,
                                                              T* __restrict__ dB, int64_t lddb) {
  typedef typename tsp::Acc<T>::type AccT;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= m * ncols) return;
  const int64_t k = t / ncols, n = t - k * ncols;
  const QT qk = Q[k];
  AccT acc = 0;
  for (int64_t i = 0; i < m; ++i) {
    const T a = A[i * lda + k] * ((Q[i] * qk > thr) ? (T)1 : (T)0);
    acc += (AccT)a * (AccT)G[i * ldg + n];
  }
  dB[k * lddb + n] = (T)acc;
}

template <typename QT>
int launch_backward(const void* A, int dtype, int64_t lda, const void* diag, double thr_sqrt, int64_t m, const void* B,
                    int64_t ldb, int64_t ncols, const void* G, int64_t ldg, void* dA, int64_t ldda, void* dB,
                    int64_t lddb, void* ws, hipStream_t st) {
  const int64_t nmt = tsp::ceil_div(m, TILE);
  QT* Q = (QT*)ws;
  QT* qmax = Q + nmt * TILE;
  const QT thr = (QT)thr_sqrt;
  if (nmt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm_backward: too many rows");
  hipLaunchKernelGGL((screened_q<QT>), dim3((unsigned)nmt), dim3(TILE), 0, st, (const QT*)diag, m, Q, qmax);
  int rc = tsp::check_launch("screened_q launch");
  if (rc) return rc;
  // streamed fp32 kernels: 16-byte aligned rows, buffer offsets within 32 bits
  auto fits = [&](const void* p, int64_t ld) {
    return (ld % 4) == 0 && ((uintptr_t)p % 16) == 0 && (m + TILE) * ld * 4 + 4 * TILE <= (int64_t)UINT32_MAX;
  };
  const bool f32 = dtype == TSP_F32 && fits(G, ldg);
  if (dA) {
    if (f32 && fits(B, ldb)) {
      const int64_t grid = tsp::ceil_div(nmt * nmt, 8) * 8;
      if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm_backward: problem too large");
      hipLaunchKernelGGL((screened_bwd_a_f32<QT>), dim3((unsigned)grid), dim3(256), 0, st, (const float*)G, ldg,
                         (const float*)B, ldb, ncols, (const QT*)Q, (const QT*)qmax, thr, m, (int)nmt, (float*)dA,
                         ldda);
      rc = tsp::check_launch("screened_bwd_a_f32 launch");
    } else {
      const int64_t grid = tsp::ceil_div(m * m, 256);
      if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm_backward: problem too large");
      if (dtype == TSP_F32)
        hipLaunchKernelGGL((screened_bwd_a_generic<float, QT>), dim3((unsigned)grid), dim3(256), 0, st,
                           (const float*)G, ldg, (const float*)B, ldb, ncols, (const QT*)Q, thr, m, (float*)dA, ldda);
      else
        hipLaunchKernelGGL((screened_bwd_a_generic<double, QT>), dim3((unsigned)grid), dim3(256), 0, st,
                           (const double*)G, ldg, (const double*)B, ldb, ncols, (const QT*)Q, thr, m, (double*)dA,
                           ldda);
      rc = tsp::check_launch("screened_bwd_a_generic launch");
    }
    if (rc) return rc;
  }
  if (dB) {
    if (f32 && fits(A, lda)) {
      const int64_t nnt = tsp::ceil_div(ncols, TILE);
      const int64_t grid = tsp::ceil_div(nmt, 8) * 8 * nnt;
      if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm_backward: problem too large");
      hipLaunchKernelGGL((screened_bwd_b_f32<QT>), dim3((unsigned)grid), dim3(256), 0, st, (const float*)A, lda,
                         (const float*)G, ldg, ncols, (const QT*)Q, (const QT*)qmax, thr, m, (int)nmt, (int)nnt,
                         (float*)dB, lddb);
      rc = tsp::check_launch("screened_bwd_b_f32 launch");
    } else {
      const int64_t grid = tsp::ceil_div(m * ncols, 256);
      if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm_backward: problem too large");
      if (dtype == TSP_F32)
        hipLaunchKernelGGL((screened_bwd_b_generic<float, QT>), dim3((unsigned)grid), dim3(256), 0, st,
                           (const float*)A, lda, (const float*)G, ldg, ncols, (const QT*)Q, thr, m, (float*)dB, lddb);
      else
        hipLaunchKernelGGL((screened_bwd_b_generic<double, QT>), dim3((unsigned)grid), dim3(256), 0, st,
                           (const double*)A, lda, (const double*)G, ldg, ncols, (const QT*)Q, thr, m, (double*)dB,
                           lddb);
      rc = tsp::check_launch("screened_bwd_b_generic launch");
    }
    if (rc) return rc;
  }
  return TSP_OK;
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
  if (dtype == TSP_F32 && (lda % 4) == 0 && (ldb % 4) == 0 && ((uintptr_t)A % 16) == 0 && ((uintptr_t)B % 16) == 0 &&
      (m + TILE) * lda * 4 + 4 * TILE <= (int64_t)UINT32_MAX && (m + TILE) * ldb * 4 + 4 * TILE <= (int64_t)UINT32_MAX) {
    // (the streamed kernel's buffer offsets fit 32 bits)
    const int64_t nnt = tsp::ceil_div(ncols, TILE);
    const int64_t grid = tsp::ceil_div(nmt, 8) * 8 * nnt;
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm: problem too large");
    hipLaunchKernelGGL((screened_f32_dma<QT, SCREENED_KC>), dim3((unsigned)grid), dim3(256), 0, st, (const float*)A, lda,
                       (const QT*)Q, (const QT*)qmax, thr, m, (const float*)B, ldb, ncols, (float*)C, ldc, (int)nmt,
                       (int)nnt);
    return tsp::check_launch("screened_f32_dma launch");
  }
  if (dtype == TSP_F32 && (lda % 4) == 0 && (ldb % 4) == 0 && ((uintptr_t)A % 16) == 0 && ((uintptr_t)B % 16) == 0) {
    const int64_t nnt = tsp::ceil_div(ncols, T32::BN);
    const int64_t grid = tsp::ceil_div(nmt, 8) * 8 * nnt;
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm: problem too large");
    hipLaunchKernelGGL((screened_f32_mfma<QT>), dim3((unsigned)grid), dim3(T32::NTHR), 0, st, (const float*)A, lda,
                       (const QT*)Q, (const QT*)qmax, thr, m, (const float*)B, ldb, ncols, (float*)C, ldc, (int)nmt,
                       (int)nnt);
    return tsp::check_launch("screened_f32_mfma launch");
  }
  if (dtype == TSP_F64 && (m % 2) == 0 && (lda % 2) == 0 && (ldb % 2) == 0 && ((uintptr_t)A % 16) == 0 &&
      ((uintptr_t)B % 16) == 0 && (m + TILE) * lda * 8 + 8 * TILE <= (int64_t)UINT32_MAX &&
      (m + TILE) * ldb * 8 + 8 * TILE <= (int64_t)UINT32_MAX) {
    const int64_t nnt = tsp::ceil_div(ncols, TILE);
    const int64_t grid = tsp::ceil_div(nmt, 8) * 8 * nnt;
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm: problem too large");
    hipLaunchKernelGGL((screened_f64_dma<QT>), dim3((unsigned)grid), dim3(256), 0, st, (const double*)A, lda,
                       (const QT*)Q, (const QT*)qmax, thr, m, (const double*)B, ldb, ncols, (double*)C, ldc, (int)nmt,
                       (int)nnt);
    return tsp::check_launch("screened_f64_dma launch");
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

// ------------------------------------------------ allocation-free variant
//
// tsp_screened_spmm_noalloc keeps the workspace (Q and the per-tile maxima)
// in this file-scope device array instead of caller memory. Each GPU holds
// its own copy for the life of the process; its device address is looked up
// once per device with hipGetSymbolAddress (the array's name is only a
// host-side stand-in) and cached. Every call on a GPU shares that GPU's
// array: calls that overlap on one GPU (other streams, other threads) race.
// screened_q rewrites every word the kernels read, so nothing needs
// clearing between calls.
constexpr int64_t SCREENED_SCRATCH_BYTES = 1 << 20;
constexpr int SCRATCH_MAX_DEVICES = 64;
static __device__ __align__(256) uint8_t scratch[SCREENED_SCRATCH_BYTES];
static std::atomic<void*> g_scratch_ptr[SCRATCH_MAX_DEVICES];

int scratch_on_current_device(void** out) {
  int dev = -1;
  int rc = tsp::check_hip(hipGetDevice(&dev), "tsp_screened_spmm_noalloc: hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm_noalloc: device %d past the %d supported", dev,
                     SCRATCH_MAX_DEVICES);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {  // first call on this device (a racing thread stores the same address)
    rc = tsp::check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "tsp_screened_spmm_noalloc: hipGetSymbolAddress");
    if (rc) return rc;
    if (!p) return tsp::fail(TSP_EHIP, "tsp_screened_spmm_noalloc: null scratch address");
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return TSP_OK;
}

int64_t workspace_bytes(int64_t m, int diag_dtype) {
  const int64_t nmt = tsp::ceil_div(m, TILE);
  return (nmt * TILE + nmt) * (diag_dtype == TSP_F64 ? 8 : 4);
}

int check_args(const char* who, const void* A, int dtype, int64_t lda, const void* diag, int diag_dtype, int64_t m,
               const void* B, int64_t ldb, int64_t ncols, const void* C, int64_t ldc) {
  if (dtype != TSP_F32 && dtype != TSP_F64) return tsp::fail(TSP_EUNSUPPORTED, "%s: dtype %d not supported", who, dtype);
  if (diag_dtype != TSP_F32 && diag_dtype != TSP_F64)
    return tsp::fail(TSP_EUNSUPPORTED, "%s: diag dtype %d not supported", who, diag_dtype);
  if (m < 0 || ncols < 0) return tsp::fail(TSP_EINVAL, "%s: negative size", who);
  if (lda < m || ldb < ncols || ldc < ncols) return tsp::fail(TSP_EINVAL, "%s: leading dimension too small", who);
  if (m > 0 && ncols > 0 && (!A || !diag || !B || !C)) return tsp::fail(TSP_EINVAL, "%s: null pointer", who);
  return TSP_OK;
}

}  // namespace

extern "C" int64_t tsp_screened_spmm_noalloc_max_rows(int diag_dtype) {
  if (diag_dtype != TSP_F32 && diag_dtype != TSP_F64) return -1;
  const int64_t per_tile = (TILE + 1) * (diag_dtype == TSP_F64 ? 8 : 4);
  return (SCREENED_SCRATCH_BYTES / per_tile) * TILE;
}

extern "C" int tsp_screened_spmm_noalloc(const void* A, int dtype, int64_t lda, const void* diag, int diag_dtype,
                                         double threshold_sqrt, int64_t m, const void* B, int64_t ldb, int64_t ncols,
                                         void* C, int64_t ldc, void* stream) {
  int rc = check_args("tsp_screened_spmm_noalloc", A, dtype, lda, diag, diag_dtype, m, B, ldb, ncols, C, ldc);
  if (rc) return rc;
  if (m == 0 || ncols == 0) return TSP_OK;
  if (workspace_bytes(m, diag_dtype) > SCREENED_SCRATCH_BYTES)
    return tsp::fail(TSP_EINVAL, "tsp_screened_spmm_noalloc: m = %lld needs %lld bytes of scratch, more than its %lld",
                     (long long)m, (long long)workspace_bytes(m, diag_dtype), (long long)SCREENED_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = scratch_on_current_device(&ws);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  return diag_dtype == TSP_F32 ? launch<float>(A, dtype, lda, diag, threshold_sqrt, m, B, ldb, ncols, C, ldc, ws, st)
                               : launch<double>(A, dtype, lda, diag, threshold_sqrt, m, B, ldb, ncols, C, ldc, ws, st);
}

extern "C" int64_t tsp_screened_workspace_size(int64_t m, int diag_dtype) {
  if (m < 0 || (diag_dtype != TSP_F32 && diag_dtype != TSP_F64)) return -1;
  return workspace_bytes(m, diag_dtype);
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

extern "C" int tsp_screened_spmm_backward(const void* A, int dtype, int64_t lda, const void* diag, int diag_dtype,
                                          double threshold_sqrt, int64_t m, const void* B, int64_t ldb, int64_t ncols,
                                          const void* dC, int64_t lddc, void* dA, int64_t ldda, void* dB,
                                          int64_t lddb, void* workspace, void* stream) {
  if (dtype != TSP_F32 && dtype != TSP_F64)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm_backward: dtype %d not supported", dtype);
  if (diag_dtype != TSP_F32 && diag_dtype != TSP_F64)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_screened_spmm_backward: diag dtype %d not supported", diag_dtype);
  if (m < 0 || ncols < 0) return tsp::fail(TSP_EINVAL, "tsp_screened_spmm_backward: negative size");
  if (lddc < ncols || (dA && (ldb < ncols || ldda < m)) || (dB && (lda < m || lddb < ncols)))
    return tsp::fail(TSP_EINVAL, "tsp_screened_spmm_backward: leading dimension too small");
  if (m == 0 || (!dA && !dB)) return TSP_OK;
  if (!diag || !dC || !workspace || (dA && !B) || (dB && !A))
    return tsp::fail(TSP_EINVAL, "tsp_screened_spmm_backward: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (ncols == 0) {  // dA = 0 (an empty sum); dB has no columns
    if (!dA) return TSP_OK;
    const int64_t es = dtype == TSP_F64 ? 8 : 4;
    for (int64_t r = 0; r < m; ++r) {
      int rc = tsp::zero_fill((char*)dA + r * ldda * es, m * es, st);
      if (rc) return rc;
    }
    return TSP_OK;
  }
  return diag_dtype == TSP_F32
             ? launch_backward<float>(A, dtype, lda, diag, threshold_sqrt, m, B, ldb, ncols, dC, lddc, dA, ldda, dB,
                                      lddb, workspace, st)
             : launch_backward<double>(A, dtype, lda, diag, threshold_sqrt, m, B, ldb, ncols, dC, lddc, dA, ldda, dB,
                                       lddb, workspace, st);
}
