// Backward of BSR SpMM for gfx950.
//
// For C = A_bsr @ B (reference autograd: trnsparse/nki/dispatch.py:331-369)
//   dA_k = dC[rows of block row i] @ B[rows of block column j]^T   (stored k = (i, j))
//   dB   = A^T @ dC
// dA is an SDDMM restricted to the stored pattern (one 128x128 product with
// K = N per stored block); dB is a BSR-transpose SpMM over the block-column
// view of the pattern (col_ptrs / col_block_ids / col_block_rows, blocks of a
// column in increasing block-row order, so every sum has a fixed order).
//
// Kernels
//   bsr_sddmm_f32_dma    b == 128, fp32: one 256-thread workgroup per stored
//                        block; 4 waves of 64x64 (four 32x32x2 MFMA
//                        accumulators). 64-wide k-slabs (k = columns of dC
//                        and B) of the two [128][64] row tiles stream through
//                        a 2-stage LDS ring by direct global->LDS buffer loads
//                        (rows past m / n and columns past N read as zero);
//                        both MFMA operands are k-contiguous, so each is one
//                        16-byte LDS read per 4 k-steps (k permuted within
//                        each 8-k group as in the forward kernels).
//   bsr_spmm_t_f32_dma   b == 128, fp32: C tile 128 (one block column of A,
//                        i.e. 128 rows of dB) x 128 columns per workgroup,
//                        walking the blocks of that column; A^T comes from
//                        the untransposed blocks ([k][m] in LDS, 4-byte reads
//                        like the forward B operand), dC rows of the block's
//                        block row as the [k][n] operand. Scheduling as the
//                        forward kernel (heaviest columns first, boustrophedon
//                        over the XCDs, one workgroup per CU).
//   bsr_sddmm_bf16_mfma / bsr_spmm_t_bf16_mfma   b == 128, bf16 (fp32
//                        accumulation, bf16 results): the same two products on
//                        v_mfma_f32_32x32x16_bf16 (operand forms at the kernels).
//   bsr_sddmm_f64_mfma / bsr_spmm_t_f64_mfma   b == 128, fp64: the same two
//                        products on v_mfma_f64_16x16x4_f64.
//   bsr_sddmm_small<b>   b in {8, 16, 32, 64}, fp32 / bf16: a wavefront per
//                        stored block on fp32 MFMAs, operands straight from
//                        memory (details at the kernel); dB at these block
//                        sizes is bsr_spmm.hip's small-block kernel walking
//                        the block-column view with A transposed.
//   bsr_sddmm_generic / bsr_spmm_t_generic   any block size, f32 / f64 / bf16
//                        (accumulating in f32, f64 for f64): one thread per
//                        output element.
#include "common.h"

#include "lds_dma.h"
#include "mfma_f32.h"
#include "mfma_f64.h"
#include "f32_pair_tiles.h"

namespace {

namespace T32 = tsp::f32tile;
using tsp::dma::i32x4;
using namespace tsp::f32pair;

// ------------------------------------------------------------- dA (SDDMM)

__global__ __launch_bounds__(256) void bsr_sddmm_f32_dma(const float* __restrict__ G, int64_t ldg, int64_t m,
                                                         const float* __restrict__ B, int64_t ldb, int64_t n,
                                                         int64_t ncols, const int64_t* __restrict__ brow,
                                                         const int64_t* __restrict__ ci, int64_t nnzb,
                                                         float* __restrict__ out) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];
  // XCD-aware: XCD x takes a contiguous range of stored blocks (same block
  // rows, so the dC panel is shared in its L2)
  const int64_t g = blockIdx.x, xcd = g & 7, slot = g >> 3;
  const int64_t per = tsp::ceil_div(nnzb, 8);
  const int64_t kb = xcd * per + slot;
  if (slot >= per || kb >= nnzb) return;
  const int64_t i = brow[kb], j = ci[kb];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;
  const i32x4 rsg = tsp::dma::make_rsrc(G, (uint32_t)(m * ldg * 4));
  const i32x4 rsb = tsp::dma::make_rsrc(B, (uint32_t)(n * ldb * 4));
  const uint32_t lds0 = tsp::dma::lds_addr(lds);
  auto issue = [&](int s) {
    const uint32_t st = lds0 + (s % NST) * STAGE;
    dma_row_tile(rsg, i * BS, ldg, (int64_t)s * KC, ncols, st, w, lane);
    dma_row_tile(rsb, j * BS, ldb, (int64_t)s * KC, ncols, st + TILE, w, lane);
  };
  Acc4 acc;
  acc.zero();
  const int ar = wm * 64 + l32, br = wn * 64 + l32;
  struct Ops {
    float x[2][4], y[2][4];
  };
  auto fetch = [&](const uint8_t* st, int gg, Ops& o) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const f32x4 a = frag_row(st, ar + 32 * t, gg, h);
      const f32x4 b = frag_row(st + TILE, br + 32 * t, gg, h);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        o.x[t][s] = a[s];
        o.y[t][s] = b[s];
      }
    }
  };
  const int nsteps = (int)tsp::ceil_div(ncols, KC);
  if (nsteps > 0) issue(0);
  for (int s = 0; s < nsteps; ++s) {
    tsp::dma::wait_vm<0>();
    tsp::dma::barrier();
    if (s + 1 < nsteps) issue(s + 1);
    const uint8_t* st = lds + (s % NST) * STAGE;
    Ops o[2];
    fetch(st, 0, o[0]);
#pragma unroll
    for (int gg = 0; gg < KC / 8; ++gg) {
      if (gg + 1 < KC / 8) fetch(st, gg + 1, o[(gg + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      acc.mma(o[gg & 1].x, o[gg & 1].y);
    }
  }
  // dA block kb, row-major [r][c]: lane holds column l32 and rows 8*(v/4) + 4h + v%4
  float* ob = out + kb * (BS * BS);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = wm * 64 + 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
        ob[r * BS + wn * 64 + 32 * u + l32] = acc.a[t][u][v];
      }
}

// ------------------------------------------------------- dB (A^T @ dC)

__global__ __launch_bounds__(256) void bsr_spmm_t_f32_dma(
    const float* __restrict__ blocks, const int64_t* __restrict__ cp, const int64_t* __restrict__ cbid,
    const int64_t* __restrict__ crow, int64_t nbc, int nt, const float* __restrict__ X, int64_t ldx, int64_t m,
    int64_t ncols, float* __restrict__ out, int64_t ldo, int64_t n, const int32_t* __restrict__ order) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];
  int64_t col;
  int ntile;
  if (!T32::tile_item(blockIdx.x, nbc, nt, order, col, ntile)) return;
  const int64_t n0 = (int64_t)ntile * BS;
  const int64_t start = cp[col];
  const int nblk = (int)(cp[col + 1] - start);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;
  Acc4 acc;
  acc.zero();
  if (nblk > 0) {
    const i32x4 rsx = tsp::dma::make_rsrc(X, (uint32_t)(m * ldx * 4));
    const uint32_t lds0 = tsp::dma::lds_addr(lds);
    // block ids and block rows of the column, 64 at a time in one VGPR each
    int cbase = 0;
    auto load_ids = [&](int base, int& idv, int& rowv) {
      const int64_t e = start + (base + lane < nblk ? base + lane : nblk - 1);
      idv = tsp::dma::load_lo32_sync(cbid + e);
      rowv = tsp::dma::load_lo32_sync(crow + e);
    };
    int idv, rowv;
    load_ids(0, idv, rowv);
    auto entry = [&](int b, int64_t& kb, int64_t& ib) {
      if (b - cbase >= 64) {
        cbase = b & ~63;
        load_ids(cbase, idv, rowv);
      }
      kb = __builtin_amdgcn_readlane(idv, b - cbase);
      ib = __builtin_amdgcn_readlane(rowv, b - cbase);
    };
    auto issue = [&](int s) {
      int64_t kb, ib;
      entry(s >> 1, kb, ib);
      const int kk = (s & 1) * KC;
      const uint32_t st = lds0 + (s % NST) * STAGE;
      // A block rows [kk, kk+64) as the [k][m] operand of A^T
      dma_k_tile_global(blocks + kb * (BS * BS) + kk * BS, BS, st, w, lane);
      // dC rows ib*128 + kk .. +64 (past m: zero), columns n0 .. n0+128
      dma_k_tile(rsx, ib * BS + kk, ldx, n0, st + TILE, w, lane);
    };
    // subtiles interleave: row subtile t holds output rows wm*64 + 2i + t,
    // column subtile u holds columns wn*64 + 2j + u, so one 8-byte read per
    // k row feeds both subtiles of an operand
    const int ac2 = wm * 64 + 2 * l32, bc2 = wn * 64 + 2 * l32;
    struct Ops {
      float x[2][4], y[2][4];
    };
    auto fetch = [&](const uint8_t* st, int gg, Ops& o) {
      frag_k2(st, ac2, gg, h, o.x);
      frag_k2(st + TILE, bc2, gg, h, o.y);
    };
    const int nsteps = nblk * (BS / KC);
    issue(0);
    for (int s = 0; s < nsteps; ++s) {
      tsp::dma::wait_vm<0>();
      tsp::dma::barrier();
      if (s + 1 < nsteps) issue(s + 1);
      const uint8_t* st = lds + (s % NST) * STAGE;
      Ops o[2];
      fetch(st, 0, o[0]);
#pragma unroll
      for (int gg = 0; gg < KC / 8; ++gg) {
        if (gg + 1 < KC / 8) fetch(st, gg + 1, o[(gg + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        acc.mma(o[gg & 1].x, o[gg & 1].y);
      }
    }
  }
  // accumulator (t, u) element v of lane (h, l32): MFMA row i = 8(v/4) + 4h +
  // v%4 and column j = l32, i.e. output row wm*64 + 2i + t, column
  // wn*64 + 2j + u; the (u = 0, 1) pair is one 8-byte store
  const int64_t c = n0 + wn * 64 + 2 * l32;
  const bool pair = c + 1 < ncols && (ldo & 1) == 0 && ((uintptr_t)out & 7) == 0;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t rb = col * BS + wm * 64 + 2 * (8 * (v >> 2) + 4 * h + (v & 3));
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int64_t r = rb + t;
      if (r < n) {
        if (pair) {
          *(f32x2*)(out + r * ldo + c) = f32x2{acc.a[t][0][v], acc.a[t][1][v]};
        } else {
          if (c < ncols) out[r * ldo + c] = acc.a[t][0][v];
          if (c + 1 < ncols) out[r * ldo + c + 1] = acc.a[t][1][v];
        }
      }
    }
  }
}

// ------------------------------------------------------------ bf16 MFMA
//
// bf16 operands, fp32 accumulation, bf16 results, b == 128, on
// v_mfma_f32_32x32x16_bf16 (lane half h supplies k = 8h .. 8h + 7 of each
// 16-k step; A rows / B columns are lane % 32). One engine for the products:
// 256 threads, 4 waves of 64x64 (2 x 2 accumulators), KC-wide k-slabs of two
// operand tiles streamed through an NST-stage LDS ring by direct loads
// issued NST - 1 slabs ahead (LPW + LPW wave instructions per slab). Each
// kernel picks its (KC, NST): the ring is sized so that several workgroups
// share a CU and one's operand reads and load waits overlap another's MFMAs
// (with one workgroup and a 4-stage ring the LDS read latency was exposed in
// every 16-k step: 23-31 % slower). Measured on cfg3b dA: KC = 64 with a
// 2-stage ring (64 KiB, two workgroups per CU) 53-54 us; KC = 32 with a
// 3-stage ring (48 KiB, three per CU) 44 us, with 4 or 5 stages (two per
// CU) 49 us, KC = 64 with 3 stages (one per CU) 60 us. Each operand tile is
// in one of two forms, TILE = 128 x KC x 2 bytes:
//   ROW: [128 rows][KC k], rows of 2 KC bytes, k contiguous: a lane's 8 k
//        values are one b128 read; the 16-byte chunk c of row r sits in slot
//        c ^ sw(r) so that 16 consecutive rows of one chunk cover the 64
//        banks (KC = 64: (r / 2) % 8; KC = 32: (r / 4) % 4);
//   TR:  [KC k][128 columns], rows of 256 B: the 8 k values come from two
//        ds_read_b64_tr_b16 (4 consecutive k rows each); chunk ^ 4 (row % 4).
// dA (SDDMM): both operands ROW (dC rows of the block row, B rows of the
// block column, k = columns). dB = A^T dC: both operands TR (the block's
// rows are k, its columns the output rows; dC rows of the block row).
namespace bfb {
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int KC_>
struct Slab {
  static constexpr int KC = KC_;
  static_assert(KC == 32 || KC == 64, "slab widths with a conflict-free ROW swizzle");
  static constexpr int RB = 2 * KC;            // bytes per ROW-tile row
  static constexpr int LPR = RB / 16;          // lanes per ROW-tile row in a 1 KiB piece
  static constexpr int RPP = 64 / LPR;         // ROW-tile rows per 1 KiB piece
  static constexpr int TILE = 128 * RB;        // bytes per operand tile
  static constexpr int STAGE = 2 * TILE;
  static constexpr int LPW = TILE / 4096;      // 1 KiB pieces per wave and tile
  __device__ static constexpr int sw(int r) { return KC == 64 ? ((r >> 1) & 7) : ((r >> 2) & 3); }
};

// ROW tile: rows [row0, row0 + 128) x columns [k0, k0 + KC) of a bf16
// row-major matrix (stride ld) behind rs; columns at or past kend read as
// zero (kend % 8 == 0).
// The ROW tile stream of one operand with the per-lane offsets computed
// once: slab s adds s * KC columns (2 bytes each) and compares with kend.
template <int KC>
struct RowStream {
  using S = Slab<KC>;
  uint32_t base[S::LPW];
  int col[S::LPW];
  __device__ RowStream(int64_t row0, int64_t ld, int w, int lane) {
#pragma unroll
    for (int q = 0; q < S::LPW; ++q) {
      const int i = S::LPW * w + q;
      const int r = S::RPP * i + lane / S::LPR;
      const int c = (lane % S::LPR) ^ S::sw(r);
      col[q] = c * 8;
      base[q] = (uint32_t)(((row0 + r) * ld + c * 8) * 2);
    }
  }
  __device__ inline void issue(i32x4 rs, int s, int64_t kend, uint32_t dst, int w) const {
    const int k0 = s * KC;
    const int lim = (int)(kend - k0);  // columns k0 + col < kend  <=>  col < lim
#pragma unroll
    for (int q = 0; q < S::LPW; ++q) {
      const uint32_t off = col[q] < lim ? base[q] + (uint32_t)(k0 * 2) : OOB;
      tsp::dma::buffer16(rs, off, dst + (S::LPW * w + q) * 1024);
    }
  }
};
// TR tile: rows [row0, row0 + KC) x columns [c0, c0 + 128) of a bf16
// row-major matrix (stride ld) behind rs.
template <int KC>
__device__ inline void dma_tr(i32x4 rs, int64_t row0, int64_t ld, int64_t c0, uint32_t dst, int w, int lane) {
  constexpr int LPW = Slab<KC>::LPW;
#pragma unroll
  for (int q = 0; q < LPW; ++q) {
    const int j = LPW * w + q;
    const int rr = 4 * j + (lane >> 4);
    const int c = (lane & 15) ^ (4 * (rr & 3));
    tsp::dma::buffer16(rs, (uint32_t)(((row0 + rr) * ld + c0 + c * 8) * 2), dst + j * 1024);
  }
}
// The same TR tile from a 128-column block that is always in bounds.
template <int KC>
__device__ inline void dma_tr_block(const uint16_t* src, uint32_t dst, int w, int lane) {
  constexpr int LPW = Slab<KC>::LPW;
#pragma unroll
  for (int q = 0; q < LPW; ++q) {
    const int j = LPW * w + q;
    const int rr = 4 * j + (lane >> 4);
    const int c = (lane & 15) ^ (4 * (rr & 3));
    tsp::dma::global16(src + rr * BS + c * 8, dst + j * 1024);
  }
}
// Operand of 16-k step ks for tile row / column `base` + lane % 32.
template <int KC>
__device__ inline bf16x8 op_row(const uint8_t* tile, int base, int ks, int lane) {
  using S = Slab<KC>;
  const int r = base + (lane & 31);
  return *(const bf16x8*)(tile + r * S::RB + (((2 * ks + (lane >> 5)) ^ S::sw(r)) * 16));
}
__device__ inline bf16x8 op_tr(const uint8_t* tile, int base, int ks, int lane) {
  const int gq = lane >> 4, jq = lane & 15;
  const int col = base + 16 * (gq & 1) + 4 * (jq & 3);
  s16x4 v[2];
#pragma unroll
  for (int kq = 0; kq < 2; ++kq) {
    const int rr = 16 * ks + 8 * (gq >> 1) + (jq >> 2) + 4 * kq;
    const uint8_t* p = tile + rr * 256 + (((col >> 3) ^ (4 * (jq >> 2))) * 16) + (col & 4) * 2;
    v[kq] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
  }
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7));
}

// Wait until this wave's loads of a slab are done while the `later` slabs
// issued after it (LPS loads each) may still be in flight.
template <int LPS, int NST>
__device__ inline void wait_slab(int later) {
  if constexpr (NST >= 4) {
    if (later >= 2) {
      tsp::dma::wait_vm<2 * LPS>();
      return;
    }
  }
  if constexpr (NST >= 3) {
    if (later >= 1) {
      tsp::dma::wait_vm<LPS>();
      return;
    }
  }
  tsp::dma::wait_vm<0>();
}

// The slab loop shared by the kernels: issue(s) fills stage s % NST,
// compute runs the KC / 16 k-steps of a stage into acc.
template <bool AROW, bool BROW, int KC, int NST, typename Issue>
__device__ inline void run(Issue&& issue, int nsteps, const uint8_t* lds, f32x16 (&acc)[2][2], int wm, int wn,
                           int lane) {
  using S = Slab<KC>;
  static_assert(NST >= 2 && NST <= 4, "ring depths with a vmcnt schedule");
  auto fetch = [&](const uint8_t* st, int ks, bf16x8 (&a)[2], bf16x8 (&b)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      a[t] = AROW ? op_row<KC>(st, wm * 64 + 32 * t, ks, lane) : op_tr(st, wm * 64 + 32 * t, ks, lane);
      b[t] = BROW ? op_row<KC>(st + S::TILE, wn * 64 + 32 * t, ks, lane) : op_tr(st + S::TILE, wn * 64 + 32 * t, ks, lane);
    }
  };
  const int pre = nsteps < NST - 1 ? nsteps : NST - 1;
  for (int s = 0; s < pre; ++s) issue(s);
  for (int s = 0; s < nsteps; ++s) {
    // this wave's loads of slab s are done when only the later slabs already
    // issued (2 LPW loads each, at most NST - 2 of them) are in flight
    const int later0 = nsteps - 1 - s;
    wait_slab<2 * S::LPW, NST>(later0 < NST - 2 ? later0 : NST - 2);
    tsp::dma::barrier();  // every wave's part of slab s is in LDS; stage (s - 1) % NST is free
    if (s + NST - 1 < nsteps) issue(s + NST - 1);
    const uint8_t* st = lds + (s % NST) * S::STAGE;
    bf16x8 a[2][2], b[2][2];
    fetch(st, 0, a[0], b[0]);
#pragma unroll
    for (int ks = 0; ks < KC / 16; ++ks) {
      if (ks + 1 < KC / 16) fetch(st, ks + 1, a[(ks + 1) & 1], b[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u)
          acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks & 1][t], b[ks & 1][u], acc[t][u], 0, 0, 0);
    }
  }
}
}  // namespace bfb

// Slab width and ring depth of each bf16 kernel. dA with bf16 blocks: the
// forms listed at the engine ran 43.5-43.7 us alike on a box whose loads
// return quickly, and 32/3 was 15-19 % faster on boxes where the same kernel
// at 64/2 took 53-54 us at the same shader clock (more loads in flight and
// three workgroups per CU hide the longer memory latency). Block scores with
// fp32 output (attention at d = 512 over the stacked mask: 331 us against
// 345 at 32/3), dB and the attention block gradient keep 64/2 (dB 44.4 us
// against 48.0, the block gradient at d = 256 555 us against 590).
constexpr int SDDMM_KC = 32, SDDMM_NST = 3;
constexpr int SCORES_KC = 64, SCORES_NST = 2;
constexpr int PGRAD_KC = 64, PGRAD_NST = 2;
constexpr int SPMMT_KC = 64, SPMMT_NST = 2;

// dA (SDDMM), bf16: workgroup per stored block, XCD x takes a contiguous
// range of blocks as in bsr_sddmm_f32_dma. OutT uint16_t: bf16 blocks (the
// gradient of bf16 blocks); float: the fp32 accumulators as they are (block
// scores that a softmax reads next).
__device__ inline void store_out(uint16_t* p, float v) { *p = tsp::f32_to_bf16_bits(v); }
__device__ inline void store_out(float* p, float v) { *p = v; }

template <typename OutT, int KC = SDDMM_KC, int NST = SDDMM_NST>
__global__ __launch_bounds__(256) void bsr_sddmm_bf16_mfma(const uint16_t* __restrict__ G, int64_t ldg, int64_t m,
                                                           const uint16_t* __restrict__ B, int64_t ldb, int64_t n,
                                                           int64_t ncols, const int64_t* __restrict__ brow,
                                                           const int64_t* __restrict__ ci, int64_t nnzb,
                                                           OutT* __restrict__ out) {
  using S = bfb::Slab<KC>;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * S::STAGE];
  const int64_t g = blockIdx.x, xcd = g & 7, slot = g >> 3;
  const int64_t per = tsp::ceil_div(nnzb, 8);
  const int64_t kb = xcd * per + slot;
  if (slot >= per || kb >= nnzb) return;
  const int64_t i = brow[kb], j = ci[kb];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;
  const i32x4 rsg = tsp::dma::make_rsrc(G, (uint32_t)(m * ldg * 2));
  const i32x4 rsb = tsp::dma::make_rsrc(B, (uint32_t)(n * ldb * 2));
  const uint32_t lds0 = tsp::dma::lds_addr(lds);
  const bfb::RowStream<KC> sg(i * BS, ldg, w, lane), sb(j * BS, ldb, w, lane);
  auto issue = [&](int s) {
    const uint32_t st = lds0 + (s % NST) * S::STAGE;
    sg.issue(rsg, s, ncols, st, w);
    sb.issue(rsb, s, ncols, st + S::TILE, w);
  };
  f32x16 acc[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) acc[t][u] = f32x16{};
  bfb::run<true, true, KC, NST>(issue, (int)tsp::ceil_div(ncols, KC), lds, acc, wm, wn, lane);
  // dA block kb, row-major: lane holds column l32 and rows 8 (v / 4) + 4 h + v % 4
  OutT* ob = out + kb * (BS * BS);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = wm * 64 + 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
        store_out(ob + r * BS + wn * 64 + 32 * u + l32, acc[t][u][v]);
      }
}

// Block gradient of block-sparse attention, bf16 (the block-product path for
// head_dims the one-pass backward kernels do not hold): per stored block kb
// = (block row i, block column j) of the mask stacked over heads, S = Q_i
// K_j^T and dP = dO_i V_j^T run through the SDDMM engine one after the other
// (both accumulators stay in registers), then
//   P  = exp(scale S - row_max) / row_denom,   dS = scale P (dP - Drow)
// are written as bf16 blocks (reference trnsparse/ops.py:461-467). The fp32
// scores never leave the workgroup.
template <int KC = PGRAD_KC, int NST = PGRAD_NST>
__global__ __launch_bounds__(256) void bsa_block_pgrad_bf16(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ dO, int64_t rows, int64_t D, const int64_t* __restrict__ brow,
    const int64_t* __restrict__ ci, int64_t nnzb, float scale, const float* __restrict__ rmax,
    const float* __restrict__ rden, const float* __restrict__ Drow, uint16_t* __restrict__ P,
    uint16_t* __restrict__ dS) {
  using S = bfb::Slab<KC>;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * S::STAGE];
  __shared__ float rstat[3][BS];
  const int64_t g = blockIdx.x, xcd = g & 7, slot = g >> 3;
  const int64_t per = tsp::ceil_div(nnzb, 8);
  const int64_t kb = xcd * per + slot;
  if (slot >= per || kb >= nnzb) return;
  const int64_t i = brow[kb], j = ci[kb];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;
  if (tid < BS) {
    rstat[0][tid] = rmax[i * BS + tid];
    rstat[1][tid] = rden[i * BS + tid];
    rstat[2][tid] = Drow[i * BS + tid];
  }
  const uint32_t bytes = (uint32_t)(rows * D * 2);
  const i32x4 rq = tsp::dma::make_rsrc(Q, bytes), rk = tsp::dma::make_rsrc(K, bytes);
  const i32x4 rv = tsp::dma::make_rsrc(V, bytes), rdo = tsp::dma::make_rsrc(dO, bytes);
  const uint32_t lds0 = tsp::dma::lds_addr(lds);
  const bfb::RowStream<KC> sq(i * BS, D, w, lane), sk(j * BS, D, w, lane);
  const bfb::RowStream<KC> sdo(i * BS, D, w, lane), sv(j * BS, D, w, lane);
  const int nsteps = (int)tsp::ceil_div(D, KC);
  f32x16 as[2][2], ap[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      as[t][u] = f32x16{};
      ap[t][u] = f32x16{};
    }
  auto issue_s = [&](int s) {
    const uint32_t st = lds0 + (s % NST) * S::STAGE;
    sq.issue(rq, s, D, st, w);
    sk.issue(rk, s, D, st + S::TILE, w);
  };
  bfb::run<true, true, KC, NST>(issue_s, nsteps, lds, as, wm, wn, lane);
  tsp::dma::barrier();  // every wave has read its last stage before the ring refills
  auto issue_p = [&](int s) {
    const uint32_t st = lds0 + (s % NST) * S::STAGE;
    sdo.issue(rdo, s, D, st, w);
    sv.issue(rv, s, D, st + S::TILE, w);
  };
  bfb::run<true, true, KC, NST>(issue_p, nsteps, lds, ap, wm, wn, lane);
  // lane holds column l32 of each 32-column tile and rows 8 (v / 4) + 4 h + v % 4.
  // Rows v and v + 1 (v even) are adjacent: neighbouring lanes swap one value
  // (DPP quad_perm [1,0,3,2]) so that the even lane stores row v's two
  // columns c, c + 1 and the odd lane row v + 1's columns c - 1, c, each as
  // one 4-byte store.
  uint32_t* pb = reinterpret_cast<uint32_t*>(P + kb * (BS * BS));
  uint32_t* db = reinterpret_cast<uint32_t*>(dS + kb * (BS * BS));
  const bool even = (lane & 1) == 0;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const int r0 = wm * 64 + 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
        const int c = wn * 64 + 32 * u + l32;
        uint32_t pw[2], dw[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int r = r0 + e;
          const float pr = __expf(scale * as[t][u][v + e] - rstat[0][r]) / rstat[1][r];
          pw[e] = tsp::f32_to_bf16_bits(pr);
          dw[e] = tsp::f32_to_bf16_bits(scale * (pr * (ap[t][u][v + e] - rstat[2][r])));
        }
        const uint32_t py = (uint32_t)__builtin_amdgcn_mov_dpp((int)(even ? pw[1] : pw[0]), 0xB1, 0xF, 0xF, false);
        const uint32_t dy = (uint32_t)__builtin_amdgcn_mov_dpp((int)(even ? dw[1] : dw[0]), 0xB1, 0xF, 0xF, false);
        const int o = even ? (r0 * BS + c) >> 1 : ((r0 + 1) * BS + c - 1) >> 1;
        pb[o] = even ? (pw[0] | (py << 16)) : (py | (pw[1] << 16));
        db[o] = even ? (dw[0] | (dy << 16)) : (dy | (dw[1] << 16));
      }
}

// dB = A^T dC, bf16: workgroup per (block column, 128-column tile) in the
// forward's schedule, walking the column's blocks.
template <int KC = SPMMT_KC, int NST = SPMMT_NST>
__global__ __launch_bounds__(256) void bsr_spmm_t_bf16_mfma(
    const uint16_t* __restrict__ blocks, const int64_t* __restrict__ cp, const int64_t* __restrict__ cbid,
    const int64_t* __restrict__ crow, int64_t nbc, int nt, const uint16_t* __restrict__ X, int64_t ldx, int64_t m,
    int64_t ncols, uint16_t* __restrict__ out, int64_t ldo, int64_t n, const int32_t* __restrict__ order) {
  using S = bfb::Slab<KC>;
  constexpr int SPB = BS / KC;  // slabs per block
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * S::STAGE];
  int64_t col;
  int ntile;
  if (!T32::tile_item(blockIdx.x, nbc, nt, order, col, ntile)) return;
  const int64_t n0 = (int64_t)ntile * BS;
  const int64_t start = cp[col];
  const int nblk = (int)(cp[col + 1] - start);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;
  f32x16 acc[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) acc[t][u] = f32x16{};
  if (nblk > 0) {
    const i32x4 rsx = tsp::dma::make_rsrc(X, (uint32_t)(m * ldx * 2));
    const uint32_t lds0 = tsp::dma::lds_addr(lds);
    int cbase = 0, idv, rowv;
    auto load_ids = [&](int base) {
      const int64_t e = start + (base + lane < nblk ? base + lane : nblk - 1);
      idv = tsp::dma::load_lo32_sync(cbid + e);
      rowv = tsp::dma::load_lo32_sync(crow + e);
    };
    load_ids(0);
    auto issue = [&](int s) {
      const int b = s / SPB;
      if (b - cbase >= 64) {
        cbase = b & ~63;
        load_ids(cbase);
      }
      const int64_t kb = __builtin_amdgcn_readlane(idv, b - cbase);
      const int64_t ib = __builtin_amdgcn_readlane(rowv, b - cbase);
      const int kk = (s % SPB) * KC;
      const uint32_t st = lds0 + (s % NST) * S::STAGE;
      bfb::dma_tr_block<KC>(blocks + kb * (BS * BS) + kk * BS, st, w, lane);
      bfb::dma_tr<KC>(rsx, ib * BS + kk, ldx, n0, st + S::TILE, w, lane);
    };
    bfb::run<false, false, KC, NST>(issue, nblk * SPB, lds, acc, wm, wn, lane);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t r0 = col * BS + wm * 64 + 32 * t + 4 * h;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t c = n0 + wn * 64 + 32 * u + l32;
      if (c < ncols) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t r = r0 + 8 * (v >> 2) + (v & 3);
          if (r < n) out[r * ldo + c] = tsp::f32_to_bf16_bits(acc[t][u][v]);
        }
      }
    }
  }
}

// ------------------------------------------------------------ fp64 MFMA
//
// fp64, b == 128, on v_mfma_f64_16x16x4_f64 with the operand tiles of
// mfma_f64.h: 4 waves of 64x64, 32-wide k-slabs of two operand tiles through
// a 2-stage direct-load ring. dA (SDDMM): both operands ROW; dB = A^T dC:
// both COL.
namespace F64 = tsp::f64tile;
namespace f64b {
namespace F = tsp::f64tile;
constexpr int NST = 2;
constexpr int STAGE = 2 * F::TILE;

template <bool AROW, bool BROW, typename Issue>
__device__ inline void run(Issue&& issue, int nsteps, const uint8_t* lds, F::f64x4 (&acc)[4][4], int wm, int wn,
                           int lane) {
  struct Ops {
    double a[4][2], b[4][2];
  };
  auto get = [&](const uint8_t* st, int p, Ops& o) {
    F::fetch<AROW>(st, wm * 64, p, lane, o.a);
    F::fetch<BROW>(st + F::TILE, wn * 64, p, lane, o.b);
  };
  if (nsteps > 0) issue(0);
  for (int s = 0; s < nsteps; ++s) {
    tsp::dma::wait_vm<0>();  // this wave's loads of slab s are done
    tsp::dma::barrier();     // every wave's part is in LDS; stage (s + 1) % NST is free
    if (s + 1 < nsteps) issue(s + 1);
    const uint8_t* st = lds + (s % NST) * STAGE;
    Ops o[2];
    get(st, 0, o[0]);
#pragma unroll
    for (int p = 0; p < F::KC / 8; ++p) {
      if (p + 1 < F::KC / 8) get(st, p + 1, o[(p + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      F::mma(o[p & 1].a, o[p & 1].b, acc);
    }
  }
}
}  // namespace f64b

// dA (SDDMM), fp64: workgroup per stored block, XCD x takes a contiguous
// range of blocks as in bsr_sddmm_f32_dma.
__global__ __launch_bounds__(256) void bsr_sddmm_f64_mfma(const double* __restrict__ G, int64_t ldg, int64_t m,
                                                          const double* __restrict__ B, int64_t ldb, int64_t n,
                                                          int64_t ncols, const int64_t* __restrict__ brow,
                                                          const int64_t* __restrict__ ci, int64_t nnzb,
                                                          double* __restrict__ out) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[f64b::NST * f64b::STAGE];
  const int64_t g = blockIdx.x, xcd = g & 7, slot = g >> 3;
  const int64_t per = tsp::ceil_div(nnzb, 8);
  const int64_t kb = xcd * per + slot;
  if (slot >= per || kb >= nnzb) return;
  const int64_t i = brow[kb], j = ci[kb];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, gq = lane >> 4, l16 = lane & 15;
  const i32x4 rsg = tsp::dma::make_rsrc(G, (uint32_t)(m * ldg * 8));
  const i32x4 rsb = tsp::dma::make_rsrc(B, (uint32_t)(n * ldb * 8));
  const uint32_t lds0 = tsp::dma::lds_addr(lds);
  auto issue = [&](int s) {
    const uint32_t st = lds0 + (s % f64b::NST) * f64b::STAGE;
    F64::dma_row(rsg, i * BS, ldg, (int64_t)s * F64::KC, ncols, st, w, lane);
    F64::dma_row(rsb, j * BS, ldb, (int64_t)s * F64::KC, ncols, st + F64::TILE, w, lane);
  };
  F64::f64x4 acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = F64::f64x4{};
  f64b::run<true, true>(issue, (int)tsp::ceil_div(ncols, F64::KC), lds, acc, wm, wn, lane);
  double* ob = out + kb * (BS * BS);
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        ob[(wm * 64 + 16 * t + gq + 4 * v) * BS + wn * 64 + 16 * u + l16] = acc[t][u][v];
}

// dB = A^T dC, fp64: workgroup per (block column, 128-column tile) in the
// forward's schedule, walking the column's blocks.
__global__ __launch_bounds__(256) void bsr_spmm_t_f64_mfma(
    const double* __restrict__ blocks, const int64_t* __restrict__ cp, const int64_t* __restrict__ cbid,
    const int64_t* __restrict__ crow, int64_t nbc, int nt, const double* __restrict__ X, int64_t ldx, int64_t m,
    int64_t ncols, double* __restrict__ out, int64_t ldo, int64_t n, const int32_t* __restrict__ order) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[f64b::NST * f64b::STAGE];
  int64_t col;
  int ntile;
  if (!T32::tile_item(blockIdx.x, nbc, nt, order, col, ntile)) return;
  const int64_t n0 = (int64_t)ntile * BS;
  const int64_t start = cp[col];
  const int nblk = (int)(cp[col + 1] - start);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, gq = lane >> 4, l16 = lane & 15;
  F64::f64x4 acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = F64::f64x4{};
  if (nblk > 0) {
    constexpr int SPB = BS / F64::KC;
    const i32x4 rsx = tsp::dma::make_rsrc(X, (uint32_t)(m * ldx * 8));
    const uint32_t lds0 = tsp::dma::lds_addr(lds);
    int cbase = 0, idv, rowv;
    auto load_ids = [&](int base) {
      const int64_t e = start + (base + lane < nblk ? base + lane : nblk - 1);
      idv = tsp::dma::load_lo32_sync(cbid + e);
      rowv = tsp::dma::load_lo32_sync(crow + e);
    };
    load_ids(0);
    auto issue = [&](int s) {
      const int b = s / SPB;
      if (b - cbase >= 64) {
        cbase = b & ~63;
        load_ids(cbase);
      }
      const int64_t kb = __builtin_amdgcn_readlane(idv, b - cbase);
      const int64_t ib = __builtin_amdgcn_readlane(rowv, b - cbase);
      const int kk = (s % SPB) * F64::KC;
      const uint32_t st = lds0 + (s % f64b::NST) * f64b::STAGE;
      F64::dma_col_block(blocks + kb * (BS * BS) + kk * BS, st, w, lane);
      F64::dma_col(rsx, ib * BS + kk, ldx, n0, st + F64::TILE, w, lane);
    };
    f64b::run<false, false>(issue, nblk * SPB, lds, acc, wm, wn, lane);
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t c = n0 + wn * 64 + 16 * u + l16;
      if (c < ncols) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t r = col * BS + wm * 64 + 16 * t + gq + 4 * v;
          if (r < n) out[r * ldo + c] = acc[t][u][v];
        }
      }
    }
}

// ------------------------------------------------------------ generic

template <typename T> __device__ inline typename tsp::Acc<T>::type ldv(const T* p) { return (typename tsp::Acc<T>::type)*p; }
template <> __device__ inline float ldv<uint16_t>(const uint16_t* p) { return tsp::bf16_bits_to_f32(*p); }
template <typename T> __device__ inline T stv(typename tsp::Acc<T>::type v) { return (T)v; }
template <> __device__ inline uint16_t stv<uint16_t>(float v) { return tsp::f32_to_bf16_bits(v); }

// dA[k][r][c] = sum_t dC[i*b + r][t] * B[j*b + c][t] (rows past m / n are zero)
template <typename T>
__global__ __launch_bounds__(256) void bsr_sddmm_generic(const T* __restrict__ G, int64_t ldg, int64_t m,
                                                         const T* __restrict__ B, int64_t ldb, int64_t n, int64_t ncols,
                                                         const int64_t* __restrict__ brow, const int64_t* __restrict__ ci,
                                                         int64_t nnzb, int64_t b, T* __restrict__ out) {
  typedef typename tsp::Acc<T>::type AccT;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nnzb * b * b) return;
  const int64_t kb = e / (b * b), rc = e - kb * b * b, r = rc / b, c = rc - r * b;
  const int64_t gr = brow[kb] * b + r, br = ci[kb] * b + c;
  AccT acc = 0;
  if (gr < m && br < n)
    for (int64_t t = 0; t < ncols; ++t) acc += ldv(G + gr * ldg + t) * ldv(B + br * ldb + t);
  out[e] = stv<T>(acc);
}

// dB[jb*b + r][c] = sum over blocks k of column jb: sum_t A_k[t][r] * dC[i_k*b + t][c]
template <typename T>
__global__ __launch_bounds__(256) void bsr_spmm_t_generic(const T* __restrict__ blocks, const int64_t* __restrict__ cp,
                                                          const int64_t* __restrict__ cbid, const int64_t* __restrict__ crow,
                                                          int64_t b, const T* __restrict__ X, int64_t ldx, int64_t m,
                                                          int64_t ncols, T* __restrict__ out, int64_t ldo, int64_t n) {
  typedef typename tsp::Acc<T>::type AccT;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n * ncols) return;
  const int64_t row = e / ncols, c = e - row * ncols;
  const int64_t jb = row / b, r = row - jb * b;
  AccT acc = 0;
  for (int64_t p = cp[jb]; p < cp[jb + 1]; ++p) {
    const T* blk = blocks + cbid[p] * b * b;
    const int64_t xr0 = crow[p] * b;
    for (int64_t t = 0; t < b; ++t) {
      if (xr0 + t >= m) break;
      acc += ldv(blk + t * b + r) * ldv(X + (xr0 + t) * ldx + c);
    }
  }
  out[row * ldo + c] = stv<T>(acc);
}

// ---------------------------------------------------------- small blocks
//
// bsr_sddmm_small<b>: dA for b = 8, 16, 32, 64 (fp32 or bf16, fp32
// accumulation): a wavefront per stored block k = (i, j), four per
// workgroup, XCD x taking the x-th eighth of the blocks (neighbouring blocks
// share block rows). dA_k = dC[rows of i] . B[rows of j]^T over the N
// columns; both operands are rows with k contiguous, so each lane reads 4
// consecutive k of its dC row and of its B row per step (k permuted the same
// way on both operands, so the products pair up):
//   b = 32, 64: v_mfma_f32_32x32x2_f32, (b/32)^2 subtiles; lane half h takes
//     k = 8g + 4h + c at step (g, c);
//   b = 16: v_mfma_f32_16x16x4_f32; lane group q takes k = 16g + 4q + c;
//   b = 8: v_mfma_f32_4x4x1_16b_f32, its 16 products = 2 x 2 subtiles of
//     4x4 x 4 k-slices: lane l feeds product l/4 = (k-slice s = (l/4) % 4,
//     subtile (l/32, (l/16) % 2)), k = 16g + 4s + c; the four k-slices are
//     summed across lanes at the end.
// Rows past m / n and columns past ncols read as zero.
template <typename T>
__device__ inline f32x4 ld4v(const T* p);
template <>
__device__ inline f32x4 ld4v<float>(const float* p) { return *(const f32x4*)p; }
template <>
__device__ inline f32x4 ld4v<uint16_t>(const uint16_t* p) {
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  const u16x4 v = *(const u16x4*)p;
  return f32x4{tsp::bf16_bits_to_f32(v[0]), tsp::bf16_bits_to_f32(v[1]), tsp::bf16_bits_to_f32(v[2]),
               tsp::bf16_bits_to_f32(v[3])};
}

// k steps of operands in flight per lane (small-block dA kernels): 3 measured
// no faster at b = 8, 16, 32 and slower at b = 64 (more registers)
constexpr int SDDMM_PF = 1;

template <int BSZ, typename T>
__global__ __launch_bounds__(256) void bsr_sddmm_small(const T* __restrict__ G, int64_t ldg, int64_t m,
                                                       const T* __restrict__ B, int64_t ldb, int64_t n, int64_t ncols,
                                                       const int64_t* __restrict__ brow, const int64_t* __restrict__ ci,
                                                       int64_t nnzb, T* __restrict__ out, int vec) {
  static_assert(BSZ == 8 || BSZ == 16 || BSZ == 32 || BSZ == 64, "block size");
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t per = gridDim.x >> 3;
  const int64_t kb = ((int64_t)(blockIdx.x & 7) * per + (blockIdx.x >> 3)) * 4 + w;
  if (kb >= nnzb) return;
  const int64_t i0 = brow[kb] * BSZ, j0 = ci[kb] * BSZ;
  // 4 consecutive k of row r of X (vec & 1: X aligned, ld % 4 == 0)
  auto ld4 = [&](const T* X, int64_t ldx, int64_t rows, int64_t r, int64_t k) {
    if (r < rows && (vec & 1) && k + 4 <= ncols) return ld4v<T>(X + r * ldx + k);
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = r < rows && k + e < ncols ? ldv(X + r * ldx + k + e) : 0.f;
    return v;
  };
  T* ob = out + kb * (BSZ * BSZ);
  if constexpr (BSZ == 8) {
    const int s4 = (lane >> 2) & 3, sc = (lane >> 4) & 1, sr = lane >> 5, l4 = lane & 3;
    const int64_t gr = i0 + 4 * sr + l4, br = j0 + 4 * sc + l4;
    f32x4 acc = {};
    const int64_t ng = tsp::ceil_div(ncols, 16);
    f32x4 a = ld4(G, ldg, m, gr, 4 * s4), b = ld4(B, ldb, n, br, 4 * s4);
    for (int64_t g = 0; g < ng; ++g) {
      const int64_t kn = 16 * (g + 1) + 4 * s4;  // the next group's k (past ncols reads as zero)
      const f32x4 an = ld4(G, ldg, m, gr, kn), bn = ld4(B, ldb, n, br, kn);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_4x4x1f32(a[c], b[c], acc, 0, 0, 0);
      a = an;
      b = bn;
    }
    // sum the four k-slices (lane bits 2 and 3)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc[r] += __shfl_xor(acc[r], 4);
      acc[r] += __shfl_xor(acc[r], 8);
    }
    if (s4 == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) ob[(4 * sr + r) * BSZ + 4 * sc + l4] = stv<T>(acc[r]);
    }
  } else if constexpr (BSZ == 16) {
    const int l16 = lane & 15, q = lane >> 4;
    const int64_t gr = i0 + l16, br = j0 + l16;
    f32x4 acc = {};
    const int64_t ng = tsp::ceil_div(ncols, 16);
    f32x4 ra[SDDMM_PF], rb[SDDMM_PF];
#pragma unroll
    for (int j = 0; j < SDDMM_PF; ++j) {
      ra[j] = ld4(G, ldg, m, gr, 16 * j + 4 * q);
      rb[j] = ld4(B, ldb, n, br, 16 * j + 4 * q);
    }
    for (int64_t g0 = 0; g0 < ng; g0 += SDDMM_PF) {
#pragma unroll
      for (int j = 0; j < SDDMM_PF; ++j) {
        if (g0 + j < ng) {
          const f32x4 a = ra[j], b = rb[j];
          const int64_t kn = 16 * (g0 + j + SDDMM_PF) + 4 * q;  // past ncols reads as zero
          ra[j] = ld4(G, ldg, m, gr, kn);
          rb[j] = ld4(B, ldb, n, br, kn);
#pragma unroll
          for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c], b[c], acc, 0, 0, 0);
        }
      }
    }
    // element r: row 4q + r, column l16
#pragma unroll
    for (int r = 0; r < 4; ++r) ob[(4 * q + r) * BSZ + l16] = stv<T>(acc[r]);
  } else {
    constexpr int RT = BSZ / 32;
    const int l32 = lane & 31, h = lane >> 5;
    f32x16 acc[RT][RT];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int u = 0; u < RT; ++u) acc[t][u] = f32x16{};
    const int64_t ng = tsp::ceil_div(ncols, 8);
    f32x4 ra[SDDMM_PF][RT], rb[SDDMM_PF][RT];
#pragma unroll
    for (int j = 0; j < SDDMM_PF; ++j)
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        ra[j][t] = ld4(G, ldg, m, i0 + 32 * t + l32, 8 * j + 4 * h);
        rb[j][t] = ld4(B, ldb, n, j0 + 32 * t + l32, 8 * j + 4 * h);
      }
    for (int64_t g0 = 0; g0 < ng; g0 += SDDMM_PF) {
#pragma unroll
      for (int j = 0; j < SDDMM_PF; ++j) {
        if (g0 + j < ng) {
          f32x4 a[RT], b[RT];
          const int64_t kn = 8 * (g0 + j + SDDMM_PF) + 4 * h;  // past ncols reads as zero
#pragma unroll
          for (int t = 0; t < RT; ++t) {
            a[t] = ra[j][t];
            b[t] = rb[j][t];
            ra[j][t] = ld4(G, ldg, m, i0 + 32 * t + l32, kn);
            rb[j][t] = ld4(B, ldb, n, j0 + 32 * t + l32, kn);
          }
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < RT; ++t)
#pragma unroll
              for (int u = 0; u < RT; ++u)
                acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t][c], b[u][c], acc[t][u], 0, 0, 0);
        }
      }
    }
    // element v of subtile (t, u): row 32t + 8(v/4) + 4h + v%4, column 32u + l32
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int u = 0; u < RT; ++u)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          ob[(32 * t + 8 * (v >> 2) + 4 * h + (v & 3)) * BSZ + 32 * u + l32] = stv<T>(acc[t][u][v]);
  }
}

// bsr_sddmm_rows<b, T>: dA at b = 8 and 16 for N up to ROWS_NMAX<b>. A
// workgroup per 64 consecutive stored blocks (XCD x taking the x-th eighth
// of the chunks). The dC rows of the chunk's first block row are staged in
// LDS (fp32, zero-padded to a multiple of 16 columns, rows 4 floats apart so
// that one read of the rows hits distinct bank groups); a lane whose block
// is in another block row reads its dC row from memory, so any block order
// is correct, and in CSR order dC is read from memory about once per 64
// blocks instead of once per block. On v_mfma_f32_16x16x4_f32 each lane
// reads 4 consecutive k of its A row and of its B row per step (16 bytes):
//   b = 16: a wavefront per block, A = the block row's 16 dC rows, B = the
//     block column's 16 B rows;
//   b = 8: a wavefront per pair of blocks (k1, k2): A rows 0-7 are the dC
//     rows of k1's block row, 8-15 those of k2's, B columns 0-7 the B rows
//     of k1's block column, 8-15 those of k2's; the diagonal 8x8 quadrants
//     of the 16x16 result are the two blocks' dA (the off-diagonal ones are
//     discarded), so no operand row is read twice.
template <int BSZ>
constexpr int rows_nmax() { return BSZ == 8 ? 2032 : 1008; }  // BSZ rows of (N + 4) floats under 64 KiB of LDS
constexpr int ROWS_CHUNK = 64;

template <int BSZ, typename T>
__global__ __launch_bounds__(256) void bsr_sddmm_rows(const T* __restrict__ G, int64_t ldg, int64_t m,
                                                      const T* __restrict__ B, int64_t ldb, int64_t n, int64_t ncols,
                                                      const int64_t* __restrict__ brow, const int64_t* __restrict__ ci,
                                                      int64_t nnzb, T* __restrict__ out, int vec) {
  static_assert(BSZ == 8 || BSZ == 16, "block size");
  constexpr int PB = 16 / BSZ;  // blocks per MFMA tile
  extern __shared__ __attribute__((aligned(16))) float gs[];  // [BSZ][ldl]
  const int64_t per = gridDim.x >> 3;
  const int64_t s0 = ((int64_t)(blockIdx.x & 7) * per + (blockIdx.x >> 3)) * ROWS_CHUNK;
  if (s0 >= nnzb) return;
  const int64_t s1 = s0 + ROWS_CHUNK < nnzb ? s0 + ROWS_CHUNK : nnzb;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ncp = (int)((ncols + 15) & ~(int64_t)15);  // columns staged (zeros past ncols)
  const int ldl = ncp + 4;
  const int64_t i0 = brow[s0];
  // 4 consecutive k of row r of X (zero past `rows` and ncols)
  auto ld4 = [&](const T* X, int64_t ldx, int64_t rows, int64_t r, int64_t k) {
    if (r < rows && (vec & 1) && k + 4 <= ncols) return ld4v<T>(X + r * ldx + k);
    f32x4 v;
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = r < rows && k + c < ncols ? ldv(X + r * ldx + k + c) : 0.f;
    return v;
  };
  for (int e = tid; e < BSZ * (ncp / 4); e += 256) {
    const int r = e / (ncp / 4), k = 4 * (e - r * (ncp / 4));
    *(f32x4*)(gs + r * ldl + k) = ld4(G, ldg, m, i0 * BSZ + r, k);
  }
  __syncthreads();
  const int l16 = lane & 15, q = lane >> 4;
  const int rl = l16 % BSZ;  // the lane's row within its block
  const int ng = ncp / 16;
  for (int64_t k1 = s0 + PB * w; k1 < s1; k1 += 4 * PB) {
    const bool two = PB == 2 && k1 + 1 < s1;
    const int64_t kl = l16 < 8 || !two ? k1 : k1 + 1;  // this lane's block (PB == 1: k1)
    const int64_t il = brow[kl];
    const int64_t br = ci[kl] * BSZ + rl;
    const bool lds_row = il == i0;
    const int64_t gr = il * BSZ + rl;
    const float* arow = gs + rl * ldl + 4 * q;
    auto lda = [&](int g) { return lds_row ? *(const f32x4*)(arow + 16 * g) : ld4(G, ldg, m, gr, 16 * (int64_t)g + 4 * q); };
    auto ldb4 = [&](int g) { return ld4(B, ldb, n, br, 16 * (int64_t)g + 4 * q); };
    // operands of SDDMM_PF steps in flight (a register ring; steps past the
    // end reload the last one)
    f32x4 acc = {};
    f32x4 ra[SDDMM_PF], rb[SDDMM_PF];
#pragma unroll
    for (int j = 0; j < SDDMM_PF; ++j) {
      ra[j] = lda(j < ng ? j : ng - 1);
      rb[j] = ldb4(j < ng ? j : ng - 1);
    }
    for (int g0 = 0; g0 < ng; g0 += SDDMM_PF) {
#pragma unroll
      for (int j = 0; j < SDDMM_PF; ++j) {
        if (g0 + j < ng) {
          const f32x4 a = ra[j], b = rb[j];
          const int gn = g0 + j + SDDMM_PF < ng ? g0 + j + SDDMM_PF : ng - 1;
          ra[j] = lda(gn);
          rb[j] = ldb4(gn);
#pragma unroll
          for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c], b[c], acc, 0, 0, 0);
        }
      }
    }
    // element r: row 4q + r, column l16 of the 16x16 tile
    if constexpr (PB == 1) {
      T* ob = out + k1 * 256;
#pragma unroll
      for (int r = 0; r < 4; ++r) ob[(4 * q + r) * 16 + l16] = stv<T>(acc[r]);
    } else {
      // diagonal quadrants: block k1 (rows and columns 0-7), k1 + 1 (8-15)
      if ((q < 2) == (l16 < 8) && (q < 2 || two)) {
        T* ob = out + (q < 2 ? k1 : k1 + 1) * 64;
#pragma unroll
        for (int r = 0; r < 4; ++r) ob[((4 * q + r) & 7) * 8 + (l16 & 7)] = stv<T>(acc[r]);
      }
    }
  }
}

template <typename T>
int launch_sddmm_small(int64_t bs, const void* G, int64_t ldg, int64_t m, const void* B, int64_t ldb, int64_t n,
                       int64_t ncols, const int64_t* brow, const int64_t* ci, int64_t nnzb, void* out, hipStream_t st) {
  const int64_t grid = tsp::ceil_div(tsp::ceil_div(nnzb, 4), 8) * 8;
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_sddmm: too many blocks");
  const int vec = ((uintptr_t)G % (4 * sizeof(T))) == 0 && ((uintptr_t)B % (4 * sizeof(T))) == 0 && ldg % 4 == 0 &&
                          ldb % 4 == 0
                      ? 1
                      : 0;
#define TSP_SD_SMALL(BSZ)                                                                                    \
  hipLaunchKernelGGL((bsr_sddmm_small<BSZ, T>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)G, ldg, m, \
                     (const T*)B, ldb, n, ncols, brow, ci, nnzb, (T*)out, vec)
  if (bs == 8 && ncols <= rows_nmax<8>()) {
    const int64_t gr = tsp::ceil_div(tsp::ceil_div(nnzb, ROWS_CHUNK), 8) * 8;
    if (gr > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_sddmm: too many blocks");
    const size_t shmem = (size_t)bs * (((ncols + 15) & ~(int64_t)15) + 4) * sizeof(float);
    hipLaunchKernelGGL((bsr_sddmm_rows<8, T>), dim3((unsigned)gr), dim3(256), shmem, st, (const T*)G, ldg, m,
                       (const T*)B, ldb, n, ncols, brow, ci, nnzb, (T*)out, vec);
    return tsp::check_launch("bsr_sddmm_rows launch");
  }
  if (bs == 8)
    TSP_SD_SMALL(8);
  else if (bs == 16)
    TSP_SD_SMALL(16);
  else if (bs == 32)
    TSP_SD_SMALL(32);
  else
    TSP_SD_SMALL(64);
#undef TSP_SD_SMALL
  return tsp::check_launch("bsr_sddmm_small launch");
}

bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

}  // namespace

extern "C" int tsp_bsr_sddmm(const void* G, int64_t ldg, int64_t m, const void* B, int64_t ldb, int64_t n,
                             int64_t ncols, const int64_t* block_rows, const int64_t* block_col_indices,
                             int64_t n_blocks, int64_t block_size, int dtype, void* grad_blocks, void* stream) {
  if (dtype != TSP_F32 && dtype != TSP_F64 && dtype != TSP_BF16)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_sddmm: dtype %d not supported", dtype);
  if (block_size <= 0 || m < 0 || n < 0 || ncols < 0 || n_blocks < 0) return tsp::fail(TSP_EINVAL, "tsp_bsr_sddmm: bad size");
  if (ldg < ncols || ldb < ncols) return tsp::fail(TSP_EINVAL, "tsp_bsr_sddmm: leading dimension < ncols");
  if (n_blocks == 0) return TSP_OK;
  if (!G || !B || !block_rows || !block_col_indices || !grad_blocks) return tsp::fail(TSP_EINVAL, "tsp_bsr_sddmm: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TSP_F32 && block_size == BS && ncols % 4 == 0 && ldg % 4 == 0 && ldb % 4 == 0 && aligned16(G) &&
      aligned16(B) && (m + BS) * ldg * 4 <= (int64_t)UINT32_MAX - 64 && (n + BS) * ldb * 4 <= (int64_t)UINT32_MAX - 64) {
    const int64_t grid = tsp::ceil_div(n_blocks, 8) * 8;
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_sddmm: too many blocks");
    hipLaunchKernelGGL(bsr_sddmm_f32_dma, dim3((unsigned)grid), dim3(256), 0, st, (const float*)G, ldg, m,
                       (const float*)B, ldb, n, ncols, block_rows, block_col_indices, n_blocks, (float*)grad_blocks);
    return tsp::check_launch("bsr_sddmm_f32_dma launch");
  }
  if (dtype == TSP_BF16 && block_size == BS && ncols % 8 == 0 && ldg % 8 == 0 && ldb % 8 == 0 && aligned16(G) &&
      aligned16(B) && (m + BS) * ldg * 2 <= (int64_t)UINT32_MAX - 64 && (n + BS) * ldb * 2 <= (int64_t)UINT32_MAX - 64) {
    const int64_t grid = tsp::ceil_div(n_blocks, 8) * 8;
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_sddmm: too many blocks");
    hipLaunchKernelGGL((bsr_sddmm_bf16_mfma<uint16_t>), dim3((unsigned)grid), dim3(256), 0, st, (const uint16_t*)G,
                       ldg, m, (const uint16_t*)B, ldb, n, ncols, block_rows, block_col_indices, n_blocks,
                       (uint16_t*)grad_blocks);
    return tsp::check_launch("bsr_sddmm_bf16_mfma launch");
  }
  if (dtype == TSP_F64 && block_size == BS && ncols % 2 == 0 && ldg % 2 == 0 && ldb % 2 == 0 && aligned16(G) &&
      aligned16(B) && (m + BS) * ldg * 8 <= (int64_t)UINT32_MAX - 64 && (n + BS) * ldb * 8 <= (int64_t)UINT32_MAX - 64) {
    const int64_t grid = tsp::ceil_div(n_blocks, 8) * 8;
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_sddmm: too many blocks");
    hipLaunchKernelGGL(bsr_sddmm_f64_mfma, dim3((unsigned)grid), dim3(256), 0, st, (const double*)G, ldg, m,
                       (const double*)B, ldb, n, ncols, block_rows, block_col_indices, n_blocks, (double*)grad_blocks);
    return tsp::check_launch("bsr_sddmm_f64_mfma launch");
  }
  if (block_size == 8 || block_size == 16 || block_size == 32 || block_size == 64) {
    if (dtype == TSP_F32)
      return launch_sddmm_small<float>(block_size, G, ldg, m, B, ldb, n, ncols, block_rows, block_col_indices, n_blocks,
                                       grad_blocks, st);
    if (dtype == TSP_BF16)
      return launch_sddmm_small<uint16_t>(block_size, G, ldg, m, B, ldb, n, ncols, block_rows, block_col_indices,
                                          n_blocks, grad_blocks, st);
  }
  const int64_t total = n_blocks * block_size * block_size;
  const int64_t grid = tsp::ceil_div(total, 256);
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_sddmm: too large for the generic kernel");
#define SDDMM_GEN(T)                                                                                              \
  hipLaunchKernelGGL((bsr_sddmm_generic<T>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)G, ldg, m, (const T*)B, \
                     ldb, n, ncols, block_rows, block_col_indices, n_blocks, block_size, (T*)grad_blocks)
  if (dtype == TSP_F32)
    SDDMM_GEN(float);
  else if (dtype == TSP_F64)
    SDDMM_GEN(double);
  else
    SDDMM_GEN(uint16_t);
#undef SDDMM_GEN
  return tsp::check_launch("bsr_sddmm_generic launch");
}

extern "C" int tsp_bsr_sddmm_ex(const void* G, int64_t ldg, int64_t m, const void* B, int64_t ldb, int64_t n,
                                int64_t ncols, const int64_t* block_rows, const int64_t* block_col_indices,
                                int64_t n_blocks, int64_t block_size, int dtype, void* out_blocks, int out_dtype,
                                void* stream) {
  if (out_dtype == dtype)
    return tsp_bsr_sddmm(G, ldg, m, B, ldb, n, ncols, block_rows, block_col_indices, n_blocks, block_size, dtype,
                         out_blocks, stream);
  if (dtype != TSP_BF16 || out_dtype != TSP_F32)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_sddmm_ex: dtype %d with out_dtype %d (bf16 -> f32 or equal dtypes)",
                     dtype, out_dtype);
  if (block_size <= 0 || m < 0 || n < 0 || ncols < 0 || n_blocks < 0) return tsp::fail(TSP_EINVAL, "tsp_bsr_sddmm_ex: bad size");
  if (ldg < ncols || ldb < ncols) return tsp::fail(TSP_EINVAL, "tsp_bsr_sddmm_ex: leading dimension < ncols");
  if (n_blocks == 0) return TSP_OK;
  if (!G || !B || !block_rows || !block_col_indices || !out_blocks) return tsp::fail(TSP_EINVAL, "tsp_bsr_sddmm_ex: null pointer");
  if (!(block_size == BS && ncols % 8 == 0 && ldg % 8 == 0 && ldb % 8 == 0 && aligned16(G) && aligned16(B) &&
        (m + BS) * ldg * 2 <= (int64_t)UINT32_MAX - 64 && (n + BS) * ldb * 2 <= (int64_t)UINT32_MAX - 64))
    return tsp::fail(TSP_EUNSUPPORTED,
                     "tsp_bsr_sddmm_ex: bf16 -> f32 needs block_size 128, ncols / ldg / ldb multiples of 8, 16-byte "
                     "aligned operands under 4 GiB");
  const int64_t grid = tsp::ceil_div(n_blocks, 8) * 8;
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_sddmm_ex: too many blocks");
  hipLaunchKernelGGL((bsr_sddmm_bf16_mfma<float, SCORES_KC, SCORES_NST>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)G, ldg, m, (const uint16_t*)B, ldb, n, ncols, block_rows, block_col_indices,
                     n_blocks, (float*)out_blocks);
  return tsp::check_launch("bsr_sddmm_bf16_mfma<float> launch");
}

extern "C" int tsp_bsa_block_pgrad(const void* Q, const void* K, const void* V, const void* dO, int dtype,
                                   int64_t rows, int64_t head_dim, const int64_t* block_rows,
                                   const int64_t* block_col_indices, int64_t n_blocks, int64_t block_size,
                                   double scale, const float* row_max, const float* row_denom, const float* Drow,
                                   void* P, void* dS, void* stream) {
  if (dtype != TSP_BF16) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_block_pgrad: dtype %d (bf16 only)", dtype);
  if (block_size != BS) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_block_pgrad: block_size %lld (128 only)", (long long)block_size);
  if (rows < 0 || head_dim <= 0 || n_blocks < 0) return tsp::fail(TSP_EINVAL, "tsp_bsa_block_pgrad: bad size");
  if (n_blocks == 0) return TSP_OK;
  if (!Q || !K || !V || !dO || !block_rows || !block_col_indices || !row_max || !row_denom || !Drow || !P || !dS)
    return tsp::fail(TSP_EINVAL, "tsp_bsa_block_pgrad: null pointer");
  if (head_dim % 8 || !aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(dO) ||
      rows * head_dim * 2 > (int64_t)UINT32_MAX - 64)
    return tsp::fail(TSP_EUNSUPPORTED,
                     "tsp_bsa_block_pgrad: head_dim a multiple of 8, 16-byte aligned operands under 4 GiB");
  const int64_t grid = tsp::ceil_div(n_blocks, 8) * 8;
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_block_pgrad: too many blocks");
  hipLaunchKernelGGL((bsa_block_pgrad_bf16<>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)Q,
                     (const uint16_t*)K, (const uint16_t*)V, (const uint16_t*)dO, rows, head_dim, block_rows,
                     block_col_indices, n_blocks, (float)scale, row_max, row_denom, Drow, (uint16_t*)P,
                     (uint16_t*)dS);
  return tsp::check_launch("bsa_block_pgrad_bf16 launch");
}

extern "C" int tsp_bsr_spmm_t(const void* blocks, int dtype, const int64_t* col_ptrs, const int64_t* col_block_ids,
                              const int64_t* col_block_rows, int64_t n_block_cols, int64_t block_size, int64_t m,
                              int64_t n, const void* X, int64_t ldx, int64_t ncols, void* out, int64_t ldo,
                              const int32_t* col_order, void* stream) {
  if (dtype != TSP_F32 && dtype != TSP_F64 && dtype != TSP_BF16)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm_t: dtype %d not supported", dtype);
  if (block_size <= 0 || m < 0 || n < 0 || ncols < 0 || n_block_cols < 0) return tsp::fail(TSP_EINVAL, "tsp_bsr_spmm_t: bad size");
  if (ldx < ncols || ldo < ncols) return tsp::fail(TSP_EINVAL, "tsp_bsr_spmm_t: leading dimension < ncols");
  if (n == 0 || ncols == 0) return TSP_OK;
  if (n_block_cols != tsp::ceil_div(n, block_size)) return tsp::fail(TSP_EINVAL, "tsp_bsr_spmm_t: n_block_cols != ceil(n / block_size)");
  // blocks is only read for stored blocks (it may be null for an empty pattern)
  if (!col_ptrs || !col_block_ids || !col_block_rows || !out || !X) return tsp::fail(TSP_EINVAL, "tsp_bsr_spmm_t: null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == TSP_F32 && block_size == BS && ldx % 4 == 0 && aligned16(X) && aligned16(blocks) &&
      (m + BS) * ldx * 4 + 4 * BS <= (int64_t)UINT32_MAX) {
    const int64_t nt = tsp::ceil_div(ncols, BS);
    const int64_t grid = tsp::ceil_div(n_block_cols, 8) * 8 * nt;
    if (grid > INT32_MAX || nt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm_t: problem too large");
    hipLaunchKernelGGL(bsr_spmm_t_f32_dma, dim3((unsigned)grid), dim3(256), 0, st, (const float*)blocks, col_ptrs,
                       col_block_ids, col_block_rows, n_block_cols, (int)nt, (const float*)X, ldx, m, ncols, (float*)out,
                       ldo, n, col_order);
    return tsp::check_launch("bsr_spmm_t_f32_dma launch");
  }
  if (dtype == TSP_BF16 && block_size == BS && ldx % 8 == 0 && aligned16(X) && aligned16(blocks) &&
      (m + BS) * ldx * 2 + 2 * BS <= (int64_t)UINT32_MAX) {
    const int64_t nt = tsp::ceil_div(ncols, BS);
    const int64_t grid = tsp::ceil_div(n_block_cols, 8) * 8 * nt;
    if (grid > INT32_MAX || nt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm_t: problem too large");
    hipLaunchKernelGGL((bsr_spmm_t_bf16_mfma<>), dim3((unsigned)grid), dim3(256), 0, st, (const uint16_t*)blocks, col_ptrs,
                       col_block_ids, col_block_rows, n_block_cols, (int)nt, (const uint16_t*)X, ldx, m, ncols,
                       (uint16_t*)out, ldo, n, col_order);
    return tsp::check_launch("bsr_spmm_t_bf16_mfma launch");
  }
  if (dtype == TSP_F64 && block_size == BS && ldx % 2 == 0 && aligned16(X) && aligned16(blocks) &&
      (m + BS) * ldx * 8 + 8 * BS <= (int64_t)UINT32_MAX) {
    const int64_t nt = tsp::ceil_div(ncols, BS);
    const int64_t grid = tsp::ceil_div(n_block_cols, 8) * 8 * nt;
    if (grid > INT32_MAX || nt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm_t: problem too large");
    hipLaunchKernelGGL(bsr_spmm_t_f64_mfma, dim3((unsigned)grid), dim3(256), 0, st, (const double*)blocks, col_ptrs,
                       col_block_ids, col_block_rows, n_block_cols, (int)nt, (const double*)X, ldx, m, ncols,
                       (double*)out, ldo, n, col_order);
    return tsp::check_launch("bsr_spmm_t_f64_mfma launch");
  }
  if ((block_size == 8 || block_size == 16 || block_size == 32 || block_size == 64) &&
      (dtype == TSP_F32 || dtype == TSP_BF16))
    return tsp::launch_bsr_small_t(dtype, block_size, blocks, col_ptrs, col_block_rows, col_block_ids, n_block_cols, m,
                                   n, X, ldx, ncols, out, ldo, st);
  const int64_t grid = tsp::ceil_div(n * ncols, 256);
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm_t: too large for the generic kernel");
#define SPMMT_GEN(T)                                                                                                     \
  hipLaunchKernelGGL((bsr_spmm_t_generic<T>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)blocks, col_ptrs,      \
                     col_block_ids, col_block_rows, block_size, (const T*)X, ldx, m, ncols, (T*)out, ldo, n)
  if (dtype == TSP_F32)
    SPMMT_GEN(float);
  else if (dtype == TSP_F64)
    SPMMT_GEN(double);
  else
    SPMMT_GEN(uint16_t);
#undef SPMMT_GEN
  return tsp::check_launch("bsr_spmm_t_generic launch");
}
