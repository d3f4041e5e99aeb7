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
//                      (v_mfma_f32_32x32x16_bf16, 64x32 wave tiles,
//                      direct-to-LDS 4-deep ring, B operand through LDS
//                      transpose reads).
//   bsr_spmm_f64_dma   b == 128, fp64 (v_mfma_f64_16x16x4_f64, the streamed
//                      structure of bsr_spmm_f32_dma).
//   bsr_spmm_small<b>  b in {8, 16, 32, 64}, fp32 or bf16 in (fp32 MFMA,
//                      bf16 widened exactly at the load), fp32 / bf16 out: a
//                      wavefront per (block row, 64 columns of C), operands
//                      straight from memory into MFMA registers (b = 8 on
//                      the 16-product 4x4x1 form).
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

#include "lds_dma.h"
#include "mfma_f32.h"
#include "mfma_f64.h"

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

// ------------------------------------------------------- fp32 MFMA, streamed
//
// bsr_spmm_f32_dma<KC>: b == 128, fp32. Same tile (128x128 of C per
// workgroup, one block row x one 128-column tile) and scheduling (tile_item:
// heaviest rows first, boustrophedon over the XCDs) as bsr_spmm_f32_mfma,
// restructured for issue efficiency:
//   * 4 waves, each a 64x64 sub-tile as four independent 32x32
//     v_mfma_f32_32x32x2_f32 accumulators: per 8 k a wave reads two 16-byte
//     A fragments and four 8-byte B pairs for 16 MFMAs. The two column
//     subtiles of a wave interleave (subtile u holds columns wn*64 + 2j + u,
//     j = lane % 32), so one 8-byte read of a B row feeds both, and the
//     epilogue stores the two subtiles' values as one 8-byte pair;
//   * KC-wide k-slabs of A (128 x KC) and B (KC x 128) stream through a
//     2-stage LDS ring by direct global->LDS loads issued one slab ahead
//     (a slab is ~KC*128 MFMA cycles per SIMD, ample time for the loads);
//     B through a buffer resource, so rows past n read as zero;
//   * k is permuted within each 8-k group as in the other MFMA kernels (lane
//     half h takes k0 + 4h + s at k-step s), so a lane's four A values are one
//     16-byte read;
//   * swizzles for the 64-bank LDS: A rows of KC*4 bytes, chunk ^ (row % 16)
//     for 256-byte rows or chunk ^ ((row / 2) % 8) for 128-byte rows, so 16
//     consecutive rows of one b128 read cover all banks; B rows (512 B)
//     chunk ^ 8*((k / 4) % 2), so the two lane halves (k rows 4 apart) of an
//     8-byte read land in different bank halves.
// KC = 64 (128 KiB ring, one workgroup per CU, so the in-order dispatcher
// list-schedules the ranked rows) measured faster on cfg3a than KC = 32
// (64 KiB, two workgroups per CU): 237 us vs 263 us; KC = 32 with 4 or 3
// stages (one workgroup per CU) 245 and 247 us against 235 us. The paired B
// reads took cfg3a from 238.6 to 235.3 us.
template <int KC_, int NST_ = 2>
struct F32S {
  static constexpr int KC = KC_;
  static constexpr int A_ROWB = KC * 4;
  static constexpr int B_ROWB = 128 * 4;
  static constexpr int A_BYTES = 128 * A_ROWB;
  static constexpr int B_BYTES = KC * B_ROWB;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int NST = NST_;
  static_assert(NST >= 2 && NST <= 4, "ring depths with a vmcnt schedule");
  static constexpr int CPR = A_ROWB / 16;     // 16-byte chunks per A row
  // A: slot of logical chunk c in row r (an involution)
  static __device__ int aswz(int c, int r) { return CPR == 16 ? (c ^ (r & 15)) : (c ^ ((r >> 1) & 7)); }
};

template <int KC_, int NST_ = 2>
__global__ __launch_bounds__(256) void bsr_spmm_f32_dma(
    const float* __restrict__ blocks, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci,
    int64_t mb, int nt, int64_t m, int64_t n, const float* __restrict__ B, int64_t ldb, int64_t ncols,
    float* __restrict__ C, int64_t ldc, const int32_t* __restrict__ order) {
  typedef F32S<KC_, NST_> G;
  constexpr int SK = G::KC;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[G::NST * G::STAGE];
  int64_t row;
  int ntile;
  if (!T32::tile_item(blockIdx.x, mb, nt, order, row, ntile)) return;
  const int64_t n0 = (int64_t)ntile * 128;
  const int64_t start = rp[row];
  const int nblk = (int)(rp[row + 1] - start);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;

  f32x16 acc[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) acc[t][u] = f32x16{};

  if (nblk > 0) {
    const tsp::dma::i32x4 brsrc = tsp::dma::make_rsrc(B, (uint32_t)(n * ldb * 4));
    const uint32_t lds0 = tsp::dma::lds_addr(lds);
    int cbase = 0;
    auto load_cols = [&](int base) {
      const int i = base + lane < nblk ? base + lane : nblk - 1;
      return tsp::dma::load_lo32_sync(ci + start + i);
    };
    int cv = load_cols(0);
    auto colblk = [&](int blk) {
      if (blk - cbase >= 64) {
        cbase = blk & ~63;
        cv = load_cols(cbase);
      }
      return __builtin_amdgcn_readlane(cv, blk - cbase);
    };

    // ---- loads of slab s into stage s % NST (1 KiB per wave instruction)
    constexpr int A_INS = G::A_BYTES / 1024 / 4;  // per wave
    constexpr int B_INS = G::B_BYTES / 1024 / 4;
    constexpr int A_RPI = 1024 / G::A_ROWB;       // A rows per instruction
    auto issue = [&](int s) {
      constexpr int SPB = BS / SK;                // slabs per block
      const int blk = s / SPB;
      const int kk = (s % SPB) * SK;
      const uint32_t st = lds0 + (s % G::NST) * G::STAGE;
      const float* ablk = blocks + (start + blk) * (BS * BS) + kk;
#pragma unroll
      for (int q = 0; q < A_INS; ++q) {
        const int i = A_INS * w + q;
        const int r = A_RPI * i + lane / G::CPR;
        const int c = G::aswz(lane % G::CPR, r);  // logical chunk held at this lane's slot
        tsp::dma::global16(ablk + r * BS + c * 4, st + i * 1024);
      }
      const int64_t brow0 = (int64_t)colblk(blk) * BS + kk;
#pragma unroll
      for (int q = 0; q < B_INS; ++q) {
        const int j = B_INS * w + q;              // B slab rows 2j, 2j+1
        const int rr = 2 * j + (lane >> 5);
        const int c = (lane & 31) ^ (8 * ((rr >> 2) & 1));
        const int64_t off = ((brow0 + rr) * ldb + n0 + c * 4) * 4;
        tsp::dma::buffer16(brsrc, (uint32_t)off, st + G::A_BYTES + j * 1024);
      }
    };

    // per-lane LDS offsets: A rows wm*64 + 32t + l32 (the swizzle term is the
    // same for both t); B columns wn*64 + 2*l32 + u, rows 8g + 4h + s
    const int arow = wm * 64 + l32;
    // subtile u holds columns wn*64 + 2*l32 + u: one b64 read serves both
    const int bc2 = wn * 64 + 2 * l32;
    const int boff2 = (((bc2 >> 2) ^ (8 * h)) * 16) + (bc2 & 3) * 4 + 4 * h * G::B_ROWB;
    struct Ops {
      f32x4 a[2];
      float b[2][4];
    };
    auto fetch = [&](const uint8_t* st, int g, Ops& o) {
      const uint8_t* As = st + arow * G::A_ROWB + G::aswz(2 * g + h, arow) * 16;
      o.a[0] = *(const f32x4*)(As);
      o.a[1] = *(const f32x4*)(As + 32 * G::A_ROWB);
      const uint8_t* Bs = st + G::A_BYTES + 8 * g * G::B_ROWB;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const f32x2 bb = *(const f32x2*)(Bs + s * G::B_ROWB + boff2);
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
    auto compute = [&](const uint8_t* st) {
      Ops o[2];
      fetch(st, 0, o[0]);
#pragma unroll
      for (int g = 0; g < SK / 8; ++g) {
        if (g + 1 < SK / 8) fetch(st, g + 1, o[(g + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
        mma(o[g & 1]);
      }
    };

    const int nsteps = nblk * (BS / SK);
    constexpr int LPS = A_INS + B_INS;  // loads per slab per wave
    const int pre = nsteps < G::NST - 1 ? nsteps : G::NST - 1;
    for (int s = 0; s < pre; ++s) issue(s);
    for (int s = 0; s < nsteps; ++s) {
      // this wave's loads of slab s are done when only the later slabs
      // already issued (at most NST - 2) are in flight
      const int later0 = nsteps - 1 - s;
      const int later = later0 < G::NST - 2 ? later0 : G::NST - 2;
      if (G::NST >= 4 && later >= 2)
        tsp::dma::wait_vm<(G::NST >= 4 ? 2 * LPS : 0)>();
      else if (G::NST >= 3 && later >= 1)
        tsp::dma::wait_vm<(G::NST >= 3 ? LPS : 0)>();
      else
        tsp::dma::wait_vm<0>();
      tsp::dma::barrier();     // every wave's part is in LDS; stage (s - 1) % NST is free
      if (s + G::NST - 1 < nsteps) issue(s + G::NST - 1);
      compute(lds + (s % G::NST) * G::STAGE);
    }
  }
  // accumulator layout: lane holds rows 8*(v/4) + 4*h + v%4 of columns
  // wn*64 + 2*l32 + u (subtile u)
  const int64_t c = n0 + wn * 64 + 2 * l32;
  const bool pair = c + 1 < ncols && (ldc & 1) == 0 && ((uintptr_t)C & 7) == 0;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t r0 = row * BS + wm * 64 + 32 * t + 4 * h;
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

#ifndef F32_DMA_KC
#define F32_DMA_KC 64
#endif

// ------------------------------------------------------- fp64 MFMA, streamed
//
// bsr_spmm_f64_dma: b == 128, fp64. The tile, scheduling and slab ring of
// bsr_spmm_f32_dma with v_mfma_f64_16x16x4_f64 (64 cycles per MFMA, the
// same cadence per slab as the fp32 kernel's 32x32x2) on the operand tiles
// of mfma_f64.h: 4 waves of 64x64 (4x4 independent 16x16 accumulators),
// 32-wide k-slabs of A as a ROW tile [128][32] (from the block, always in
// bounds) and B as a COL tile [32][128] (through a buffer resource, rows
// past n read as zero) in a 2-stage direct-to-LDS ring (128 KiB).
__global__ __launch_bounds__(256) void bsr_spmm_f64_dma(
    const double* __restrict__ blocks, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci,
    int64_t mb, int nt, int64_t m, int64_t n, const double* __restrict__ B, int64_t ldb, int64_t ncols,
    double* __restrict__ C, int64_t ldc, const int32_t* __restrict__ order) {
  namespace F = tsp::f64tile;
  constexpr int NST = 2, STAGE = 2 * F::TILE;
  constexpr int SPB = BS / F::KC;  // slabs per block
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];
  int64_t row;
  int ntile;
  if (!T32::tile_item(blockIdx.x, mb, nt, order, row, ntile)) return;
  const int64_t n0 = (int64_t)ntile * 128;
  const int64_t start = rp[row];
  const int nblk = (int)(rp[row + 1] - start);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, g = lane >> 4, l16 = lane & 15;

  F::f64x4 acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = F::f64x4{};

  if (nblk > 0) {
    const tsp::dma::i32x4 brsrc = tsp::dma::make_rsrc(B, (uint32_t)(n * ldb * 8));
    const uint32_t lds0 = tsp::dma::lds_addr(lds);
    int cbase = 0;
    auto load_cols = [&](int base) {
      const int i = base + lane < nblk ? base + lane : nblk - 1;
      return tsp::dma::load_lo32_sync(ci + start + i);
    };
    int cv = load_cols(0);
    auto colblk = [&](int blk) {
      if (blk - cbase >= 64) {
        cbase = blk & ~63;
        cv = load_cols(cbase);
      }
      return __builtin_amdgcn_readlane(cv, blk - cbase);
    };
    // ---- loads of slab s into stage s % NST: 8 A + 8 B wave instructions
    auto issue = [&](int s) {
      const int blk = s / SPB;
      const int kk = (s % SPB) * F::KC;
      const uint32_t st = lds0 + (s % NST) * STAGE;
      F::dma_row_block(blocks + (start + blk) * (BS * BS) + kk, st, w, lane);
      F::dma_col(brsrc, (int64_t)colblk(blk) * BS + kk, ldb, n0, st + F::TILE, w, lane);
    };
    struct Ops {
      double a[4][2], b[4][2];
    };
    auto get = [&](const uint8_t* st, int p, Ops& o) {
      F::fetch<true>(st, wm * 64, p, lane, o.a);
      F::fetch<false>(st + F::TILE, wn * 64, p, lane, o.b);
    };
    const int nsteps = nblk * SPB;
    issue(0);
    for (int s = 0; s < nsteps; ++s) {
      tsp::dma::wait_vm<0>();  // this wave's loads of slab s are done
      tsp::dma::barrier();     // every wave's part is in LDS; stage (s+1) % NST is free
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
  // accumulator layout of v_mfma_f64_16x16x4_f64 (checked on the device):
  // lane holds column l16 and rows g + 4*v (unlike the fp32 16x16 forms,
  // whose lane group g owns the 4 consecutive rows 4*g .. 4*g + 3)
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t r0 = row * BS + wm * 64 + 16 * t + g;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t c = n0 + wn * 64 + 16 * u + l16;
      if (c < ncols) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t r = r0 + 4 * v;
          if (r < m) C[r * ldc + c] = acc[t][u][v];
        }
      }
    }
  }
}

// ---------------------------------------------------------------- bf16 MFMA
//
// bsr_spmm_bf16_mfma: b == 128, bf16 operands, fp32 accumulation, fp32 or
// bf16 output. Same tile (128x128 of C per workgroup) and scheduling as the
// fp32 kernel, with v_mfma_f32_32x32x16_bf16 on 64-wide k-slabs; the 8 waves
// form a 2(M) x 4(N) grid of 64x32 wave tiles. A bf16 slab is only ~512 MFMA
// cycles per SIMD, far shorter than a memory round trip, so slabs stream
// through a 4-deep LDS ring filled by direct global->LDS loads (no register
// staging), issued 3 slabs ahead:
//   A: global_load_lds_dwordx4 of the block (always in bounds);
//   B: buffer_load_dwordx4 ... lds with a buffer resource over B, so rows
//      past n read as zero (columns past ncols only feed output columns that
//      are not stored).
// B stays [k][n] in LDS and the MFMA B operand (8 consecutive k per lane) is
// read with ds_read_b64_tr_b16: in each 16-lane group, lane i receives
// element i%4 of the 8-byte pieces given by lanes 4t + i/4, t = 0..3, i.e.
// column n_base + i of four consecutive k rows when lane j points at row
// k0 + j/4, columns n_base + 4(j%4).
// LDS budget (gfx950: 64 banks of 4 bytes; b128 reads ~256 B/clk per CU,
// transpose reads half that): 16-byte chunks are XOR-swizzled so both read
// kinds are conflict-free — A rows of 128 B: chunk ^ ((row/2) % 8), so 16
// consecutive rows cover all 64 banks; B rows of 256 B: chunk ^ 4*(row % 4),
// so the four k rows of one transpose read land on distinct banks. The
// 64x32 wave tile puts the larger share of operand bytes on the fast b128
// path (2 KB of A, 1 KB of B per 16-k step and two MFMAs).
#ifndef BF16_NST
#define BF16_NST 4
#endif
namespace bf {
constexpr int KC = 64;
constexpr int NST = BF16_NST;              // LDS ring depth
constexpr int A_BYTES = 128 * KC * 2;      // 16 KiB, rows of 128 B
constexpr int B_BYTES = KC * 128 * 2;      // 16 KiB, rows of 256 B
constexpr int STAGE = A_BYTES + B_BYTES;   // 32 KiB
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
}  // namespace bf

template <typename OutT>
__global__ __launch_bounds__(512) void bsr_spmm_bf16_mfma(
    const uint16_t* __restrict__ blocks, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci,
    int64_t mb, int nt, int64_t m, int64_t n, const uint16_t* __restrict__ B, int64_t ldb, int64_t ncols,
    OutT* __restrict__ C, int64_t ldc, const int32_t* __restrict__ order) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[bf::NST * bf::STAGE];
  int64_t row;
  int ntile;
  if (!T32::tile_item(blockIdx.x, mb, nt, order, row, ntile)) return;
  const int64_t n0 = (int64_t)ntile * 128;
  const int64_t start = rp[row];
  const int nblk = (int)(rp[row + 1] - start);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1, h = lane >> 5, l32 = lane & 31;
  // buffer resource over B (rows past n read as zero)
  const tsp::dma::i32x4 brsrc = tsp::dma::make_rsrc(B, (uint32_t)(n * ldb * 2));
  const uint32_t lds0 = tsp::dma::lds_addr(lds);

  // Column-block indices of the row, 64 at a time in one VGPR (lane i holds
  // block cbase + i), read out with readlane: no scalar load (and its wait)
  // on the slab path.
  if (nblk <= 0) {
    // empty block row: zero tile
    f32x16 z = {};
    T32::Coords<64> q;
    T32::store_tile(C, ldc, row * BS, n0, m, ncols, q, z, z, cvt_out<OutT>);
    return;
  }
  int cbase = 0;
  auto load_cols = [&](int base) {
    const int i = base + lane < nblk ? base + lane : nblk - 1;
    return tsp::dma::load_lo32_sync(ci + start + i);
  };
  int cv = load_cols(0);
  auto colblk = [&](int blk) {
    if (blk - cbase >= 64) {
      cbase = blk & ~63;
      cv = load_cols(cbase);
    }
    return __builtin_amdgcn_readlane(cv, blk - cbase);
  };

  // ---- loads of slab s into ring stage s % NST: 2 A + 2 B wave instructions
  auto issue = [&](int s) {
    const int blk = s >> 1;
    const int64_t idx = start + blk;
    const int kk = (s & 1) * bf::KC;
    const uint32_t st = lds0 + (s % bf::NST) * bf::STAGE;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = 2 * w + q;                          // A rows [8i, 8i+8)
      const int r = 8 * i + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);        // logical chunk held at this lane's LDS slot
      const uint16_t* g = blocks + idx * (BS * BS) + r * BS + kk + c * 8;
      tsp::dma::global16(g, st + i * 1024);
    }
    const int64_t brow0 = (int64_t)colblk(blk) * BS + kk;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int j = 2 * w + q;                          // B slab rows [4j, 4j+4)
      const int rr = 4 * j + (lane >> 4);
      const int c = (lane & 15) ^ (4 * (rr & 3));
      const int64_t off = ((brow0 + rr) * ldb + n0 + c * 8) * 2;
      tsp::dma::buffer16(brsrc, (uint32_t)off, st + bf::A_BYTES + j * 1024);
    }
  };

  // ---- per-lane LDS read offsets (wave tile: rows wm*64 + [0,64), columns wn*32 + [0,32))
  // A operand: rows am and am + 32 (same swizzle), logical chunk 2*ks + h
  const int am = wm * 64 + l32;
  const int asw = (am >> 1) & 7;
  // B operand (tr reads): 16-lane group g = lane/16, lane j in group
  const int gq = lane >> 4, jq = lane & 15;
  const int bkq = 8 * (gq >> 1) + (jq >> 2);            // k row within the 16-k step (plus 4*kq)
  const int ncol = wn * 32 + 16 * (gq & 1) + 4 * (jq & 3);
  const int bsw = 4 * (jq >> 2);                        // 4 * (k row % 4)

  f32x16 acc0 = {}, acc1 = {};
  auto compute = [&](const uint8_t* st) {
    const uint8_t* As = st;
    const uint8_t* Bs = st + bf::A_BYTES;
#pragma unroll
    for (int ks = 0; ks < bf::KC / 16; ++ks) {
      const int ca = ((2 * ks + h) ^ asw) * 16;
      const bf16x8 a0 = *(const bf16x8*)(As + am * 128 + ca);
      const bf16x8 a1 = *(const bf16x8*)(As + (am + 32) * 128 + ca);
      bf::s16x4 v[2];
#pragma unroll
      for (int kq = 0; kq < 2; ++kq) {
        const int rr = 16 * ks + bkq + 4 * kq;
        const uint8_t* p = Bs + rr * 256 + (((ncol >> 3) ^ bsw) * 16) + (ncol & 4) * 2;
        v[kq] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((bf::lds_s16x4*)(p));
      }
      // whole-vector reinterpretation: k = 4*kq + e (per-element bf16 casts
      // of the i16 lanes are mis-packed by the compiler)
      const bf16x8 bop = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7));
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, bop, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, bop, acc1, 0, 0, 0);
    }
  };

  const int nsteps = nblk * (BS / bf::KC);
  const int pre = nsteps < bf::NST - 1 ? nsteps : bf::NST - 1;
  for (int s = 0; s < pre; ++s) issue(s);
  for (int s = 0; s < nsteps; ++s) {
    // this wave's loads of slab s are done when at most the later slabs' are in flight
    // (4 loads per slab per wave; up to NST-2 later slabs may be in flight)
    const int later = nsteps - 1 - s;
    if (bf::NST >= 5 && later >= 3)
      tsp::dma::wait_vm<12>();
    else if (later >= 2)
      tsp::dma::wait_vm<8>();
    else if (later == 1)
      tsp::dma::wait_vm<4>();
    else
      tsp::dma::wait_vm<0>();
    tsp::dma::barrier();  // every wave's part of slab s is in LDS; stage (s-1)%NST is free
    if (s + bf::NST - 1 < nsteps) issue(s + bf::NST - 1);
    compute(lds + (s % bf::NST) * bf::STAGE);
  }
  // accumulator layout: lane holds column l32 and rows 8*(v/4) + 4*h + v%4
  const int64_t r0 = row * BS + wm * 64 + 4 * h;
  const int64_t c0 = n0 + wn * 32 + l32;
  if (c0 < ncols) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t r = r0 + 8 * (v >> 2) + (v & 3);
      if (r < m) C[r * ldc + c0] = cvt_out<OutT>(acc0[v]);
      if (r + 32 < m) C[(r + 32) * ldc + c0] = cvt_out<OutT>(acc1[v]);
    }
  }
}

// ------------------------------------------------------ small block sizes
//
// bsr_spmm_small<BSZ>: b = 8, 16, 32 or 64. A block row of C is only b rows, so
// a wavefront owns one (block row, 64-column) tile of C and walks the row's
// stored blocks with its operands loaded directly into registers (4 waves
// per workgroup take consecutive column tiles of one block row and share
// its A blocks through L1):
//   b = 32, 64: v_mfma_f32_32x32x2_f32, b/32 row subtiles x 2 column
//     subtiles; at step 4g + c lane half h supplies k = 8g + 4h + c, so the
//     lane's A values for four MFMAs are one 16-byte read of its block row
//     (8 bytes for bf16); its column in subtile u is n0 + 2 (lane % 32) + u,
//     so its B values of both subtiles are one 8-byte read of row
//     8g + 4h + c;
//   b = 8: v_mfma_f32_4x4x1_16b_f32 (16 products of 4x4 per instruction
//     as 2 row groups x 8 column groups, 4 instructions per k for the 128
//     columns), 8 k-steps per block; B rows as 16-byte reads split between
//     the lane halves by v_permlane32_swap;
//   b = 16: v_mfma_f32_16x16x4_f32, 4 column subtiles; lane group q = lane/16
//     supplies k = 4q + c at step c, one 16-byte A read per block; the
//     lane's column in subtile u is n0 + 4 (lane % 16) + u, one 16-byte B
//     read per step.
// The output column of a lane is its B column, so the column permutation
// needs no shuffle; full column tiles of whole blocks with aligned B use the
// vector reads, the others read element by element in the same layout.
// B rows at or past n read as zero, C rows past m and columns past ncols are
// not written.
template <typename T>
__device__ inline f32x4 load4_acc(const T* p);
template <>
__device__ inline f32x4 load4_acc<float>(const float* p) { return *(const f32x4*)p; }
template <>
__device__ inline f32x4 load4_acc<uint16_t>(const uint16_t* p) {
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  const u16x4 v = *(const u16x4*)p;
  return f32x4{tsp::bf16_bits_to_f32(v[0]), tsp::bf16_bits_to_f32(v[1]), tsp::bf16_bits_to_f32(v[2]),
               tsp::bf16_bits_to_f32(v[3])};
}

template <typename T>
__device__ inline f32x2 load2_acc(const T* p);
template <>
__device__ inline f32x2 load2_acc<float>(const float* p) { return *(const f32x2*)p; }
template <>
__device__ inline f32x2 load2_acc<uint16_t>(const uint16_t* p) {
  const uint32_t v = *(const uint32_t*)p;
  return f32x2{tsp::bf16_bits_to_f32((uint16_t)(v & 0xffffu)), tsp::bf16_bits_to_f32((uint16_t)(v >> 16))};
}
// 2 consecutive outputs of one row as one store (8 bytes fp32, 4 bytes bf16)
__device__ inline void store2_out(float* p, float a, float b) { *(f32x2*)p = f32x2{a, b}; }
__device__ inline void store2_out(uint16_t* p, float a, float b) {
  *(uint32_t*)p = (uint32_t)tsp::f32_to_bf16_bits(a) | ((uint32_t)tsp::f32_to_bf16_bits(b) << 16);
}
// 4 consecutive outputs of one row as one store (16 bytes fp32, 8 bytes bf16)
__device__ inline void store4_out(float* p, f32x4 v) { *(f32x4*)p = v; }
__device__ inline void store4_out(uint16_t* p, f32x4 v) {
  typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
  *(u16x4*)p = u16x4{tsp::f32_to_bf16_bits(v[0]), tsp::f32_to_bf16_bits(v[1]), tsp::f32_to_bf16_bits(v[2]),
                     tsp::f32_to_bf16_bits(v[3])};
}

// TA = true: the product A^T X of the backward (dB = A^T dC). rp, ci and bid
// are then the block-column view (col_ptrs; per entry the block row, which
// selects the rows of X, and the stored block's id), an item's "row" is a
// block column, and each A block enters transposed at the load (element
// (r, k) of the operand is A_block[k][r]).
template <int BSZ, typename T, typename OutT, bool TA = false>
__global__ __launch_bounds__(256) void bsr_spmm_small(const T* __restrict__ blocks, const int64_t* __restrict__ rp,
                                                      const int64_t* __restrict__ ci, int64_t mb, int64_t m, int64_t n,
                                                      const T* __restrict__ B, int64_t ldb, int64_t ncols,
                                                      OutT* __restrict__ C, int64_t ldc, int64_t nct, int vec,
                                                      const int64_t* __restrict__ bid = nullptr) {
  static_assert(BSZ == 8 || BSZ == 16 || BSZ == 32 || BSZ == 64, "block size");
  constexpr int TW = BSZ == 8 ? 128 : 64;  // columns of C per wavefront
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // XCD x (= blockIdx % 8) takes the x-th eighth of the workgroups in row
  // order, so neighbouring block rows (which share the B panels of a band)
  // run on one L2; the grid is 8 * per workgroups
  const int64_t per = gridDim.x >> 3;
  const int64_t wg = (int64_t)(blockIdx.x & 7) * per + (blockIdx.x >> 3);
  const int64_t item = wg * 4 + w;  // (block row, column tile)
  const int64_t row = item / nct;
  if (row >= mb) return;
  const int64_t n0 = (item - row * nct) * TW;
  const int64_t start = rp[row], end = rp[row + 1];
  auto bval = [&](int64_t k, int64_t c) {
    return k < n && c < ncols ? tsp::to_acc<T>(B[k * ldb + c]) : 0.f;
  };
  // the stored block of entry idx, and element (r, k) of its A operand (TA: transposed)
  auto block_of = [&](int64_t idx) { return blocks + (TA ? bid[idx] : idx) * (BSZ * BSZ); };
  auto aop = [&](const T* blk, int r, int k) { return tsp::to_acc<T>(TA ? blk[k * BSZ + r] : blk[r * BSZ + k]); };
  if constexpr (BSZ == 8) {
    // v_mfma_f32_4x4x1_16b_f32: 16 independent 4x4 outer products (k = 1)
    // per instruction; lane l feeds product l/4 = (row group l/32, column
    // group (l/4) % 8): A row ra = 4 (l/32) + l%4 and one B column, and
    // holds its C rows 4 (l/32) + i (register i) of that column. The
    // wavefront's 128 columns are 4 groups u of 32: lane l's column in group
    // u is n0 + 4 (l%32) + u, so one 16-byte load per lane reads a B row's
    // 4 columns of the lane in all groups. The two lane halves load two
    // consecutive k rows (row 2p + l/32); v_permlane32_swap of a loaded
    // value with itself gives every lane both rows (r[0] from the low half,
    // r[1] from the high half). Per stored block: 4 B loads, 16 swaps, 32
    // MFMAs (k in order, so each sum runs in the generic kernel's order).
    // Tiles at the right edge, blocks past n, or unaligned B read element by
    // element in the same lane layout.
    const int m32 = lane & 31, hh = lane >> 5;
    const int ra = 4 * hh + (lane & 3);
    const int64_t nc = n0 + 4 * m32;  // the lane's column in group 0
    f32x4 acc[4] = {f32x4{}, f32x4{}, f32x4{}, f32x4{}};
    const int64_t nst = end - start;
    const bool cfull = (vec & 1) && n0 + 128 <= ncols;
    struct Ops {
      f32x4 a[2];
      f32x4 b[4];  // b[p]: row kb + 2p + l/32, the lane's column in each group
    };
    auto load = [&](int64_t st_, Ops& o) {
      const int64_t idx = start + (st_ < nst ? st_ : nst - 1);
      const int64_t kb = ci[idx] * BSZ;
      const T* blk = block_of(idx);
      if constexpr (TA) {
#pragma unroll
        for (int k = 0; k < 8; ++k) o.a[k >> 2][k & 3] = aop(blk, ra, k);
      } else {
        o.a[0] = load4_acc<T>(blk + ra * BSZ);
        o.a[1] = load4_acc<T>(blk + ra * BSZ + 4);
      }
      if (cfull && kb + BSZ <= n) {
#pragma unroll
        for (int q = 0; q < 4; ++q) o.b[q] = load4_acc<T>(B + (kb + 2 * q + hh) * ldb + nc);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int u = 0; u < 4; ++u) o.b[q][u] = bval(kb + 2 * q + hh, nc + u);
      }
    };
    auto mma = [&](const Ops& o) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(o.b[q][u]), __float_as_uint(o.b[q][u]),
                                                          false, false);
          acc[u] = __builtin_amdgcn_mfma_f32_4x4x1f32(o.a[q >> 1][2 * (q & 1)], __uint_as_float(r[0]), acc[u], 0, 0, 0);
          acc[u] = __builtin_amdgcn_mfma_f32_4x4x1f32(o.a[q >> 1][2 * (q & 1) + 1], __uint_as_float(r[1]), acc[u], 0, 0, 0);
        }
    };
    if (nst > 0) {
      Ops o0, o1;
      load(0, o0);
      int64_t st_ = 0;
      for (; st_ + 1 < nst; st_ += 2) {
        load(st_ + 1, o1);
        mma(o0);
        load(st_ + 2, o0);
        mma(o1);
      }
      if (st_ < nst) mma(o0);
    }
    const bool vstore = cfull && (vec & 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t rr = row * BSZ + 4 * hh + i;
      if (rr >= m) continue;
      OutT* cr = C + rr * ldc + nc;
      if (vstore) {
        store4_out(cr, f32x4{acc[0][i], acc[1][i], acc[2][i], acc[3][i]});
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (nc + u < ncols) cr[u] = tsp::from_acc<OutT>(acc[u][i]);
      }
    }
  } else if constexpr (BSZ == 16) {
    // lane group q = lane / 16 supplies k = 4q + c at step c; lane l16's
    // column in subtile u is n0 + 4 l16 + u, so one 16-byte load per step
    // reads its B row's columns of all 4 subtiles
    const int l16 = lane & 15, q = lane >> 4;
    const int64_t nc = n0 + 4 * l16;
    const bool cfull = (vec & 1) && n0 + 64 <= ncols;
    f32x4 acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = f32x4{};
    // one step per stored block; the next block's operands load while this one's MFMAs run
    // (the last block is loaded again past the end, so the loop has no conditional loads)
    const int64_t nst = end - start;
    auto load = [&](int64_t st_, f32x4& a, f32x4 (&bq)[4]) {
      const int64_t idx = start + (st_ < nst ? st_ : nst - 1);
      const int64_t k0 = ci[idx] * BSZ;
      const int64_t kb = k0 + 4 * q;
      const T* blk = block_of(idx);
      if constexpr (TA) {
#pragma unroll
        for (int c = 0; c < 4; ++c) a[c] = aop(blk, l16, 4 * q + c);
      } else {
        a = load4_acc<T>(blk + l16 * BSZ + 4 * q);
      }
      if (cfull && k0 + BSZ <= n) {
#pragma unroll
        for (int c = 0; c < 4; ++c) bq[c] = load4_acc<T>(B + (kb + c) * ldb + nc);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int u = 0; u < 4; ++u) bq[c][u] = bval(kb + c, nc + u);
      }
    };
    auto mma = [&](const f32x4& a, const f32x4 (&bq)[4]) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c], bq[c][u], acc[u], 0, 0, 0);
    };
    if (nst > 0) {
      f32x4 a0, a1;
      f32x4 b0[4], b1[4];
      load(0, a0, b0);
      int64_t st_ = 0;
      for (; st_ + 1 < nst; st_ += 2) {
        load(st_ + 1, a1, b1);
        mma(a0, b0);
        load(st_ + 2, a0, b0);
        mma(a1, b1);
      }
      if (st_ < nst) mma(a0, b0);
    }
    // element r of subtile u: row 4q + r, column n0 + 4 l16 + u
    const bool vstore = cfull && (vec & 2);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t rr = row * BSZ + 4 * q + r;
      if (rr >= m) continue;
      OutT* cr = C + rr * ldc + nc;
      if (vstore) {
        store4_out(cr, f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]});
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (nc + u < ncols) cr[u] = tsp::from_acc<OutT>(acc[u][r]);
      }
    }
  } else {
    // lane half h supplies k = 8g + 4h + c at step (g, c); lane l32's column
    // in subtile u is n0 + 2 l32 + u, so one 8-byte load per step reads its
    // B row's columns of both subtiles
    constexpr int RT = BSZ / 32;
    const int h = lane >> 5, l32 = lane & 31;
    const int64_t nc = n0 + 2 * l32;
    const bool cfull = (vec & 4) && n0 + 64 <= ncols;
    f32x16 acc[RT][2];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t][0] = acc[t][1] = f32x16{};
    for (int64_t idx = start; idx < end; ++idx) {
      const int64_t kb = ci[idx] * BSZ;
      const bool bfull = cfull && kb + BSZ <= n;
      const T* Ab = block_of(idx);
#pragma unroll
      for (int g = 0; g < BSZ / 8; ++g) {
        f32x4 a[RT];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          if constexpr (TA) {
#pragma unroll
            for (int c = 0; c < 4; ++c) a[t][c] = aop(Ab, 32 * t + l32, 8 * g + 4 * h + c);
          } else {
            a[t] = load4_acc<T>(Ab + (32 * t + l32) * BSZ + 8 * g + 4 * h);
          }
        }
        f32x2 bv[4];
        if (bfull) {
#pragma unroll
          for (int c = 0; c < 4; ++c) bv[c] = load2_acc<T>(B + (kb + 8 * g + 4 * h + c) * ldb + nc);
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int u = 0; u < 2; ++u) bv[c][u] = bval(kb + 8 * g + 4 * h + c, nc + u);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int u = 0; u < 2; ++u)
              acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t][c], bv[c][u], acc[t][u], 0, 0, 0);
      }
    }
    // element v of subtile (t, u): row 32t + 8(v/4) + 4h + v%4, column n0 + 2 l32 + u
    const bool vstore = cfull && (vec & 8);
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t rr = row * BSZ + 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
        if (rr >= m) continue;
        OutT* cr = C + rr * ldc + nc;
        if (vstore) {
          store2_out(cr, acc[t][0][v], acc[t][1][v]);
        } else {
#pragma unroll
          for (int u = 0; u < 2; ++u)
            if (nc + u < ncols) cr[u] = tsp::from_acc<OutT>(acc[t][u][v]);
        }
      }
  }
}

template <typename T, typename OutT, bool TA = false>
int launch_small(int64_t bs, const void* blocks, const int64_t* rp, const int64_t* ci, int64_t mb, int64_t m, int64_t n,
                 const void* B, int64_t ldb, int64_t ncols, void* C, int64_t ldc, hipStream_t st,
                 const int64_t* bid = nullptr) {
  const int64_t nct = tsp::ceil_div(ncols, bs == 8 ? 128 : 64);
  const int64_t grid = tsp::ceil_div(tsp::ceil_div(mb * nct, 4), 8) * 8;
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm: problem too large");
  // bits 0 / 1: B rows read / C rows written 4 columns at a time (b = 8, 16);
  // bits 2 / 3: 2 columns at a time (b = 32, 64)
  const int vec = (((uintptr_t)B % (4 * sizeof(T))) == 0 && ldb % 4 == 0 ? 1 : 0) |
                  (((uintptr_t)C % (4 * sizeof(OutT))) == 0 && ldc % 4 == 0 ? 2 : 0) |
                  (((uintptr_t)B % (2 * sizeof(T))) == 0 && ldb % 2 == 0 ? 4 : 0) |
                  (((uintptr_t)C % (2 * sizeof(OutT))) == 0 && ldc % 2 == 0 ? 8 : 0);
#define TSP_SMALL(BSZ)                                                                                     \
  hipLaunchKernelGGL((bsr_spmm_small<BSZ, T, OutT, TA>), dim3((unsigned)grid), dim3(256), 0, st, (const T*)blocks, \
                     rp, ci, mb, m, n, (const T*)B, ldb, ncols, (OutT*)C, ldc, nct, vec, bid)
  if (bs == 8)
    TSP_SMALL(8);
  else if (bs == 16)
    TSP_SMALL(16);
  else if (bs == 32)
    TSP_SMALL(32);
  else
    TSP_SMALL(64);
#undef TSP_SMALL
  return tsp::check_launch("bsr_spmm_small launch");
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

// dB = A^T X for block sizes 8, 16, 32 and 64 (the backward of bsr_spmm):
// bsr_spmm_small over the block-column view with A transposed at the load.
// X has m rows; dB has n rows. f32 in and out, or bf16 in and out.
int tsp::launch_bsr_small_t(int dtype, int64_t bs, const void* blocks, const int64_t* col_ptrs,
                            const int64_t* col_block_rows, const int64_t* col_block_ids, int64_t n_block_cols, int64_t m,
                            int64_t n, const void* X, int64_t ldx, int64_t ncols, void* out, int64_t ldo, hipStream_t st) {
  if (dtype == TSP_F32)
    return launch_small<float, float, true>(bs, blocks, col_ptrs, col_block_rows, n_block_cols, n, m, X, ldx, ncols,
                                            out, ldo, st, col_block_ids);
  return launch_small<uint16_t, uint16_t, true>(bs, blocks, col_ptrs, col_block_rows, n_block_cols, n, m, X, ldx, ncols,
                                                out, ldo, st, col_block_ids);
}

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
      ((uintptr_t)blocks % 16) == 0 && (n + BS) * ldb * 4 + 4 * BS <= (int64_t)UINT32_MAX) {
    // (the kernel's B offsets, rows < n + 128 and columns < ldb + 128, fit 32 bits)
    const int64_t nt = tsp::ceil_div(ncols, 128);
    const int64_t grid = tsp::ceil_div(mb, 8) * 8 * nt;
    if (grid > INT32_MAX || nt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm: problem too large");
    hipLaunchKernelGGL(bsr_spmm_f32_dma<F32_DMA_KC>, dim3((unsigned)grid), dim3(256), 0, st, (const float*)blocks, block_row_ptrs,
                       block_col_indices, mb, (int)nt, m, n, (const float*)B, ldb, ncols, (float*)C, ldc, row_order);
    return tsp::check_launch("bsr_spmm_f32_dma launch");
  }
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
      ((uintptr_t)blocks % 16) == 0 && (n + BS) * ldb * 2 + 2 * BS <= (int64_t)UINT32_MAX) {
    // (the kernel's B offsets, rows < n + 128 and columns < ldb + 128, fit 32 bits)
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
  if (dtype == TSP_F64 && block_size == BS && (ldb % 2) == 0 && ((uintptr_t)B % 16) == 0 &&
      ((uintptr_t)blocks % 16) == 0 && (n + BS) * ldb * 8 + 8 * BS <= (int64_t)UINT32_MAX) {
    // (the kernel's B offsets, rows < n + 128 and columns < ldb + 128, fit 32 bits)
    const int64_t nt = tsp::ceil_div(ncols, 128);
    const int64_t grid = tsp::ceil_div(mb, 8) * 8 * nt;
    if (grid > INT32_MAX || nt > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsr_spmm: problem too large");
    hipLaunchKernelGGL(bsr_spmm_f64_dma, dim3((unsigned)grid), dim3(256), 0, st, (const double*)blocks, block_row_ptrs,
                       block_col_indices, mb, (int)nt, m, n, (const double*)B, ldb, ncols, (double*)C, ldc, row_order);
    return tsp::check_launch("bsr_spmm_f64_dma launch");
  }
  if ((block_size == 8 || block_size == 16 || block_size == 32 || block_size == 64) && ((uintptr_t)blocks % 16) == 0) {
    if (dtype == TSP_F32)
      return launch_small<float, float>(block_size, blocks, block_row_ptrs, block_col_indices, mb, m, n, B, ldb, ncols,
                                        C, ldc, st);
    if (dtype == TSP_BF16 && out_dtype == TSP_F32)
      return launch_small<uint16_t, float>(block_size, blocks, block_row_ptrs, block_col_indices, mb, m, n, B, ldb,
                                           ncols, C, ldc, st);
    if (dtype == TSP_BF16)
      return launch_small<uint16_t, uint16_t>(block_size, blocks, block_row_ptrs, block_col_indices, mb, m, n, B, ldb,
                                              ncols, C, ldc, st);
  }
  if (dtype == TSP_F32) return launch_generic<float, float>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
  if (dtype == TSP_F64) return launch_generic<double, double>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
  if (out_dtype == TSP_F32) return launch_generic<uint16_t, float>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
  return launch_generic<uint16_t, uint16_t>(blocks, block_row_ptrs, block_col_indices, block_size, m, n, B, ldb, ncols, C, ldc, st);
}
