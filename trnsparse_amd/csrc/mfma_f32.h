// fp32 MFMA tile core shared by the BSR SpMM and screened SpMM kernels.
//
// One 512-thread workgroup (8 wavefronts, 4(M) x 2(N)) accumulates a 128x128
// fp32 tile of C over a sequence of KC-wide k-slabs (KC = 32 or 64). The
// caller supplies the slab source: `src.load(s, a, b)` fetches slab s from
// global memory into registers — NA float4 of A (rows q.ar + i*q.astep, four
// k values at column q.ac) and NB float4 of B (rows q.br + 16*i, four n
// values at column q.bc). Slabs pass through a double-buffered LDS ring fed
// from registers: slab s+1 is written to LDS halfway through slab s's
// v_mfma_f32_32x32x2_f32 work and the loads of slab s+2 are issued right
// after, so LDS writes overlap MFMAs and every load has a slab of time to
// land; within a slab the LDS operands of the next 8-k group are read while
// the current group's MFMAs run. One barrier per slab. With KC = 64 the ring
// takes 137 KiB of LDS, so one workgroup owns a CU and the hardware
// dispatcher schedules the grid in order (longest-first lists stay
// longest-first).
#pragma once

#include "common.h"

namespace tsp {
namespace f32tile {

constexpr int BM = 128;          // tile rows
constexpr int BN = 128;          // tile columns
constexpr int NTHR = 512;        // 8 wavefronts
constexpr int B_LD = BN + 4;     // LDS row stride (floats) of the B slab [k][n]

// Geometry of a KC-wide k-slab.
template <int KC>
struct Slab {
  static constexpr int A_LD = KC + 4;       // LDS row stride (floats) of the A slab [m][k]
  static constexpr int A_SLAB = BM * A_LD;
  static constexpr int B_SLAB = KC * B_LD;
  static constexpr int STAGE = A_SLAB + B_SLAB;
  static constexpr int LDS_FLOATS = 2 * STAGE;
  static constexpr int NA = KC / 16;        // float4 of A per thread per slab
  static constexpr int NB = KC / 16;        // float4 of B per thread per slab
};

template <int KC>
struct Coords {
  int ar, ac, astep;  // A staging: rows ar + i*astep, k columns ac..ac+3
  int br, bc;         // B staging: rows br + 16*i, n columns bc..bc+3
  int wm, wn, h, l32;
  __device__ Coords() {
    const int tid = threadIdx.x;
    ar = tid / (KC / 4);
    ac = (tid % (KC / 4)) * 4;
    astep = NTHR / (KC / 4);
    br = tid >> 5;
    bc = (tid & 31) * 4;
    const int lane = tid & 63, w = tid >> 6;
    wm = w & 3;
    wn = w >> 2;
    h = lane >> 5;
    l32 = lane & 31;
  }
};

// Accumulate `nsteps` slabs into acc0 (columns wn*64 + l32) and acc1 (+32).
template <int KC, class Src>
__device__ inline void run(Src& src, int nsteps, float* lds, const Coords<KC>& q, f32x16& acc0, f32x16& acc1) {
  typedef Slab<KC> G;
  f32x4 ra[G::NA], rb[G::NB];
  auto lstore = [&](float* st) {
    float* As = st;
    float* Bs = st + G::A_SLAB;
#pragma unroll
    for (int i = 0; i < G::NA; ++i) *(f32x4*)(As + (q.ar + i * q.astep) * G::A_LD + q.ac) = ra[i];
#pragma unroll
    for (int i = 0; i < G::NB; ++i) *(f32x4*)(Bs + (q.br + 16 * i) * B_LD + q.bc) = rb[i];
  };
  // MFMA k-step s of a group of 8 k values uses k = k0 + s (lanes 0-31) and
  // k = k0 + 4 + s (lanes 32-63): a lane's 4 A values are one 16-byte LDS
  // load. A and B follow the same k order, so the sum is unchanged. The
  // operands of group g+1 are read from LDS while group g's 8 MFMAs run
  // (register double buffering), so LDS latency stays off the MFMA pipe.
  struct Ops {
    f32x4 a;
    float b0[4], b1[4];
  };
  auto fetch = [&](const float* st, int k0, Ops& o) {
    const float* As = st;
    const float* Bs = st + G::A_SLAB;
    o.a = *(const f32x4*)(As + (q.wm * 32 + q.l32) * G::A_LD + k0 + 4 * q.h);
    const float* bp = Bs + (k0 + 4 * q.h) * B_LD + q.wn * 64 + q.l32;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      o.b0[s] = bp[s * B_LD];
      o.b1[s] = bp[s * B_LD + 32];
    }
  };
  auto mma = [&](const Ops& o) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(o.a[s], o.b0[s], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(o.a[s], o.b1[s], acc1, 0, 0, 0);
    }
  };
  // Groups [g0, g1) of one slab; operands of the next group are read while
  // the current group's MFMAs run.
  auto compute = [&](const float* st, int g0, int g1) {
    Ops o[2];
    fetch(st, 8 * g0, o[0]);
#pragma unroll
    for (int g = g0; g < g1; ++g) {
      if (g + 1 < g1) fetch(st, 8 * (g + 1), o[(g + 1 - g0) & 1]);
      // keep the scheduler from sinking the reads next to their MFMAs
      __builtin_amdgcn_sched_barrier(0);
      mma(o[(g - g0) & 1]);
    }
  };
  // Pipeline: slab s+1 sits in registers (its global loads were issued half
  // a slab into s-1) and is written to the other LDS buffer halfway through
  // slab s's MFMAs, right before the loads of slab s+2 are issued. The LDS
  // writes thus overlap MFMA work and each load has a full slab of time to
  // arrive; one barrier per slab.
  if (nsteps <= 0) return;
  constexpr int NG = KC / 8;
  src.load(0, ra, rb);
  lstore(lds);
  if (nsteps > 1) src.load(1, ra, rb);
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const float* cur = lds + (s & 1) * G::STAGE;
    float* nxt = lds + ((s + 1) & 1) * G::STAGE;
    compute(cur, 0, NG / 2);
    if (s + 1 < nsteps) {
      lstore(nxt);
      if (s + 2 < nsteps) src.load(s + 2, ra, rb);
    }
    compute(cur, NG / 2, NG);
    __syncthreads();
  }
}

// Four consecutive elements of row r from column c, zero outside
// [0, nrows) x [0, ncols). The vector path needs 16-byte alignment of the
// row start (ld % 4 == 0, 16-byte base) and c % 4 == 0.
__device__ inline f32x4 load4_guard(const float* __restrict__ p0, int64_t r, int64_t c, int64_t nrows,
                                    int64_t ncols, int64_t ld) {
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  if (r < nrows) {
    const float* p = p0 + r * ld + c;
    if (c + 3 < ncols) {
      v = *(const f32x4*)p;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c + i < ncols) v[i] = p[i];
    }
  }
  return v;
}

// Store the tile (accumulator layout: lane holds column l32 and rows
// 8*(v/4) + 4*h + v%4, v = 0..15) to C rows [row0, row0+128) clipped to m,
// columns [col0, col0+128) clipped to ncols.
template <typename OutT, typename Cvt, int KC>
__device__ inline void store_tile(OutT* __restrict__ C, int64_t ldc, int64_t row0, int64_t col0, int64_t m,
                                  int64_t ncols, const Coords<KC>& q, const f32x16& acc0, const f32x16& acc1,
                                  Cvt cvt) {
  const int64_t rbase = row0 + q.wm * 32 + 4 * q.h;
  const int64_t c0 = col0 + q.wn * 64 + q.l32;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t r = rbase + 8 * (v >> 2) + (v & 3);
    if (r < m) {
      OutT* crow = C + r * ldc;
      if (c0 < ncols) crow[c0] = cvt(acc0[v]);
      if (c0 + 32 < ncols) crow[c0 + 32] = cvt(acc1[v]);
    }
  }
}

// Work item of a tiled launch over `mb` row tiles (ranked heaviest first by
// `order`, or in natural order when it is null) and `nt` column tiles.
// Consecutive workgroup ids go round-robin over the 8 XCDs: ranks are dealt
// to XCDs in boustrophedon order (0..7, 15..8, 16..23, ...) so every XCD
// gets an equal share of heavy and light rows, and the column tiles of one
// row sit in consecutive slots of one XCD (they share its L2 for the A row
// panel). Returns false for padding slots.
__device__ inline bool tile_item(int64_t g, int64_t mb, int64_t nt, const int32_t* __restrict__ order,
                                 int64_t& row, int& ntile) {
  const int64_t xcd = g & 7, slot = g >> 3;
  const int64_t rl = slot / nt;
  ntile = (int)(slot - rl * nt);
  const int64_t k = (rl & 1) ? 8 * rl + 7 - xcd : 8 * rl + xcd;
  if (k >= mb) return false;
  row = order ? (int64_t)order[k] : k;
  return true;
}

}  // namespace f32tile
}  // namespace tsp
