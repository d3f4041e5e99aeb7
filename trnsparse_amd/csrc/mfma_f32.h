// fp32 MFMA tile core shared by the BSR SpMM and screened SpMM kernels.
//
// One 512-thread workgroup (8 wavefronts, 4(M) x 2(N)) accumulates a 128x128
// fp32 tile of C over a sequence of 32-wide k-slabs. The caller supplies the
// slab source: `src.load(s, a0, a1, b0, b1)` fetches slab s from global
// memory into registers (A rows ar and ar+64, four k values at column ac; B
// rows br and br+16, four n values at column bc — see the staging coordinates
// below). Slabs pass through a double-buffered LDS ring: the loads of slab
// s+1 are in flight while slab s feeds v_mfma_f32_32x32x2_f32; one barrier
// per slab.
#pragma once

#include "common.h"

namespace tsp {
namespace f32tile {

constexpr int BM = 128;          // tile rows
constexpr int BN = 128;          // tile columns
constexpr int KC = 32;           // k-slab
constexpr int NTHR = 512;        // 8 wavefronts
constexpr int A_LD = KC + 4;     // LDS row stride (floats) of the A slab [m][k]
constexpr int B_LD = BN + 4;     // LDS row stride (floats) of the B slab [k][n]
constexpr int A_SLAB = BM * A_LD;
constexpr int B_SLAB = KC * B_LD;
constexpr int STAGE = A_SLAB + B_SLAB;
constexpr int LDS_FLOATS = 2 * STAGE;

struct Coords {
  int ar, ac;  // A staging: rows ar, ar+64; k columns ac..ac+3
  int br, bc;  // B staging: rows br, br+16; n columns bc..bc+3
  int wm, wn, h, l32;
  __device__ Coords() {
    const int tid = threadIdx.x;
    ar = tid >> 3;
    ac = (tid & 7) * 4;
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
template <class Src>
__device__ inline void run(Src& src, int nsteps, float* lds, const Coords& q, f32x16& acc0, f32x16& acc1) {
  f32x4 ra0, ra1, rb0, rb1;
  auto lstore = [&](float* st) {
    float* As = st;
    float* Bs = st + A_SLAB;
    *(f32x4*)(As + q.ar * A_LD + q.ac) = ra0;
    *(f32x4*)(As + (q.ar + 64) * A_LD + q.ac) = ra1;
    *(f32x4*)(Bs + q.br * B_LD + q.bc) = rb0;
    *(f32x4*)(Bs + (q.br + 16) * B_LD + q.bc) = rb1;
  };
  // MFMA k-step s of a group of 8 k values uses k = k0 + s (lanes 0-31) and
  // k = k0 + 4 + s (lanes 32-63): a lane's 4 A values are one 16-byte LDS
  // load. A and B follow the same k order, so the sum is unchanged.
  auto compute = [&](const float* st) {
    const float* As = st;
    const float* Bs = st + A_SLAB;
#pragma unroll
    for (int k0 = 0; k0 < KC; k0 += 8) {
      const f32x4 a = *(const f32x4*)(As + (q.wm * 32 + q.l32) * A_LD + k0 + 4 * q.h);
      const float* bp = Bs + (k0 + 4 * q.h) * B_LD + q.wn * 64 + q.l32;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float b0 = bp[s * B_LD];
        const float b1 = bp[s * B_LD + 32];
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b1, acc1, 0, 0, 0);
      }
    }
  };
  if (nsteps <= 0) return;
  src.load(0, ra0, ra1, rb0, rb1);
  lstore(lds);
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const float* cur = lds + (s & 1) * STAGE;
    float* nxt = lds + ((s + 1) & 1) * STAGE;
    const bool more = s + 1 < nsteps;
    if (more) src.load(s + 1, ra0, ra1, rb0, rb1);
    compute(cur);
    if (more) lstore(nxt);
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
template <typename OutT, typename Cvt>
__device__ inline void store_tile(OutT* __restrict__ C, int64_t ldc, int64_t row0, int64_t col0, int64_t m,
                                  int64_t ncols, const Coords& q, const f32x16& acc0, const f32x16& acc1, Cvt cvt) {
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

}  // namespace f32tile
}  // namespace tsp
