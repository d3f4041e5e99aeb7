// fp64 MFMA operand tiles shared by the fp64 BSR SpMM, its backward and the
// fp64 screened SpMM (v_mfma_f64_16x16x4_f64: A[i = lane % 16][k = lane / 16],
// B[k = lane / 16][j = lane % 16]; accumulator element v of lane l is row
// l / 16 + 4 v, column l % 16).
//
// A workgroup of 4 waves owns a 128x128 fp64 tile of the output as 2 x 2 wave
// tiles of 64x64 (4 x 4 accumulators each) and streams 32-wide k-slabs of two
// operand tiles, 32 KiB each, through an LDS ring by direct global->LDS
// loads (8 wave instructions per tile per wave). Within a slab the k index
// is permuted so that lane group g takes k = 8g + 2p + s at k-step (p, s).
// An operand tile has one of two forms:
//   ROW: [128 rows][32 k], rows of 256 B: a lane's k pair is one b128 read;
//        16-byte chunk ^ (row % 16), so 16 rows of one chunk cover the banks;
//   COL: [32 k][128 columns], rows of 1 KiB: one b64 read per k-step;
//        chunk ^ 8 ((k / 8) % 2), so the four k groups' rows split the banks.
#pragma once

#include "lds_dma.h"

namespace tsp {
namespace f64tile {

constexpr int BS = 128;
constexpr int KC = 32;
constexpr int TILE = 32768;                // bytes of one operand tile
constexpr uint32_t OOB = 0xFFFFFFF0u;      // a buffer offset past any range: reads zero
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));

// ROW tile: rows [row0, row0 + 128) x columns [k0, k0 + 32) of a row-major
// fp64 matrix (stride ld) behind rs; columns at or past kend read as zero
// (kend even).
__device__ inline void dma_row(dma::i32x4 rs, int64_t row0, int64_t ld, int64_t k0, int64_t kend, uint32_t dst, int w,
                               int lane) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = 8 * w + q;
    const int r = 4 * i + (lane >> 4);
    const int c = (lane & 15) ^ (r & 15);
    const int64_t col = k0 + 2 * c;
    const uint32_t off = col < kend ? (uint32_t)(((row0 + r) * ld + col) * 8) : OOB;
    dma::buffer16(rs, off, dst + i * 1024);
  }
}
// The same ROW tile from a 128x128 block (k columns [0, 32) of src, row
// stride BS; always in bounds).
__device__ inline void dma_row_block(const double* src, uint32_t dst, int w, int lane) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = 8 * w + q;
    const int r = 4 * i + (lane >> 4);
    const int c = (lane & 15) ^ (r & 15);
    dma::global16(src + r * BS + 2 * c, dst + i * 1024);
  }
}
// COL tile: rows [row0, row0 + 32) x columns [c0, c0 + 128) behind rs.
__device__ inline void dma_col(dma::i32x4 rs, int64_t row0, int64_t ld, int64_t c0, uint32_t dst, int w, int lane) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int j = 8 * w + q;
    const int c = lane ^ (8 * ((j >> 3) & 1));
    dma::buffer16(rs, (uint32_t)(((row0 + j) * ld + c0 + 2 * c) * 8), dst + j * 1024);
  }
}
// The same COL tile from a 128-column block (always in bounds).
__device__ inline void dma_col_block(const double* src, uint32_t dst, int w, int lane) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int j = 8 * w + q;
    const int c = lane ^ (8 * ((j >> 3) & 1));
    dma::global16(src + j * BS + 2 * c, dst + j * 1024);
  }
}

// Operand values of k-steps (p, 0) and (p, 1) for tile rows / columns
// base + 16 t + lane % 16, t = 0..3: v[t][s].
template <bool ROWF>
__device__ inline void fetch(const uint8_t* tile, int base, int p, int lane, double (&v)[4][2]) {
  const int g = lane >> 4, l16 = lane & 15;
  if (ROWF) {
    const uint8_t* a = tile + (base + l16) * 256 + (((4 * g + p) ^ l16) * 16);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f64x2 x = *(const f64x2*)(a + 16 * t * 256);
      v[t][0] = x[0];
      v[t][1] = x[1];
    }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int col = base + 16 * t + l16;
      const int off = (((col >> 1) ^ (8 * (g & 1))) * 16) + (col & 1) * 8;
#pragma unroll
      for (int s = 0; s < 2; ++s) v[t][s] = *(const double*)(tile + (8 * g + 2 * p + s) * 1024 + off);
    }
  }
}

// The 32 MFMAs of k-steps (p, 0), (p, 1) of a 64x64 wave tile.
__device__ inline void mma(const double (&a)[4][2], const double (&b)[4][2], f64x4 (&acc)[4][4]) {
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[t][u] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[t][k], b[u][k], acc[t][u], 0, 0, 0);
}

}  // namespace f64tile
}  // namespace tsp
