// fp32 operand tiles shared by the streamed MFMA products of the BSR
// backward (bsr_backward.hip) and the screened SpMM backward (screened.hip):
// 128-row tiles with 64-wide k-slabs, filled by direct global->LDS loads
// (lds_dma.h) into a 2-stage ring, read as v_mfma_f32_32x32x2_f32 operands.
//   row tile [128][64]: k = columns (16-byte chunk c of row r in slot c ^ (r % 16));
//   k tile   [64][128]: k = rows (chunk c of row rr in slot c ^ 8 ((rr / 4) % 2)).
// Include after common.h and lds_dma.h.
#pragma once

namespace tsp {
namespace f32pair {

using tsp::dma::i32x4;
constexpr int BS = 128;
constexpr int KC = 64;
constexpr int TROWB = KC * 4;            // row tile [128][64] fp32: 256-byte rows
constexpr int KROWB = BS * 4;            // k tile [64][128] fp32: 512-byte rows
constexpr int TILE = 128 * TROWB;        // 32 KiB (== KC * KROWB)
constexpr int STAGE = 2 * TILE;          // 64 KiB
constexpr int NST = 2;
constexpr uint32_t OOB = 0xFFFFFFF0u;    // a buffer offset past any range: reads zero

// ---- tile loads (each wave issues 8 of the 32 1-KiB instructions of a tile)
// Row tile: rows [row0, row0+128) x columns [k0, k0+64) of a row-major fp32
// matrix with row stride ld; 16-byte chunk c of row r sits in slot
// c ^ (r % 16). Columns at or past kend read as zero.
__device__ inline void dma_row_tile(i32x4 rs, int64_t row0, int64_t ld, int64_t k0, int64_t kend, uint32_t dst, int w,
                                    int lane) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = 8 * w + q;
    const int r = 4 * i + (lane >> 4);
    const int c = (lane & 15) ^ (r & 15);
    const int64_t col = k0 + c * 4;
    const uint32_t off = col < kend ? (uint32_t)(((row0 + r) * ld + col) * 4) : OOB;
    tsp::dma::buffer16(rs, off, dst + i * 1024);
  }
}
// k tile: rows [krow0, krow0+64) x columns [n0, n0+128) of a row-major fp32
// matrix with row stride ld; chunk c of row rr sits in slot c ^ 8*((rr/4)%2).
__device__ inline void dma_k_tile(i32x4 rs, int64_t krow0, int64_t ld, int64_t n0, uint32_t dst, int w, int lane) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int j = 8 * w + q;
    const int rr = 2 * j + (lane >> 5);
    const int c = (lane & 31) ^ (8 * ((rr >> 2) & 1));
    tsp::dma::buffer16(rs, (uint32_t)(((krow0 + rr) * ld + n0 + c * 4) * 4), dst + j * 1024);
  }
}
// The same k tile from memory that is always in bounds.
__device__ inline void dma_k_tile_global(const float* src, int64_t ld, uint32_t dst, int w, int lane) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int j = 8 * w + q;
    const int rr = 2 * j + (lane >> 5);
    const int c = (lane & 31) ^ (8 * ((rr >> 2) & 1));
    tsp::dma::global16(src + rr * ld + c * 4, dst + j * 1024);
  }
}

// ---- operand fragments for v_mfma_f32_32x32x2_f32 over one 8-k group g:
// lane half h takes k = 8g + 4h + s at k-step s (s = 0..3).
// From a row tile: row r -> the 4 values are one 16-byte read.
__device__ inline f32x4 frag_row(const uint8_t* tile, int r, int g, int h) {
  return *(const f32x4*)(tile + r * TROWB + (((2 * g + h) ^ (r & 15)) * 16));
}
// From a k tile: the column pair c2, c2 + 1 (c2 even) -> 4 values each from
// rows 8g + 4h + s, one 8-byte read per row; v[i] feeds the subtile whose
// columns are the ones of parity i.
__device__ inline void frag_k2(const uint8_t* tile, int c2, int g, int h, float (&v)[2][4]) {
  const uint8_t* p = tile + (8 * g + 4 * h) * KROWB + ((((c2 >> 2) ^ (8 * h))) * 16) + (c2 & 3) * 4;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const f32x2 x = *(const f32x2*)(p + s * KROWB);
    v[0][s] = x[0];
    v[1][s] = x[1];
  }
}

struct Acc4 {
  f32x16 a[2][2];
  __device__ void zero() {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) a[t][u] = f32x16{};
  }
  __device__ void mma(const float (&x)[2][4], const float (&y)[2][4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) a[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(x[t][s], y[u][s], a[t][u], 0, 0, 0);
  }
};

}  // namespace f32pair
}  // namespace tsp
