// Block-sparse attention backward, fp32, head_dim 256, 128-blocks, for gfx950.
//
// The passes and semantics of the fp32 kernels in attention_bwd.hip (the
// reference tiled backward, trnsparse/ops.py:360-473; the reference device
// path K-tiles head_dim > 128 in 128-wide pieces, trnsparse/nki/kernels.py:
// 192-200): a row pass for dQ that also writes the query stats, and a column
// pass for dK / dV over the column plan, whose split columns are summed by
// bsa_bwd_reduce_f32<256> there. At head_dim 256 the 32-row tiles of those
// kernels do not fit a wavefront (the wave's Q and dO rows take 256
// registers, its dK and dV accumulators another 256), so here a wavefront
// owns 16 rows on v_mfma_f32_16x16x4_f32 and a workgroup covers half a
// 128-block (64 queries, or 64 keys):
//   * products over head_dim (S, dP): at step 4t + c lane group g = lane / 16
//     supplies d = 16t + 4g + c, so one b128 LDS read of a stage row feeds
//     four MFMAs (chunk read) against the wave's own rows held as register
//     fragments X[row][16t + 4g .. +3] (64 registers per operand);
//   * products over rows (dQ, dK, dV): row i of output subtile u = 4b + c is
//     d = 64b + 4i + c, so a lane's A operands for subtiles 4b .. 4b + 3 are
//     one b128 read X[row][64b + 4 l16 .. +3] (row piece); the k index is
//     the row, in the accumulator order of the S / dP tiles (k = g at step r
//     is row 4g + r of a 16-row tile), so their elements are the B operand
//     in place;
//   * stage rows (32 per stage, 1 KiB each: K and V in the row pass, Q and
//     dO plus their stats in the column pass) stream through a 2-stage LDS
//     ring (130 KiB, one workgroup per CU) by direct buffer loads issued one
//     stage ahead, stored 16-byte chunk ^ (row % 16), so chunk reads (one
//     chunk of 16 rows) and row pieces (16 chunks of one row) hit distinct
//     banks. Rows at or past seq_len read as zero.
// This file is built without the VGPR MFMA form: the 64 (dQ) or 128 (dK,
// dV) accumulator registers per lane live in AGPRs.
#include "common.h"
#include "lds_dma.h"

namespace {

constexpr float LOG2E = 1.4426950408889634f;
constexpr int D = 256, BS = 128;
constexpr int HR = 32;               // rows per ring stage
constexpr int ROWB = D * 4;          // bytes per row
constexpr int HBYTES = HR * ROWB;    // 32 KiB of one operand per stage
constexpr int NST = 2;
constexpr int SPB = BS / HR;         // stages per block
constexpr int NI = HBYTES / 4096;    // 1 KiB loads per wave per operand and stage
constexpr int KT = D / 16;           // chunk reads per 16-row tile
constexpr int NT = HR / 16;          // 16-row tiles per stage
constexpr int NU = D / 16;           // output subtiles

__device__ inline f32x4 mfma16(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// This wave's share of a stage: rows [row0, row0 + HR) of the buffer rs into
// LDS dst, one 1 KiB row per instruction, chunk p of row j at slot p ^ (j % 16).
__device__ inline void dma_rows(tsp::dma::i32x4 rs, int64_t row0, uint32_t dst, int w, int lane) {
#pragma unroll
  for (int qq = 0; qq < NI; ++qq) {
    const int j = NI * w + qq;
    tsp::dma::buffer16(rs, (uint32_t)((row0 + j) * ROWB + ((lane ^ (j & 15)) << 4)), dst + j * 1024);
  }
}
// Logical 16-byte chunk c of stage row `row`.
__device__ inline f32x4 chunk(const uint8_t* base, int row, int c) {
  return *(const f32x4*)(base + row * ROWB + ((c ^ (row & 15)) << 4));
}
// Row piece j of a stage: step i = j / 4 (rows 16 (i / 4) + 4g + i % 4 of
// the stage), column group b = j % 4, floats 64b + 4 l16 .. +3.
__device__ inline f32x4 piece(const uint8_t* base, int j, int g, int l16) {
  const int i = j >> 2, b = j & 3;
  return chunk(base, 16 * (i >> 2) + 4 * g + (i & 3), 16 * b + l16);
}
// Store the lane's row of a 16-row x 256 tile held as NU accumulators
// (element r of subtile 4b + c is d = 64b + 16g + 4r + c), times f.
__device__ inline void store_row(float* dst, const f32x4* acc, int g, float f) {
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f32x4 t;
#pragma unroll
      for (int c = 0; c < 4; ++c) t[c] = acc[4 * b + c][r] * f;
      *(f32x4*)(dst + 64 * b + 16 * g + 4 * r) = t;
    }
}

// Row pass: workgroup per (head, query block row m < Mt, half), XCD-aware
// order (XCD x walks heads x, x + 8, ...); wavefront w owns queries
// m * 128 + 64 half + 16 w + [0, 16) with their Q and dO rows in registers.
// Per 16-key tile: S^T = K Q^T and dP^T = V dO^T, dS^T = P^T (dP^T - D) in
// place, dQ^T += K^T dS^T. Writes the column pass's query stats: plane 0
// r = log2e * row_max + log2 row_denom (P = exp2(log2e * scale * s - r)),
// plane 1 D.
__global__ __launch_bounds__(256, 1) void bsa_bwd_dq_f32_d256(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V, const float* __restrict__ O,
    const float* __restrict__ dO, int64_t S, int64_t H, const int64_t* __restrict__ rp,
    const int64_t* __restrict__ ci, int64_t Mt, float scale_log2, float scale, const float* __restrict__ rmax,
    const float* __restrict__ rden, float* __restrict__ qstat, float* __restrict__ dQ) {
  constexpr int STAGE = 2 * HBYTES;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];

  const int64_t gid = blockIdx.x;
  const int64_t xcd = gid & 7, slot = gid >> 3;
  const int64_t head = xcd + 8 * (slot / (2 * Mt));
  const int64_t rem = slot % (2 * Mt);
  const int64_t m = rem >> 1, half = rem & 1;
  if (head >= H) return;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int64_t hs = head * S * D;
  const int64_t q = m * BS + 64 * half + 16 * w + l16;  // < S since m < Mt

  f32x4 qf[KT], dof[KT];
  float dsum = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    qf[t] = *(const f32x4*)(Q + hs + q * D + 16 * t + 4 * g);
    dof[t] = *(const f32x4*)(dO + hs + q * D + 16 * t + 4 * g);
    const f32x4 of = *(const f32x4*)(O + hs + q * D + 16 * t + 4 * g);
#pragma unroll
    for (int c = 0; c < 4; ++c) dsum += dof[t][c] * of[c];
  }
  dsum += __shfl_xor(dsum, 16, 64);
  const float Dq = dsum + __shfl_xor(dsum, 32, 64);
  const float rq = rmax[head * Mt * BS + q] * LOG2E + __builtin_amdgcn_logf(rden[head * Mt * BS + q]);
  if (g == 0) {
    qstat[head * S + q] = rq;
    qstat[H * S + head * S + q] = Dq;
  }

  f32x4 acc[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) acc[u] = f32x4{};

  const int64_t start = rp[m];
  const int nblk = (int)(rp[m + 1] - start);
  const int nsteps = SPB * nblk;
  const tsp::dma::i32x4 krs = tsp::dma::make_rsrc(K + hs, (uint32_t)(S * ROWB));
  const tsp::dma::i32x4 vrs = tsp::dma::make_rsrc(V + hs, (uint32_t)(S * ROWB));
  const uint32_t lds0 = tsp::dma::lds_addr(lds);

  // key-block indices of the row, 64 at a time in one VGPR, read with readlane
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
    dma_rows(krs, key0, st, w, lane);
    dma_rows(vrs, key0, st + HBYTES, w, lane);
  };

  // one 16-key tile at a time: S^T / dP^T, dS^T in place, then dQ^T += K^T dS^T
  auto compute = [&](const uint8_t* st, int64_t key0) {
    const uint8_t* Ks = st;
    const uint8_t* Vs = st + HBYTES;
    const bool tail = key0 + HR > S;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      // S^T / dP^T element r: key key0 + 16 tt + 4g + r, query q
      f32x4 sc, dp;
      f32x4 ka[2], va[2];
      ka[0] = chunk(Ks, 16 * tt + l16, g);
      va[0] = chunk(Vs, 16 * tt + l16, g);
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        if (t + 1 < KT) {
          ka[(t + 1) & 1] = chunk(Ks, 16 * tt + l16, 4 * (t + 1) + g);
          va[(t + 1) & 1] = chunk(Vs, 16 * tt + l16, 4 * (t + 1) + g);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const bool first = t == 0 && c == 0;
          sc = mfma16(ka[t & 1][c], qf[t][c], first ? f32x4{} : sc);
          dp = mfma16(va[t & 1][c], dof[t][c], first ? f32x4{} : dp);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], scale_log2, -rq));
        if (tail && key0 + 16 * tt + 4 * g + r >= S) p = 0.f;
        sc[r] = p * (dp[r] - Dq);
      }
      // piece j feeds subtiles 4 (j % 4) .. +3 at step j / 4
      f32x4 kb[2];
      kb[0] = piece(Ks, 16 * tt, g, l16);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (j + 1 < 16) kb[(j + 1) & 1] = piece(Ks, 16 * tt + j + 1, g, l16);
        __builtin_amdgcn_sched_barrier(0);
        const int r = j >> 2, b = j & 3;
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[4 * b + c] = mfma16(kb[j & 1][c], sc[r], acc[4 * b + c]);
      }
    }
  };

  if (nsteps > 0) issue(0);
  for (int s = 0; s < nsteps; ++s) {
    const int64_t key0 = first_key(s);
    tsp::dma::wait_vm<0>();  // this wave's loads of stage s are done
    tsp::dma::barrier();     // every wave's part is in LDS; stage (s+1) % NST is free
    if (s + 1 < nsteps) issue(s + 1);
    compute(lds + (s % NST) * STAGE, key0);
  }
  store_row(dQ + hs + q * D, acc, g, scale);
}

// Column pass: workgroup per (plan item, head, half), items heaviest first;
// an item is (key block column, range [p0, p1) of its column view, partial
// slot or -1). Wavefront w owns keys col * 128 + 64 half + 16 w + [0, 16)
// with their K and V rows in registers. Per 16-query tile of a stored block
// row m < Mt: S = Q K^T and dP = dO V^T, P and dS = P (dP - D) in place with
// the query stats staged beside the rows, dV^T += dO^T P and dK^T += Q^T dS.
// An item covering a whole column writes dK / dV, a segment of a split
// column writes fp32 partials (rows 0..127 of the block) for the reduce.
__global__ __launch_bounds__(256, 1) void bsa_bwd_dkdv_f32_d256(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, int64_t S, int64_t H, const int64_t* __restrict__ crow,
    const int32_t* __restrict__ items, int n_partials, int64_t Mt, float scale_log2, float scale,
    const float* __restrict__ qstat, float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ partial) {
  constexpr int STAGE = 2 * HBYTES + 1024;  // Q rows, dO rows, stats (r[HR], D[HR], then repeats)
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];

  const int64_t it = blockIdx.x / (2 * H), rem = blockIdx.x % (2 * H);
  const int64_t head = rem >> 1, half = rem & 1;
  const int col = items[4 * it], p0 = items[4 * it + 1], p1 = items[4 * it + 2], pslot = items[4 * it + 3];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int64_t hs = head * S * D, HS = H * S;
  const int krow = 64 * (int)half + 16 * w + l16;  // the lane's key within the block
  const int64_t key = (int64_t)col * BS + krow;
  const bool kvalid = key < S;

  f32x4 kf[KT], vf[KT];
  const int64_t kload = kvalid ? key : 0;  // rows past seq_len: zero fragments
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const f32x4 kv = *(const f32x4*)(K + hs + kload * D + 16 * t + 4 * g);
    const f32x4 vv = *(const f32x4*)(V + hs + kload * D + 16 * t + 4 * g);
    kf[t] = kvalid ? kv : f32x4{};
    vf[t] = kvalid ? vv : f32x4{};
  }
  f32x4 dk[NU], dv[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) dk[u] = dv[u] = f32x4{};

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
  // stage s: block row rowblk(s / SPB), queries from m * 128 + HR * (s % SPB).
  // A block row >= Mt has no forward queries: its stage is filled with zeros
  // (zero Q and dO rows and stats add nothing to dK and dV), so every stage
  // runs the same code and no branch around the products makes the compiler
  // carry the accumulators through VGPRs.
  auto issue = [&](int s, int64_t mrow) {
    if (mrow >= Mt) {
      uint8_t* z = lds + (s % NST) * STAGE;
#pragma unroll
      for (int qq = 0; qq < NI; ++qq) {
        const int j = NI * w + qq;
        *(f32x4*)(z + j * 1024 + 16 * lane) = f32x4{};
        *(f32x4*)(z + HBYTES + j * 1024 + 16 * lane) = f32x4{};
      }
      if (w == 0) *(f32x4*)(z + 2 * HBYTES + 16 * lane) = f32x4{};
      return;
    }
    const int64_t q0 = mrow * BS + HR * (s % SPB);
    const uint32_t st = lds0 + (s % NST) * STAGE;
    dma_rows(qrs, q0, st, w, lane);
    dma_rows(ors, q0, st + HBYTES, w, lane);
    if (w == 0) {  // lanes [0, HR/4): r, the rest D (the lanes past 2 HR / 4 repeat D)
      constexpr int LPP = HR / 4;
      const int plane = lane >= LPP ? 1 : 0;
      tsp::dma::global16(qstat + plane * HS + head * S + q0 + 4 * (lane % LPP), st + 2 * HBYTES);
    }
  };

  // one 16-query tile at a time: S / dP, then P / dS in place, then the row
  // products (few live registers beside the K and V fragments)
  auto compute = [&](const uint8_t* st) {
    const uint8_t* Qs = st;
    const uint8_t* Os = st + HBYTES;
    const float* stats = (const float*)(st + 2 * HBYTES);
#pragma unroll
    for (int qt = 0; qt < NT; ++qt) {
      // S / dP element r: query 16 qt + 4g + r of the stage, the lane's key
      f32x4 sc, dp;
      f32x4 qa[2], oa[2];
      qa[0] = chunk(Qs, 16 * qt + l16, g);
      oa[0] = chunk(Os, 16 * qt + l16, g);
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        if (t + 1 < KT) {
          qa[(t + 1) & 1] = chunk(Qs, 16 * qt + l16, 4 * (t + 1) + g);
          oa[(t + 1) & 1] = chunk(Os, 16 * qt + l16, 4 * (t + 1) + g);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const bool first = t == 0 && c == 0;
          sc = mfma16(qa[t & 1][c], kf[t][c], first ? f32x4{} : sc);
          dp = mfma16(oa[t & 1][c], vf[t][c], first ? f32x4{} : dp);
        }
      }
      const f32x4 r4 = *(const f32x4*)(stats + 16 * qt + 4 * g);
      const f32x4 d4 = *(const f32x4*)(stats + HR + 16 * qt + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], scale_log2, -r4[r]));
        sc[r] = p;
        dp[r] = p * (dp[r] - d4[r]);
      }
      // dV^T += dO^T P, dK^T += Q^T dS: piece j feeds subtiles 4 (j % 4) .. +3 at step j / 4
      f32x4 ob[2], qb[2];
      ob[0] = piece(Os, 16 * qt, g, l16);
      qb[0] = piece(Qs, 16 * qt, g, l16);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (j + 1 < 16) {
          ob[(j + 1) & 1] = piece(Os, 16 * qt + j + 1, g, l16);
          qb[(j + 1) & 1] = piece(Qs, 16 * qt + j + 1, g, l16);
        }
        __builtin_amdgcn_sched_barrier(0);
        const int r = j >> 2, b = j & 3;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          dv[4 * b + c] = mfma16(ob[j & 1][c], sc[r], dv[4 * b + c]);
          dk[4 * b + c] = mfma16(qb[j & 1][c], dp[r], dk[4 * b + c]);
        }
      }
    }
  };

  if (nsteps > 0) issue(0, rowblk(0));
  for (int s = 0; s < nsteps; ++s) {
    tsp::dma::wait_vm<0>();  // this wave's loads of stage s are done
    tsp::dma::barrier();     // every wave's part (or zero fill) is in LDS; stage (s+1) % NST is free
    if (s + 1 < nsteps) issue(s + 1, rowblk((s + 1) / SPB));
    compute(lds + (s % NST) * STAGE);
  }

  if (pslot < 0) {
    if (kvalid) {
      store_row(dK + hs + key * D, dk, g, scale);
      store_row(dV + hs + key * D, dv, g, 1.f);
    }
  } else {
    float* pk = partial + (((int64_t)head * n_partials + pslot) * 2) * (BS * D) + krow * D;
    store_row(pk, dk, g, scale);
    store_row(pk + BS * D, dv, g, 1.f);
  }
}

}  // namespace

namespace tsp {

// Row pass of the fp32 head_dim-256 backward (grid: 8 * ceil(H / 8) * Mt * 2).
int bsa_bwd_f32_d256_rows(const float* Q, const float* K, const float* V, const float* O, const float* dO, int64_t S,
                        int64_t H, const int64_t* rp, const int64_t* ci, int64_t Mt, float scale_log2, float scale,
                        const float* rmax, const float* rden, float* qstat, float* dQ, hipStream_t st) {
  const int64_t grid = tsp::ceil_div(H, 8) * Mt * 2 * 8;
  if (grid == 0) return TSP_OK;
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_bwd: problem too large");
  hipLaunchKernelGGL(bsa_bwd_dq_f32_d256, dim3((unsigned)grid), dim3(256), 0, st, Q, K, V, O, dO, S, H, rp, ci, Mt,
                     scale_log2, scale, rmax, rden, qstat, dQ);
  return tsp::check_launch("bsa_bwd_dq_f32_d256 launch");
}

// Column pass of the fp32 head_dim-256 backward (grid: n_items * H * 2).
int bsa_bwd_f32_d256_cols(const float* Q, const float* K, const float* V, const float* dO, int64_t S, int64_t H,
                          const int64_t* crow, const int32_t* items, int64_t n_items, int n_partials, int64_t Mt,
                          float scale_log2, float scale, const float* qstat, float* dK, float* dV, float* partial,
                          hipStream_t st) {
  const int64_t grid = n_items * H * 2;
  if (grid == 0) return TSP_OK;
  if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_bwd: problem too large");
  hipLaunchKernelGGL(bsa_bwd_dkdv_f32_d256, dim3((unsigned)grid), dim3(256), 0, st, Q, K, V, dO, S, H, crow, items,
                     n_partials, Mt, scale_log2, scale, qstat, dK, dV, partial);
  return tsp::check_launch("bsa_bwd_dkdv_f32_d256 launch");
}

}  // namespace tsp
