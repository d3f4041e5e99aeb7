// Block-sparse attention forward for gfx950.
//
// Semantics follow the reference spec `_block_sparse_attn_pytorch`
// (trnsparse/ops.py:280-357), per head:
//   score(q, k) = (Q[q] . K[k]) * scale for keys k of the stored mask blocks
//                 of q's block row (all b columns of a stored block)
//   row_max     = max score, row_denom = max(sum exp(score - row_max), 1e-12)
//   O[q]        = sum exp(score - row_max) / row_denom * V[k]
// Empty block rows give O = 0, row_max = 0, row_denom = 1e-12 (:320-337).
// Keys at or beyond seq_len do not exist (the reference's K slice is short).
// The reference's two passes plus host reduction (and the NKI path's
// device->host->device round trip, trnsparse/nki/dispatch.py:580-677)
// become one pass with an online softmax; the stats are returned for the
// autograd context.
//
// Kernels
//   bsa_fwd_bf16_mfma<D>  bf16, 128-blocks, D in {64, 128}: one 256-thread
//       workgroup per (head, 128-query block row); each wavefront owns 32
//       queries. Scores are formed transposed, S^T = K Q^T, with
//       v_mfma_f32_32x32x16_bf16 (A = K rows from LDS, B = the wave's Q rows
//       held in registers), so a lane holds all scores of one query: the
//       softmax needs one cross-lane shuffle. O^T = V^T P^T consumes P from
//       registers (bf16) with V staged transposed in LDS. fp32 softmax with
//       exp2, fp32 accumulation, bf16 output. Kept for operands past 4 GiB.
//   bsa_fwd_bf16_stream<D> the same work split with K/V streamed through an
//       LDS ring by direct loads (D in {64, 128, 256}).
//   bsa_fwd_bf16_d512     bf16, D = 512: the streamed kernel's math with the
//       head dimension split between the two wavefronts of a pair, which
//       add their partial scores through LDS.
//   bsa_fwd_f32_mfma<D>   fp32, 128-blocks, D in {64, 128, 256}: the same
//       work split on v_mfma_f32_32x32x2_f32 with K/V streamed through an
//       LDS ring.
// head_dim 256 keeps the whole score product in one workgroup (16 k-steps
// of 16 bf16 / 128 of 2 fp32 per 32-key tile), bf16 512 as well (split
// over wavefront pairs); other head_dims are padded with zero columns by
// the caller.
//   bsa_fwd_generic<T>    fp32/fp64/bf16, any block size and head_dim: one
//       thread per (query, 32-wide slice of head_dim), online softmax in
//       the accumulation type (double for fp64).
#include "common.h"
#include "lds_dma.h"

namespace {

constexpr float LOG2E = 1.4426950408889634f;

// ------------------------------------------------------------------ generic

template <typename T> struct AttnAcc { typedef float type; };
template <> struct AttnAcc<double> { typedef double type; };

template <typename T> __device__ inline typename AttnAcc<T>::type ld_acc(const T* p) { return (typename AttnAcc<T>::type)*p; }
template <> __device__ inline float ld_acc<uint16_t>(const uint16_t* p) { return tsp::bf16_bits_to_f32(*p); }
template <typename T> __device__ inline T st_cvt(typename AttnAcc<T>::type v) { return (T)v; }
template <> __device__ inline uint16_t st_cvt<uint16_t>(float v) { return tsp::f32_to_bf16_bits(v); }

__device__ inline float acc_exp(float v) { return __expf(v); }
__device__ inline double acc_exp(double v) { return exp(v); }

constexpr int GEN_DC = 32;  // head_dim slice per thread

template <typename T>
__global__ __launch_bounds__(128) void bsa_fwd_generic(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V, int64_t S, int64_t D,
    int64_t head_stride, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci, int64_t b, int64_t Mt,
    typename AttnAcc<T>::type scale, T* __restrict__ O, typename AttnAcc<T>::type* __restrict__ rmax,
    typename AttnAcc<T>::type* __restrict__ rden) {
  typedef typename AttnAcc<T>::type AccT;
  // blockIdx.x: query chunk of 128 rows; blockIdx.y: head_dim slice; blockIdx.z: head
  const int64_t head = blockIdx.z;
  const int64_t q = (int64_t)blockIdx.x * 128 + threadIdx.x;
  if (q >= Mt * b) return;
  const int64_t d0 = (int64_t)blockIdx.y * GEN_DC;
  const int64_t m = q / b;
  const T* Qh = Q + head * head_stride;
  const T* Kh = K + head * head_stride;
  const T* Vh = V + head * head_stride;
  AccT acc[GEN_DC];
#pragma unroll
  for (int i = 0; i < GEN_DC; ++i) acc[i] = 0;
  AccT mrun = -INFINITY, lrun = 0;
  const int64_t e = rp[m + 1];
  for (int64_t idx = rp[m]; idx < e; ++idx) {
    const int64_t k0 = ci[idx] * b;
    for (int64_t k = k0; k < k0 + b && k < S; ++k) {
      AccT s = 0;
      for (int64_t d = 0; d < D; ++d) s += ld_acc(Qh + q * D + d) * ld_acc(Kh + k * D + d);
      s *= scale;
      const AccT mnew = s > mrun ? s : mrun;
      const AccT alpha = acc_exp(mrun - mnew);
      const AccT p = acc_exp(s - mnew);
      lrun = lrun * alpha + p;
#pragma unroll
      for (int i = 0; i < GEN_DC; ++i) {
        const AccT v = d0 + i < D ? ld_acc(Vh + k * D + d0 + i) : (AccT)0;
        acc[i] = acc[i] * alpha + p * v;
      }
      mrun = mnew;
    }
  }
  const bool empty = rp[m] == e;
  const AccT den = lrun > (AccT)1e-12 ? lrun : (AccT)1e-12;
  T* Oq = O + head * head_stride + q * D;
#pragma unroll
  for (int i = 0; i < GEN_DC; ++i)
    if (d0 + i < D) Oq[d0 + i] = st_cvt<T>(empty ? (AccT)0 : acc[i] / den);
  if (blockIdx.y == 0 && rmax) {
    rmax[head * Mt * b + q] = empty ? (AccT)0 : mrun;
    rden[head * Mt * b + q] = empty ? (AccT)1e-12 : den;
  }
}

// ------------------------------------------------------------- bf16 MFMA

constexpr int AB = 128;  // block size served by the MFMA kernel

template <int D>
__global__ __launch_bounds__(256, 2) void bsa_fwd_bf16_mfma(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, int64_t S,
    int64_t head_stride, int64_t H, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci, int64_t Mt,
    float scale_log2, uint16_t* __restrict__ O, float* __restrict__ rmax, float* __restrict__ rden) {
  constexpr int KS = D / 16;      // k-steps of S^T = K Q^T
  constexpr int K_LD = D + 8;     // LDS row stride (bf16) of K [key][d]
  constexpr int V_LD = AB + 4;    // LDS row stride (bf16) of V^T [d][key]
  constexpr int NU = D / 32;      // 32-wide d subtiles of O^T
  __shared__ __attribute__((aligned(16))) uint16_t Ks[AB * K_LD];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[D * V_LD];

  // XCD-aware order: XCD x walks heads x, x+8, ...; the block rows of one
  // head run side by side and share that head's K/V in the XCD's L2.
  const int64_t g = blockIdx.x;
  const int64_t xcd = g & 7, slot = g >> 3;
  const int64_t head = xcd + 8 * (slot / Mt);
  const int64_t m = slot % Mt;
  if (head >= H) return;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const uint16_t* Qh = Q + head * head_stride;
  const uint16_t* Kh = K + head * head_stride;
  const uint16_t* Vh = V + head * head_stride;
  const int64_t q = m * AB + w * 32 + l32;  // this lane's query (always < S: m < Mt)

  // Q fragments for the B operand: Q[q][16s + 8h .. +7]
  bf16x8 qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qf[s] = *(const bf16x8*)(Qh + q * D + 16 * s + 8 * h);

  f32x16 o[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) o[u] = f32x16{};
  float mrun = -INFINITY, lrun = 0.f;

  const int64_t e = rp[m + 1];
  for (int64_t idx = rp[m]; idx < e; ++idx) {
    const int64_t key0 = ci[idx] * AB;
    __syncthreads();  // previous block's LDS reads are done
    // ---- stage K block [key][d] and V block transposed [d][key] (4 keys x 8 d
    // patches); rows past seq_len are zero. `full` (uniform) drops the guards.
    const int nvalid = (int)((S - key0) < AB ? (S - key0) : AB);
    const bool full = nvalid == AB;
    u16x8 kreg[(AB * D / 8) / 256];
#pragma unroll
    for (int i = 0; i < (AB * D / 8) / 256; ++i) {
      const int c = tid + 256 * i;
      const int key = c / (D / 8), col = (c % (D / 8)) * 8;
      if (full || key < nvalid)
        kreg[i] = *(const u16x8*)(Kh + (key0 + key) * D + col);
      else
        kreg[i] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < (AB * D / 8) / 256; ++i) {
      const int c = tid + 256 * i;
      const int key = c / (D / 8), col = (c % (D / 8)) * 8;
      *(u16x8*)(Ks + key * K_LD + col) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < (AB / 4) * (D / 8) / 256; ++i) {
      const int p = tid + 256 * i;
      const int kg = p % (AB / 4), dg = p / (AB / 4);
      u16x8 r[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = 4 * kg + j;
        if (full || key < nvalid)
          r[j] = *(const u16x8*)(Vh + (key0 + key) * D + 8 * dg);
        else
          r[j] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) {
        typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
        u16x4 t = {r[0][dd], r[1][dd], r[2][dd], r[3][dd]};
        *(u16x4*)(Vt + (8 * dg + dd) * V_LD + 4 * kg) = t;
      }
    }
    __syncthreads();

    // The block's 128 keys are taken as two halves of 64 (register budget):
    // each half forms its S^T tiles, updates the online softmax and adds its
    // P V contribution.
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      // ---- S^T tiles: keys 32t + 8*(v/4) + 4h + v%4 (t = 2*half + tt), query l32
      f32x16 st[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int t = 2 * half + tt;
        st[tt] = f32x16{};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const bf16x8 a = *(const bf16x8*)(Ks + (32 * t + l32) * K_LD + 16 * s + 8 * h);
          st[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[s], st[tt], 0, 0, 0);
        }
      }
      // ---- online softmax (log2 domain), keys past seq_len excluded
      float mx = mrun;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = 32 * (2 * half + tt) + 8 * (v >> 2) + 4 * h + (v & 3);
          const float val = (full || key < nvalid) ? st[tt][v] * scale_log2 : -INFINITY;
          st[tt][v] = val;
          mx = fmaxf(mx, val);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float alpha = mx == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(mrun - mx);
      float lsum = 0.f;
      bf16x8 pb[2][2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float p = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st[tt][v] - mx);
          lsum += p;
          pb[tt][v >> 3][v & 7] = (__bf16)p;
        }
      }
      lsum += __shfl_xor(lsum, 32, 64);
      lrun = lrun * alpha + lsum;
      mrun = mx;
#pragma unroll
      for (int u = 0; u < NU; ++u) o[u] *= alpha;
      // ---- O^T += V^T P^T; k-step (t, a) covers keys 32t+16a+[0,16): lane
      // half h supplies keys 4h+{0..3} and 8+4h+{0..3} (its own S^T rows).
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const uint16_t* vrow = Vt + (32 * u + l32) * V_LD;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int t = 2 * half + tt;
#pragma unroll
          for (int a = 0; a < 2; ++a) {
            typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
            const u16x4 lo = *(const u16x4*)(vrow + 32 * t + 16 * a + 4 * h);
            const u16x4 hi = *(const u16x4*)(vrow + 32 * t + 16 * a + 8 + 4 * h);
            const u16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av), pb[tt][a], o[u], 0, 0, 0);
          }
        }
      }
    }
  }

  // ---- epilogue: O[q][32u + 8*(v/4) + 4h + v%4] = o / denom
  const bool empty = rp[m] == e;
  const float den = lrun > 1e-12f ? lrun : 1e-12f;
  const float inv = empty ? 0.f : 1.f / den;
  uint16_t* Oq = O + head * head_stride + q * D;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
      u16x4 t;
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = tsp::f32_to_bf16_bits(o[u][4 * g4 + i] * inv);
      *(u16x4*)(Oq + 32 * u + 8 * g4 + 4 * h) = t;
    }
  }
  if (h == 0 && rmax) {
    const int64_t r = head * Mt * AB + q;
    rmax[r] = empty ? 0.f : mrun * 0.69314718055994531f;
    rden[r] = empty ? 1e-12f : den;
  }
}

// ------------------------------------------- bf16 MFMA, d = 64, 128 and 256
//
// bsa_fwd_bf16_stream<D>: same work split and math as bsa_fwd_bf16_mfma (one
// 256-thread workgroup per (head, 128-query block row), a wavefront per 32
// queries, S^T = K Q^T with the wave's Q rows in registers, online softmax in
// the exp2 domain, O^T += V^T P^T with P from registers), restructured so the
// key blocks stream while the MFMAs run:
//   * keys are consumed in stages of HK keys (64 at D <= 128, 32 at D = 256)
//     that go through a 2-stage LDS ring (K part + V part per stage: 64 KiB
//     per workgroup at D = 128 and 256, 32 KiB at D = 64), filled by direct
//     global->LDS buffer loads issued one stage ahead; rows at or past
//     seq_len read as zero;
//   * V stays [key][d] in LDS and the A operand of O^T += V^T P^T (8 keys of
//     one d column per lane) comes from ds_read_b64_tr_b16;
//   * 16-byte chunks are XOR-swizzled for conflict-free reads on the 64-bank
//     LDS (att::Geo: K rows for b128 reads of 16 consecutive keys, V rows for
//     transpose reads of 4 consecutive keys);
//   * each MFMA's LDS operand is read one step ahead.
namespace att {
constexpr int NST = 2;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
// Row geometry and swizzles per head_dim: K rows are read as 16-byte pieces
// of 16 consecutive keys (one chunk), V rows through transpose reads of 4
// consecutive keys. D = 128 (256-byte rows, 16 chunks): K chunk ^ (key % 16),
// V chunk ^ 4 (key % 4); D = 256 (512-byte rows, 32 chunks, again starting
// at bank 0) uses the same terms on the low chunk bits. D = 64 (128-byte
// rows, where keys k and k + 2 share banks): K chunk ^ ((key / 2) % 8), V
// chunk ^ 4 ((key / 2) % 2).
template <int D>
struct Geo {
  static constexpr int HK = D > 128 ? 32 : 64; // keys per ring stage
  static constexpr int NT = HK / 32;           // 32-key S^T tiles per stage
  static constexpr int SPB = AB / HK;          // stages per key block
  static constexpr int ROWB = D * 2;           // bytes per K/V row
  static constexpr int HBYTES = HK * ROWB;     // bytes per K (or V) half
  static constexpr int STAGE = 2 * HBYTES;
  static constexpr int KS = D / 16;            // k-steps of S^T
  static constexpr int NU = D / 32;            // 32-wide d subtiles of O^T
  static constexpr int LPR = ROWB / 16;        // lanes per row in a 1 KiB load
  static constexpr int RPI = 64 / LPR;         // rows per load instruction
  __host__ __device__ static constexpr int kswz(int key) { return D >= 128 ? (key & 15) : ((key >> 1) & 7); }
  __host__ __device__ static constexpr int vswz(int key) { return D >= 128 ? (key & 3) : ((key >> 1) & 1); }
};
// max / sum of v over lanes l and l ^ 32 (the two halves of a 64-lane wave)
// with one v_permlane32_swap: with both operands v, the pair it returns holds
// v[l] and v[l ^ 32] in every lane
__device__ inline float halves_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float halves_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
}  // namespace att

// D = 64 fits three wavefronts per SIMD (136 registers, 32 KiB of LDS per
// workgroup). D = 256 takes 32-key stages so that two workgroups fit per CU
// (64 KiB of ring each): its 64 + 128 registers of Q and O per lane leave
// room for one 32-key score tile, and the loop body stays within the 256
// registers of two wavefronts per SIMD (a few values live across the loop
// are spilled outside it). Per stage that is 32 MFMAs, as at D = 128.
template <int D>
__global__ __launch_bounds__(256, D == 64 ? 3 : 2) void bsa_fwd_bf16_stream(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, int64_t S,
    int64_t head_stride, int64_t H, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci, int64_t Mt,
    float scale_log2, uint16_t* __restrict__ O, float* __restrict__ rmax, float* __restrict__ rden) {
  using namespace att;
  typedef Geo<D> G;
  constexpr int ROWB = G::ROWB, HBYTES = G::HBYTES, STAGE = G::STAGE, KS = G::KS, NU = G::NU;
  constexpr int HK = G::HK, NT = G::NT, SPB = G::SPB;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];

  // XCD-aware order: XCD x walks heads x, x+8, ...; the block rows of one
  // head run side by side and share that head's K/V in the XCD's L2.
  const int64_t g = blockIdx.x;
  const int64_t xcd = g & 7, slot = g >> 3;
  const int64_t head = xcd + 8 * (slot / Mt);
  const int64_t m = slot % Mt;
  if (head >= H) return;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int gq = lane >> 4, jq = lane & 15;
  const uint16_t* Qh = Q + head * head_stride;
  const uint16_t* Kh = K + head * head_stride;
  const uint16_t* Vh = V + head * head_stride;
  const int64_t q = m * AB + w * 32 + l32;  // this lane's query (always < S: m < Mt)

  // Q fragments for the B operand of S^T: Q[q][16s + 8h .. +7]
  bf16x8 qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qf[s] = *(const bf16x8*)(Qh + q * D + 16 * s + 8 * h);

  f32x16 o[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) o[u] = f32x16{};
  // mtrue: running max of the scaled scores (log2 domain); mref: the
  // reference P and the sums are taken against (see the rescale below)
  constexpr float RESCALE = 8.f;
  float mtrue = -INFINITY, mref = -INFINITY, lrun = 0.f;

  const int64_t start = rp[m];
  const int nblk = (int)(rp[m + 1] - start);
  const int nsteps = SPB * nblk;
  const tsp::dma::i32x4 krs = tsp::dma::make_rsrc(Kh, (uint32_t)(S * D * 2));
  const tsp::dma::i32x4 vrs = tsp::dma::make_rsrc(Vh, (uint32_t)(S * D * 2));
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
  auto first_key = [&](int s) { return (int64_t)colblk(s / SPB) * AB + HK * (s % SPB); };

  // ---- loads of stage s into ring slot s % NST: per wave HBYTES / 4 KiB K and V instructions
  auto issue = [&](int s) {
    const int64_t key0 = first_key(s);
    const uint32_t st = lds0 + (s % NST) * STAGE;
    constexpr int NI = HBYTES / 4096;
#pragma unroll
    for (int qq = 0; qq < NI; ++qq) {
      const int j = NI * w + qq;                // rows [RPI j, RPI j + RPI) of the stage
      const int rr = G::RPI * j + lane / G::LPR;
      const int p = lane % G::LPR;              // this lane's 16-byte slot in the row
      const int64_t rowoff = (key0 + rr) * ROWB;
      tsp::dma::buffer16(krs, (uint32_t)(rowoff + ((p ^ G::kswz(rr)) * 16)), st + j * 1024);
      tsp::dma::buffer16(vrs, (uint32_t)(rowoff + ((p ^ (4 * G::vswz(rr))) * 16)), st + HBYTES + j * 1024);
    }
  };

  // per-lane LDS offsets
  // O^T A operand via transpose reads: lane j of 16-lane group gq points at
  // key row kb + 8*r + 4*(gq>>1) + j/4 (r: which 4-key read), d column
  // 32u + 16*(gq&1) + 4*(j%4); the swizzle term is 4*vswz(row).
  const int vrow = 4 * (gq >> 1) + (jq >> 2);
  const int vsw = 4 * G::vswz(vrow);  // rows read are vrow + multiples of 8, same swizzle
  const int vcol = 16 * (gq & 1) + 4 * (jq & 3);  // plus 32u

  // K reads: logical chunk 2ks + h of row 32tt + l32 sits in slot
  // (2ks + h) ^ kswz(row), the same for both 32-key tiles
  const int kx = G::kswz(l32) ^ h;
  // V transpose reads: byte offset within a row for d subtile u is
  // ((4u + c0) ^ vsw) * 16 + (col & 4) * 2 = ((u ^ (vsw/4)) << 6) + c0 * 16 + ...
  const int vlane = vrow * ROWB + ((vcol >> 3) & 3) * 16 + (vcol & 4) * 2;

  auto compute = [&](const uint8_t* st, int64_t key0) {
    const uint8_t* Ks = st + l32 * ROWB;
    const uint8_t* Vs = st + HBYTES + vlane;
    auto kread = [&](int ks, int tile) {
      return *(const bf16x8*)(Ks + tile * 32 * ROWB + (((2 * ks) ^ kx) * 16));
    };
    // ---- S^T tiles (keys 32*tt + 8*(v/4) + 4h + v%4, query l32): two
    // independent accumulator chains, operands read one k-step ahead
    f32x16 sc[NT];
    bf16x8 ka[2][NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) ka[0][tt] = kread(0, tt);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) ka[(ks + 1) & 1][tt] = kread(ks + 1, tt);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
        sc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[ks & 1][tt], qf[ks], ks == 0 ? f32x16{} : sc[tt], 0, 0, 0);
    }
    // ---- online softmax in the log2 domain (scale_log2 > 0, so the max of
    // the raw scores scales to the max of the scaled ones); keys at or past
    // seq_len (only in a block that crosses it) are excluded
    if (key0 + HK > S) {
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (key0 + 32 * tt + 8 * (v >> 2) + 4 * h + (v & 3) >= S) sc[tt][v] = -INFINITY;
    }
    float mraw = sc[0][0];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int v = 0; v < 16; ++v) mraw = fmaxf(mraw, sc[tt][v]);
    mraw = att::halves_max(mraw);
    mtrue = fmaxf(mtrue, mraw * scale_log2);
    // Lazy rescaling: P is taken relative to a reference max mref that only
    // moves when the true running max exceeds it by more than RESCALE (log2
    // units), so P <= 2^RESCALE and o, l rarely need the multiply; o / l is
    // the same quantity for any reference.
    if (__builtin_amdgcn_ballot_w64(mtrue > mref + RESCALE) != 0) {
      const bool move = mtrue > mref + RESCALE;
      const float alpha = move ? (mref == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mref - mtrue)) : 1.f;
      mref = move ? mtrue : mref;
      lrun *= alpha;
#pragma unroll
      for (int u = 0; u < NU; ++u) o[u] *= alpha;
    }
    const float nmx = mref == -INFINITY ? 0.f : -mref;  // -inf scores give p = 0 either way
    float lsum = 0.f;
    bf16x8 pb[NT][2];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        typedef float f32x8 __attribute__((ext_vector_type(8)));
        f32x8 pv;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[tt][8 * a + i], scale_log2, nmx));
          lsum += p;
          pv[i] = p;
        }
        pb[tt][a] = __builtin_convertvector(pv, bf16x8);
      }
    }
    lrun += lsum;  // this lane half's part; the halves are combined at the end
    // ---- O^T += V^T P^T. k-step (tt, a) covers keys 32tt + 16a + [0,16):
    // MFMA k index i < 4 is key 32tt + 16a + 4h + i, i >= 4 is key
    // 32tt + 16a + 8 + 4h + (i-4) — the lane's own S^T rows, so pb[tt][a]
    // (values v = 8a .. 8a+7) is the matching B operand.
    const int vx = vsw >> 2;
    auto vread = [&](int tt, int a, int u) {
      att::s16x4 r[2];
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const uint8_t* p = Vs + (32 * tt + 16 * a + 8 * rr) * ROWB + ((u ^ vx) << 6);
        r[rr] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((att::lds_s16x4*)p);
      }
      return __builtin_bit_cast(bf16x8, __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7));
    };
    bf16x8 vb[2];
    vb[0] = vread(0, 0, 0);
#pragma unroll
    for (int step = 0; step < 2 * NT * NU; ++step) {
      const int tt = step / (2 * NU), a = (step / NU) % 2, u = step % NU;
      if (step + 1 < 2 * NT * NU) {
        const int s1 = step + 1;
        vb[s1 & 1] = vread(s1 / (2 * NU), (s1 / NU) % 2, s1 % NU);
      }
      __builtin_amdgcn_sched_barrier(0);
      o[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb[step & 1], pb[tt][a], o[u], 0, 0, 0);
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

  // ---- epilogue: O[q][32u + 8*(v/4) + 4h + v%4] = o / l (both relative to
  // mref); the returned denominator is relative to the true max
  lrun = att::halves_sum(lrun);
  const bool empty = nblk == 0;
  const float lref = lrun > 1e-12f ? lrun : 1e-12f;
  const float inv = empty ? 0.f : 1.f / lref;
  const float ltrue = mref == -INFINITY ? lrun : lrun * __builtin_amdgcn_exp2f(mref - mtrue);
  const float den = ltrue > 1e-12f ? ltrue : 1e-12f;
  uint16_t* Oq = O + head * head_stride + q * D;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
      u16x4 t;
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = tsp::f32_to_bf16_bits(o[u][4 * g4 + i] * inv);
      *(u16x4*)(Oq + 32 * u + 8 * g4 + 4 * h) = t;
    }
  }
  if (h == 0 && rmax) {
    const int64_t r = head * Mt * AB + q;
    rmax[r] = empty ? 0.f : mtrue * 0.69314718055994531f;
    rden[r] = empty ? 1e-12f : den;
  }
}

// ------------------------------------------------- bf16 MFMA, d = 512
//
// bsa_fwd_bf16_d512: head_dim 512 in one pass. At 32 queries per wavefront
// the d = 512 score tile and output rows need 16 + 256 accumulator registers
// next to 128 of Q (more than a lane's 512), so the head dimension is split
// between the two wavefronts of a pair: one 512-thread workgroup per
// (head, 128-query block row), wavefront w owns queries 32 (w % 4) + [0, 32)
// and head dims 256 (w / 4) + [0, 256) — its Q columns and its half of O —
// the register footprint of the d = 256 kernel. Per 32-key stage a
// wavefront forms the partial scores of its half (S^T over 16 k-steps),
// stores them to LDS, and after a barrier adds its partner's: both
// wavefronts of a pair then hold the same scores bit for bit (fp32
// addition is commutative), run the same online softmax and multiply P by
// their half of V. Keys stream through a 2-stage LDS ring (K and V, 64 KiB
// per stage) as in bsa_fwd_bf16_stream; with the 32 KiB exchange the
// workgroup takes the 160 KiB of a CU, two wavefronts per SIMD.
namespace a512 {
constexpr int D = 512, DH = 256, HK = 32, SPB = AB / HK, ROWB = D * 2;
constexpr int HBYTES = HK * ROWB, STAGE = 2 * HBYTES, NST = 2;
constexpr int KS = DH / 16;  // k-steps of a partial S^T
constexpr int NU = DH / 32;  // 32-wide d subtiles of a half of O^T
constexpr int XBYTES = 8 * 16 * 64 * 4;  // partial scores: 8 waves x 16 values x 64 lanes
__host__ __device__ constexpr int kswz(int key) { return key & 15; }
__host__ __device__ constexpr int vswz(int key) { return key & 3; }
}  // namespace a512

__global__ __launch_bounds__(512, 1) void bsa_fwd_bf16_d512(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, int64_t S,
    int64_t head_stride, int64_t H, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci, int64_t Mt,
    float scale_log2, uint16_t* __restrict__ O, float* __restrict__ rmax, float* __restrict__ rden) {
  using namespace a512;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE + XBYTES];
  float* xch = (float*)(lds + NST * STAGE);

  const int64_t g = blockIdx.x;
  const int64_t xcd = g & 7, slot = g >> 3;
  const int64_t head = xcd + 8 * (slot / Mt);
  const int64_t m = slot % Mt;
  if (head >= H) return;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wq = w & 3, dh = w >> 2;  // query group, head-dim half
  const int h = lane >> 5, l32 = lane & 31;
  const int gq = lane >> 4, jq = lane & 15;
  const uint16_t* Qh = Q + head * head_stride;
  const uint16_t* Kh = K + head * head_stride;
  const uint16_t* Vh = V + head * head_stride;
  const int64_t q = m * AB + wq * 32 + l32;

  // Q fragments of this half: Q[q][256 dh + 16 s + 8 h .. +7]
  bf16x8 qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qf[s] = *(const bf16x8*)(Qh + q * D + DH * dh + 16 * s + 8 * h);

  f32x16 o[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) o[u] = f32x16{};
  constexpr float RESCALE = 8.f;
  float mtrue = -INFINITY, mref = -INFINITY, lrun = 0.f;

  const int64_t start = rp[m];
  const int nblk = (int)(rp[m + 1] - start);
  const int nsteps = SPB * nblk;
  const tsp::dma::i32x4 krs = tsp::dma::make_rsrc(Kh, (uint32_t)(S * D * 2));
  const tsp::dma::i32x4 vrs = tsp::dma::make_rsrc(Vh, (uint32_t)(S * D * 2));
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
  auto first_key = [&](int s) { return (int64_t)colblk(s / SPB) * AB + HK * (s % SPB); };

  // ---- stage s into ring slot s % NST: one 1 KiB row per instruction,
  // rows 4w .. 4w + 3 of K and of V per wavefront
  auto issue = [&](int s) {
    const int64_t key0 = first_key(s);
    const uint32_t st = lds0 + (s % NST) * STAGE;
#pragma unroll
    for (int qq = 0; qq < HK / 8; ++qq) {
      const int rr = (HK / 8) * w + qq;
      const int64_t rowoff = (key0 + rr) * ROWB;
      tsp::dma::buffer16(krs, (uint32_t)(rowoff + ((lane ^ kswz(rr)) * 16)), st + rr * 1024);
      tsp::dma::buffer16(vrs, (uint32_t)(rowoff + ((lane ^ (4 * vswz(rr))) * 16)), st + HBYTES + rr * 1024);
    }
  };

  const int vrow = 4 * (gq >> 1) + (jq >> 2);
  const int vsw = 4 * vswz(vrow);
  const int vcol = 16 * (gq & 1) + 4 * (jq & 3);
  const int kx = kswz(l32) ^ h;
  const int vlane = vrow * ROWB + ((vcol >> 3) & 3) * 16 + (vcol & 4) * 2;
  float* xown = xch + w * (16 * 64) + lane;
  const float* xpart = xch + (w ^ 4) * (16 * 64) + lane;

  auto compute = [&](const uint8_t* st, int64_t key0) {
    // ---- partial S^T over this half's head dims (key l32 of the stage,
    // logical chunk 32 dh + 2 ks + h of its row)
    const uint8_t* Ks = st + l32 * ROWB + DH * 2 * dh;
    auto kread = [&](int ks) { return *(const bf16x8*)(Ks + (((2 * ks) ^ kx) * 16)); };
    f32x16 sc;
    bf16x8 ka[2];
    ka[0] = kread(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) ka[(ks + 1) & 1] = kread(ks + 1);
      __builtin_amdgcn_sched_barrier(0);
      sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[ks & 1], qf[ks], ks == 0 ? f32x16{} : sc, 0, 0, 0);
    }
    // ---- exchange: the pair's two halves summed in both wavefronts
#pragma unroll
    for (int v = 0; v < 16; ++v) xown[v * 64] = sc[v];
    tsp::dma::barrier();
#pragma unroll
    for (int v = 0; v < 16; ++v) sc[v] += xpart[v * 64];
    if (key0 + HK > S) {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (key0 + 8 * (v >> 2) + 4 * h + (v & 3) >= S) sc[v] = -INFINITY;
    }
    float mraw = sc[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) mraw = fmaxf(mraw, sc[v]);
    mraw = att::halves_max(mraw);
    mtrue = fmaxf(mtrue, mraw * scale_log2);
    if (__builtin_amdgcn_ballot_w64(mtrue > mref + RESCALE) != 0) {
      const bool move = mtrue > mref + RESCALE;
      const float alpha = move ? (mref == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mref - mtrue)) : 1.f;
      mref = move ? mtrue : mref;
      lrun *= alpha;
#pragma unroll
      for (int u = 0; u < NU; ++u) o[u] *= alpha;
    }
    const float nmx = mref == -INFINITY ? 0.f : -mref;
    float lsum = 0.f;
    bf16x8 pb[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      typedef float f32x8 __attribute__((ext_vector_type(8)));
      f32x8 pv;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[8 * a + i], scale_log2, nmx));
        lsum += p;
        pv[i] = p;
      }
      pb[a] = __builtin_convertvector(pv, bf16x8);
    }
    lrun += lsum;
    // ---- O^T (this half) += V^T P^T; d subtile u of the half is global
    // subtile 8 dh + u, whose swizzled 64-byte piece is 8 dh + (u ^ vx)
    const uint8_t* Vs = st + HBYTES + vlane + DH * 2 * dh;
    const int vx = vsw >> 2;
    auto vread = [&](int a, int u) {
      att::s16x4 r[2];
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const uint8_t* p = Vs + (16 * a + 8 * rr) * ROWB + ((u ^ vx) << 6);
        r[rr] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((att::lds_s16x4*)p);
      }
      return __builtin_bit_cast(bf16x8, __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7));
    };
    bf16x8 vb[2];
    vb[0] = vread(0, 0);
#pragma unroll
    for (int step = 0; step < 2 * NU; ++step) {
      const int a = step / NU, u = step % NU;
      if (step + 1 < 2 * NU) vb[(step + 1) & 1] = vread((step + 1) / NU, (step + 1) % NU);
      __builtin_amdgcn_sched_barrier(0);
      o[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb[step & 1], pb[a], o[u], 0, 0, 0);
    }
  };

  if (nsteps > 0) issue(0);
  for (int s = 0; s < nsteps; ++s) {
    const int64_t key0 = first_key(s);
    tsp::dma::wait_vm<0>();
    tsp::dma::barrier();  // stage s in LDS; slot (s+1) % NST and the exchange are free
    if (s + 1 < nsteps) issue(s + 1);
    compute(lds + (s % NST) * STAGE, key0);
  }

  lrun = att::halves_sum(lrun);
  const bool empty = nblk == 0;
  const float lref = lrun > 1e-12f ? lrun : 1e-12f;
  const float inv = empty ? 0.f : 1.f / lref;
  const float ltrue = mref == -INFINITY ? lrun : lrun * __builtin_amdgcn_exp2f(mref - mtrue);
  const float den = ltrue > 1e-12f ? ltrue : 1e-12f;
  uint16_t* Oq = O + head * head_stride + q * D + DH * dh;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
      u16x4 t;
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = tsp::f32_to_bf16_bits(o[u][4 * g4 + i] * inv);
      *(u16x4*)(Oq + 32 * u + 8 * g4 + 4 * h) = t;
    }
  }
  if (dh == 0 && h == 0 && rmax) {
    const int64_t r = head * Mt * AB + q;
    rmax[r] = empty ? 0.f : mtrue * 0.69314718055994531f;
    rden[r] = empty ? 1e-12f : den;
  }
}

// ---------------------------------------------------------------- fp32 MFMA
//
// bsa_fwd_f32_mfma<D>: fp32, 128-blocks, D in {64, 128, 256}. The work split and
// math of the bf16 kernels (one 256-thread workgroup per (head, 128-query
// block row), a wavefront per 32 queries, S^T = K Q^T with the wave's Q rows
// in registers, online softmax in the exp2 domain with lazy rescaling,
// O^T += V^T P^T with P from registers) on v_mfma_f32_32x32x2_f32:
//   * keys stream through a 2-stage LDS ring of HK = max(32, 4096 / D) keys
//     per stage (K rows then V rows: 32 KiB per stage and two workgroups per
//     CU for D <= 128, 64 KiB per stage and one workgroup per CU for
//     D = 256), filled by direct global->LDS buffer loads issued one stage
//     ahead; rows at or past seq_len read as zero;
//   * S^T: the MFMA k index is the head dimension; at step 4t + c lane half h
//     supplies d = 8t + 4h + c, so one b128 LDS read of a K row feeds four
//     MFMAs and Q[q][8t + 4h .. +3] is the matching register fragment. K
//     rows are stored 16-byte chunk ^ (key % 16) (conflict-free reads of one
//     chunk from 32 rows);
//   * O^T: with NUH = min(NU, 4) subtiles per 128 columns, row r of d
//     subtile u is d = 128*(u / NUH) + NUH*r + u % NUH, so a lane's A
//     operands are one contiguous read V[key][NUH*l32 .. +NUH) per 128
//     columns (conflict-free b128 reads at D = 256) and its outputs cover
//     4*NUH consecutive d per 128 columns; the k index is the key: at step s
//     lane half h supplies key 8*(s/4) + 4h + s%4 of the 32-key tile, which
//     is its own S^T element s, so P is consumed where it was computed.
namespace attf {
template <int D>
struct Cfg {
  static constexpr int HK = D > 128 ? 32 : 4096 / D;  // keys per ring stage
  static constexpr int ROWB = D * 4;        // bytes per K/V row
  static constexpr int HBYTES = HK * ROWB;  // K (or V) bytes per stage: 16 KiB, 32 KiB at D = 256
  static constexpr int STAGE = 2 * HBYTES;
  static constexpr int NST = 2;
  static constexpr int NT = HK / 32;        // 32-key S^T tiles per stage
  static constexpr int NU = D / 32;         // d subtiles of O^T
  static constexpr int NUH = NU < 4 ? NU : 4;  // subtiles per 128 columns
  static constexpr int NB = NU / NUH;       // 128-column groups
  static constexpr int KT = D / 8;          // b128 K reads per S^T tile
  static constexpr int SPB = AB / HK;       // stages per key block
  static constexpr int NI = HBYTES / 4096;  // 1 KiB K (and V) loads per wave per stage
};
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <int NU> struct VRow;
template <> struct VRow<4> { typedef f32x4 type; };
template <> struct VRow<2> { typedef f32x2 type; };
}  // namespace attf

template <int D>
__global__ __launch_bounds__(256, D > 128 ? 1 : 2) void bsa_fwd_f32_mfma(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V, int64_t S,
    int64_t head_stride, int64_t H, const int64_t* __restrict__ rp, const int64_t* __restrict__ ci, int64_t Mt,
    float scale_log2, float* __restrict__ O, float* __restrict__ rmax, float* __restrict__ rden) {
  typedef attf::Cfg<D> C;
  constexpr int HK = C::HK, ROWB = C::ROWB, HBYTES = C::HBYTES, STAGE = C::STAGE, NST = C::NST;
  constexpr int NT = C::NT, NU = C::NU, NUH = C::NUH, NB = C::NB, KT = C::KT, SPB = C::SPB, NI = C::NI;
  typedef typename attf::VRow<NUH>::type vrow_t;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NST * STAGE];

  // XCD-aware order: XCD x walks heads x, x+8, ...; the block rows of one
  // head run side by side and share that head's K/V in the XCD's L2.
  const int64_t g = blockIdx.x;
  const int64_t xcd = g & 7, slot = g >> 3;
  const int64_t head = xcd + 8 * (slot / Mt);
  const int64_t m = slot % Mt;
  if (head >= H) return;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const float* Qh = Q + head * head_stride;
  const float* Kh = K + head * head_stride;
  const float* Vh = V + head * head_stride;
  const int64_t q = m * AB + w * 32 + l32;  // this lane's query (always < S: m < Mt)

  // B operand of S^T: Q[q][8t + 4h + c] at step 4t + c
  f32x4 qf[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) qf[t] = *(const f32x4*)(Qh + q * D + 8 * t + 4 * h);

  f32x16 o[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) o[u] = f32x16{};
  // mtrue: running max of the scaled scores (log2 domain); mref: the
  // reference P and the sums are taken against (lazy rescaling, below)
  constexpr float RESCALE = 8.f;
  float mtrue = -INFINITY, mref = -INFINITY, lrun = 0.f;

  const int64_t start = rp[m];
  const int nblk = (int)(rp[m + 1] - start);
  const int nsteps = SPB * nblk;
  const tsp::dma::i32x4 krs = tsp::dma::make_rsrc(Kh, (uint32_t)(S * D * 4));
  const tsp::dma::i32x4 vrs = tsp::dma::make_rsrc(Vh, (uint32_t)(S * D * 4));
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
  auto first_key = [&](int s) { return (int64_t)colblk(s / SPB) * AB + HK * (s % SPB); };

  // ---- loads of stage s: K and V instructions of 1 KiB, NI + NI per wave
  auto issue = [&](int s) {
    constexpr int LPR = D / 4, RPI = 64 / LPR;  // lanes per row, rows per instruction
    const int64_t key0 = first_key(s);
    const uint32_t st = lds0 + (s % NST) * STAGE;
#pragma unroll
    for (int qq = 0; qq < NI; ++qq) {
      const int j = NI * w + qq;
      const int rr = RPI * j + lane / LPR;  // row of the stage
      const int p = lane % LPR;             // this lane's 16-byte slot in the row
      const uint32_t rowoff = (uint32_t)((key0 + rr) * ROWB);
      tsp::dma::buffer16(krs, rowoff + ((p ^ (rr & 15)) * 16), st + j * 1024);
      tsp::dma::buffer16(vrs, rowoff + p * 16, st + HBYTES + j * 1024);
    }
  };

  const int kx = l32 & 15;  // K swizzle term: row % 16 for rows 32tt + l32
  auto compute = [&](const uint8_t* st, int64_t key0) {
    const uint8_t* Ks = st + l32 * ROWB;
    const uint8_t* Vs = st + HBYTES + 4 * h * ROWB + l32 * NUH * 4;
    auto kread = [&](int tt, int t) { return *(const f32x4*)(Ks + tt * 32 * ROWB + (((2 * t + h) ^ kx) * 16)); };
    struct vrows { vrow_t b[NB]; };
    auto vread = [&](int i) {  // step i of the stage: tile i / 16, step s = i % 16
      const int tt = i >> 4, s = i & 15;
      vrows r;
#pragma unroll
      for (int b = 0; b < NB; ++b) r.b[b] = *(const vrow_t*)(Vs + (32 * tt + 8 * (s >> 2) + (s & 3)) * ROWB + 512 * b);
      return r;
    };
    // ---- S^T tiles (keys 32tt + 8*(v/4) + 4h + v%4, query l32): NT
    // independent chains, K operands read one t ahead
    f32x16 sc[NT];
    f32x4 ka[2][NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) ka[0][tt] = kread(tt, 0);
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      if (t + 1 < KT) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) ka[(t + 1) & 1][tt] = kread(tt, t + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
          sc[tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[t & 1][tt][c], qf[t][c],
                                                        (t == 0 && c == 0) ? f32x16{} : sc[tt], 0, 0, 0);
    }
    // ---- online softmax in the log2 domain (scale_log2 > 0); keys at or
    // past seq_len (only in a block that crosses it) are excluded
    if (key0 + HK > S) {
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (key0 + 32 * tt + 8 * (v >> 2) + 4 * h + (v & 3) >= S) sc[tt][v] = -INFINITY;
    }
    float mraw = sc[0][0];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int v = 0; v < 16; ++v) mraw = fmaxf(mraw, sc[tt][v]);
    mraw = fmaxf(mraw, __shfl_xor(mraw, 32, 64));
    mtrue = fmaxf(mtrue, mraw * scale_log2);
    // P is taken relative to a reference max mref that only moves when the
    // true running max exceeds it by more than RESCALE (log2 units), so
    // P <= 2^RESCALE and o, l rarely need the multiply; o / l is the same
    // quantity for any reference.
    if (__builtin_amdgcn_ballot_w64(mtrue > mref + RESCALE) != 0) {
      const bool move = mtrue > mref + RESCALE;
      const float alpha = move ? (mref == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mref - mtrue)) : 1.f;
      mref = move ? mtrue : mref;
      lrun *= alpha;
#pragma unroll
      for (int u = 0; u < NU; ++u) o[u] *= alpha;
    }
    const float nmx = mref == -INFINITY ? 0.f : -mref;  // -inf scores give p = 0 either way
    float lsum = 0.f;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[tt][v], scale_log2, nmx));
        lsum += p;
        sc[tt][v] = p;
      }
    lsum += __shfl_xor(lsum, 32, 64);
    lrun += lsum;
    // ---- O^T += V^T P^T, V operands read one step ahead
    vrows vb[2];
    vb[0] = vread(0);
#pragma unroll
    for (int i = 0; i < 16 * NT; ++i) {
      if (i + 1 < 16 * NT) vb[(i + 1) & 1] = vread(i + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < NU; ++u)
        o[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(vb[i & 1].b[u / NUH][u % NUH], sc[i >> 4][i & 15], o[u], 0, 0, 0);
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

  // ---- epilogue: element v of subtile u is
  // O[q][128*(u/NUH) + NUH*(8*(v/4) + 4h + v%4) + u%NUH] (o and l both
  // relative to mref); the returned denominator is relative to the true max
  const bool empty = nblk == 0;
  const float lref = lrun > 1e-12f ? lrun : 1e-12f;
  const float inv = empty ? 0.f : 1.f / lref;
  const float ltrue = mref == -INFINITY ? lrun : lrun * __builtin_amdgcn_exp2f(mref - mtrue);
  const float den = ltrue > 1e-12f ? ltrue : 1e-12f;
  float* Oq = O + head * head_stride + q * D;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      float* dst = Oq + 128 * b + NUH * (8 * a + 4 * h);  // 4*NUH consecutive floats: index NUH*c + u
#pragma unroll
      for (int k = 0; k < NUH; ++k) {
        f32x4 t;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int idx = 4 * k + e;  // = NUH*c + u
          t[e] = o[NUH * b + idx % NUH][4 * a + idx / NUH] * inv;
        }
        *(f32x4*)(dst + 4 * k) = t;
      }
    }
  if (h == 0 && rmax) {
    const int64_t r = head * Mt * AB + q;
    rmax[r] = empty ? 0.f : mtrue * 0.69314718055994531f;
    rden[r] = empty ? 1e-12f : den;
  }
}

template <typename T>
int launch_generic(const void* Q, const void* K, const void* V, int64_t H, int64_t S, int64_t D, const int64_t* rp,
                   const int64_t* ci, int64_t b, int64_t Mt, double scale, void* O, void* rmax, void* rden,
                   hipStream_t st) {
  typedef typename AttnAcc<T>::type AccT;
  const int64_t gx = tsp::ceil_div(Mt * b, 128), gy = tsp::ceil_div(D, GEN_DC);
  if (gx > INT32_MAX || gy > 65535 || H > 65535) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_fwd: problem too large for the generic kernel");
  hipLaunchKernelGGL((bsa_fwd_generic<T>), dim3((unsigned)gx, (unsigned)gy, (unsigned)H), dim3(128), 0, st, (const T*)Q,
                     (const T*)K, (const T*)V, S, D, S * D, rp, ci, b, Mt, (AccT)scale, (T*)O, (AccT*)rmax, (AccT*)rden);
  return tsp::check_launch("bsa_fwd_generic launch");
}

}  // namespace

extern "C" int tsp_bsa_fwd(const void* Q, const void* K, const void* V, int dtype, int64_t n_heads, int64_t seq_len,
                           int64_t head_dim, const int64_t* block_row_ptrs, const int64_t* block_col_indices,
                           int64_t block_size, double scale, void* O, void* row_max, void* row_denom, void* stream) {
  if (dtype != TSP_F32 && dtype != TSP_F64 && dtype != TSP_BF16)
    return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_fwd: dtype %d not supported", dtype);
  if (n_heads < 0 || seq_len < 0 || head_dim < 0 || block_size <= 0) return tsp::fail(TSP_EINVAL, "tsp_bsa_fwd: bad size");
  if ((row_max == nullptr) != (row_denom == nullptr)) return tsp::fail(TSP_EINVAL, "tsp_bsa_fwd: row_max and row_denom go together");
  const int64_t Mt = seq_len / block_size;
  if (n_heads == 0 || seq_len == 0 || head_dim == 0) return TSP_OK;
  if (!Q || !K || !V || !O || !block_row_ptrs || !block_col_indices) return tsp::fail(TSP_EINVAL, "tsp_bsa_fwd: null pointer");
  hipStream_t st = (hipStream_t)stream;
  // rows past Mt*block_size have no block row: zero output (the reference's out starts at zero)
  if (Mt * block_size < seq_len) {
    const int64_t es = dtype == TSP_F64 ? 8 : (dtype == TSP_F32 ? 4 : 2);
    const int64_t tail = (seq_len - Mt * block_size) * head_dim * es;
    for (int64_t hh = 0; hh < n_heads; ++hh) {
      int rc = tsp::zero_fill((char*)O + (hh * seq_len + Mt * block_size) * head_dim * es, tail, st);
      if (rc) return rc;
    }
  }
  if (Mt == 0) return TSP_OK;
  const bool bf16_streamed = scale > 0 && (seq_len + AB) * head_dim * 2 <= (int64_t)UINT32_MAX;
  if (dtype == TSP_BF16 && block_size == AB &&
      (head_dim == 64 || head_dim == 128 || ((head_dim == 256 || head_dim == 512) && bf16_streamed)) &&
      ((uintptr_t)Q % 16) == 0 &&
      ((uintptr_t)K % 16) == 0 && ((uintptr_t)V % 16) == 0 && ((uintptr_t)O % 8) == 0) {
    const int64_t grid = tsp::ceil_div(n_heads, 8) * Mt * 8;
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_fwd: problem too large");
    const float sl2 = (float)(scale * 1.4426950408889634);
#define TSP_FWD_BF16(KERNEL)                                                                                        \
  hipLaunchKernelGGL((KERNEL), dim3((unsigned)grid), dim3(256), 0, st, (const uint16_t*)Q, (const uint16_t*)K,       \
                     (const uint16_t*)V, seq_len, seq_len * head_dim, n_heads, block_row_ptrs, block_col_indices, Mt, \
                     sl2, (uint16_t*)O, (float*)row_max, (float*)row_denom)
    if (head_dim == 512)
      hipLaunchKernelGGL(bsa_fwd_bf16_d512, dim3((unsigned)grid), dim3(512), 0, st, (const uint16_t*)Q,
                         (const uint16_t*)K, (const uint16_t*)V, seq_len, seq_len * head_dim, n_heads, block_row_ptrs,
                         block_col_indices, Mt, sl2, (uint16_t*)O, (float*)row_max, (float*)row_denom);
    else if (bf16_streamed && head_dim == 256)
      TSP_FWD_BF16(bsa_fwd_bf16_stream<256>);
    else if (bf16_streamed && head_dim == 128)
      TSP_FWD_BF16(bsa_fwd_bf16_stream<128>);
    else if (bf16_streamed)
      TSP_FWD_BF16(bsa_fwd_bf16_stream<64>);
    else if (head_dim == 128)
      TSP_FWD_BF16(bsa_fwd_bf16_mfma<128>);
    else
      TSP_FWD_BF16(bsa_fwd_bf16_mfma<64>);
#undef TSP_FWD_BF16
    return tsp::check_launch("bsa_fwd_bf16_mfma launch");
  }
  if (dtype == TSP_F32 && block_size == AB && (head_dim == 64 || head_dim == 128 || head_dim == 256) && scale > 0 &&
      ((uintptr_t)Q % 16) == 0 && ((uintptr_t)K % 16) == 0 && ((uintptr_t)V % 16) == 0 && ((uintptr_t)O % 16) == 0 &&
      (seq_len + AB) * head_dim * 4 <= (int64_t)UINT32_MAX) {
    const int64_t grid = tsp::ceil_div(n_heads, 8) * Mt * 8;
    if (grid > INT32_MAX) return tsp::fail(TSP_EUNSUPPORTED, "tsp_bsa_fwd: problem too large");
    const float sl2 = (float)(scale * 1.4426950408889634);
#define TSP_FWD_F32(KERNEL)                                                                                       \
  hipLaunchKernelGGL((KERNEL), dim3((unsigned)grid), dim3(256), 0, st, (const float*)Q, (const float*)K,           \
                     (const float*)V, seq_len, seq_len * head_dim, n_heads, block_row_ptrs, block_col_indices, Mt, \
                     sl2, (float*)O, (float*)row_max, (float*)row_denom)
    if (head_dim == 256)
      TSP_FWD_F32(bsa_fwd_f32_mfma<256>);
    else if (head_dim == 128)
      TSP_FWD_F32(bsa_fwd_f32_mfma<128>);
    else
      TSP_FWD_F32(bsa_fwd_f32_mfma<64>);
#undef TSP_FWD_F32
    return tsp::check_launch("bsa_fwd_f32_mfma launch");
  }
  if (dtype == TSP_F64)
    return launch_generic<double>(Q, K, V, n_heads, seq_len, head_dim, block_row_ptrs, block_col_indices, block_size, Mt,
                                  scale, O, row_max, row_denom, st);
  if (dtype == TSP_F32)
    return launch_generic<float>(Q, K, V, n_heads, seq_len, head_dim, block_row_ptrs, block_col_indices, block_size, Mt,
                                 scale, O, row_max, row_denom, st);
  return launch_generic<uint16_t>(Q, K, V, n_heads, seq_len, head_dim, block_row_ptrs, block_col_indices, block_size,
                                  Mt, scale, O, row_max, row_denom, st);
}
