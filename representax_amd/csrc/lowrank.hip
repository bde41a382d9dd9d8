// Rank-r products of the LoRA adapter and the generic any-shape kernels.
//
//   rank_nt: out[M, r] = bf16(sum_k op(A[m, k]) R[j, k])   (h = x A^T, dh = g_a B)
//   rank_tn: out[P, Q] = f32(bf16(sum_m op(X[m, p]) Y[m, q]))  (dB = g_a^T h,
//            dA = dh^T x), split over token chunks with fp32 partials and a
//            deterministic second-pass sum.
// Both use v_mfma_f32_16x16x32_bf16: lane l of a 16x16 block owns column
// l % 16 and rows 4*(l/16) + v.
#include <cstdlib>

#include "common.h"
#include "kernels.h"
#include "tuning.h"

namespace rpx {

namespace {

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ u32x4_t scale_round8(u32x4_t v, float s) {
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack_bf16x2(bf16lo_to_f32(v[e]) * s, bf16hi_to_f32(v[e]) * s);
  return o;
}

// Loads 8 consecutive bf16 starting at p when all are in range, else only the
// first `valid` (the rest are zero).
__device__ __forceinline__ u32x4_t load8(const uint16_t* p, int valid, bool aligned) {
  if (valid >= 8 && aligned) return *reinterpret_cast<const u32x4_t*>(p);
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t lo = (2 * e < valid) ? p[2 * e] : 0u;
    const uint32_t hi = (2 * e + 1 < valid) ? p[2 * e + 1] : 0u;
    w[e] = lo | (hi << 16);
  }
  return u32x4_t{w[0], w[1], w[2], w[3]};
}

// Output column blocks of the rank-r row kernel: block b is up to 16 rows of
// some R (the rank rows r[b], r[b] + ldr[b], ..., `valid[b]` of them) and
// the matching columns out[b], out[b] + 1, ... of an output with row stride
// ldo[b]. One matrix R [rank, K] is blocks of 16 consecutive rows; several
// adapters of one input (shared-input projections) are their blocks side by
// side.
constexpr int kRankNtMaxBlocks = 8;
struct RankNtBlocks {
  const uint16_t* r[kRankNtMaxBlocks];
  int64_t ldr[kRankNtMaxBlocks];
  uint16_t* out[kRankNtMaxBlocks];
  int64_t ldo[kRankNtMaxBlocks];
  int valid[kRankNtMaxBlocks];
};

// One workgroup per 16 G output rows (G row groups of 16); its four waves
// split K in interleaved 32-deep steps and reduce in LDS. Every fragment of R
// a wave loads serves the G row groups, so R's L2 traffic per row falls by G.
// Each column block's sums are independent of the others', so a block gives
// the same bits whichever blocks share its launch.
template <int RB, int G, int U>
__global__ void __launch_bounds__(256)
    k_rank_nt(const uint16_t* __restrict__ A, int64_t lda, RankNtBlocks blk, int64_t M, int64_t K,
              int round_a, float a_scale) {
  // [v][lane]: a wave's reads and writes of one v are 64 consecutive words
  __shared__ float red[3][G][RB][4][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * 16 * G;
  const int koff = (lane >> 4) * 8;
  const bool a_al = (lda % 8 == 0) && ((reinterpret_cast<uintptr_t>(A) & 15) == 0);
  bool r_al[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
    r_al[rb] = (blk.ldr[rb] % 8 == 0) && ((reinterpret_cast<uintptr_t>(blk.r[rb]) & 15) == 0);
  f32x4_t acc[G][RB];
#pragma unroll
  for (int gi = 0; gi < G; ++gi)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[gi][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // each wave keeps the loads of U steps in flight before their MFMAs
  for (int64_t kb = static_cast<int64_t>(wave) * 32; kb < K; kb += 128 * U) {
    u32x4_t av[U][G];
    u32x4_t rv[U][RB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t kc = kb + 128 * u + koff;
      int kv = static_cast<int>(K - kc);
      kv = kv < 0 ? 0 : (kv > 8 ? 8 : kv);
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        const int64_t row = m0 + 16 * gi + (lane & 15);
        av[u][gi] = load8(A + row * lda + kc, row < M ? kv : 0, a_al);
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int j = lane & 15;
        rv[u][rb] = load8(blk.r[rb] + j * blk.ldr[rb] + kc, j < blk.valid[rb] ? kv : 0, r_al[rb]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        u32x4_t a = av[u][gi];
        if (round_a) a = scale_round8(a, a_scale);
        const bf16x8_t af = as_bf16x8(a);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[gi][rb] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, as_bf16x8(rv[u][rb]), acc[gi][rb], 0, 0, 0);
      }
  }
  // waves 1-3 hand their sums to wave 0 through LDS, which adds them in
  // wave order and stores (lane: rows 4 (lane >> 4) + v, column j = lane & 15)
  if (wave > 0) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[wave - 1][gi][rb][v][lane] = acc[gi][rb][v];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int gi = 0; gi < G; ++gi)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int j = lane & 15;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t mm = m0 + 16 * gi + 4 * (lane >> 4) + v;
        const float s = acc[gi][rb][v] + red[0][gi][rb][v][lane] + red[1][gi][rb][v][lane] +
                        red[2][gi][rb][v][lane];
        if (mm < M && j < blk.valid[rb]) blk.out[rb][mm * blk.ldo[rb] + j] = f32_to_bf16(s);
      }
    }
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// Operand fragment of v_mfma_f32_16x16x32_bf16 whose reduction axis is the
// row axis of a row-major LDS tile (tokens are rows, the output index is a
// column): lane l gets tile[m0 + 8 (l >> 4) + t][c0 + (l & 15)], t = 0..7.
// ds_read_b64_tr_b16 hands lane i of each 16-lane group element i & 3 of the
// 8-byte chunks that lanes 4 e + (i >> 2) address (e = 0..3), so lane j
// addresses row m0 + 8 g + (j >> 2) (+ 4 for the second read) at columns
// c0 + 4 (j & 3): each read yields 4 consecutive tokens of column c0 + i.
// `pitch` (elements) and c0 are multiples of 4, keeping every address 8-byte
// aligned.
__device__ __forceinline__ bf16x8_t tr_frag(const uint16_t* tile, int pitch, int m0, int c0,
                                            int lane) {
  const int j = lane & 15;
  const uint16_t* p = tile + (m0 + 8 * (lane >> 4) + (j >> 2)) * pitch + c0 + 4 * (j & 3);
  const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)p);
  const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + 4 * pitch));
  typedef short i16x8_t __attribute__((ext_vector_type(8)));
  const i16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_t, v);
}

// Token-reduction product: partials[z][p][q] = sum over the token chunk z of
// op(X[m, p]) * Y[m, q]. Tile BP x BQ outputs, `chunk` tokens per workgroup,
// 256 tokens per LDS step; the MFMA operands come straight from the
// token-major LDS tiles through transposing reads.
struct RankTnArgs {
  const uint16_t* X;
  int64_t ldx;
  const uint16_t* Y;
  int64_t ldy;
  int64_t M, P, Q;
  int round_x;
  float x_scale;
  int64_t chunk;
  float* partials;
  int64_t gp, gq, blocks;  // tile grid and gp * gq * splits
  int wide_p;              // 64 x 16 tiles when P is the long side, else 16 x 64
};

constexpr int kTokStep = 256;
constexpr int kRankLds = kTokStep * ((64 + 8) + (16 + 8));  // elements

template <int BP, int BQ>
__device__ __forceinline__ void rank_tn_body(const RankTnArgs& a, int64_t bx, int64_t by,
                                             int64_t bz, uint16_t* lds) {
  // 256 tokens per step: every thread's loads of a step are issued together,
  // and the next step's loads are in flight while this step's MFMAs run from
  // LDS
  constexpr int TS = kTokStep;
  constexpr int PP = 16 / 2;  // padding (elements) per LDS row
  typedef uint16_t RowX[BP + PP];
  typedef uint16_t RowY[BQ + PP];
  RowX* sX = reinterpret_cast<RowX*>(lds);
  RowY* sY = reinterpret_cast<RowY*>(lds + TS * (BP + PP));
  constexpr int XV = TS * (BP / 8) / 256;  // 16-byte vectors per thread per step
  constexpr int YV = TS * (BQ / 8) / 256;
  constexpr int NB = (BP / 16) * (BQ / 16);
  constexpr int PER_WAVE = (NB + 3) / 4;
  const uint16_t* __restrict__ X = a.X;
  const uint16_t* __restrict__ Y = a.Y;
  const int64_t ldx = a.ldx, ldy = a.ldy, P = a.P, Q = a.Q;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t p0 = bx * BP;
  const int64_t q0 = by * BQ;
  const int64_t mbeg = bz * a.chunk;
  int64_t mend = mbeg + a.chunk;
  if (mend > a.M) mend = a.M;
  const bool x_al = (ldx % 8 == 0) && ((reinterpret_cast<uintptr_t>(X) & 15) == 0);
  const bool y_al = (ldy % 8 == 0) && ((reinterpret_cast<uintptr_t>(Y) & 15) == 0);
  f32x4_t acc[PER_WAVE];
#pragma unroll
  for (int b = 0; b < PER_WAVE; ++b) acc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  u32x4_t xr[XV], yr[YV];
  auto load_step = [&](int64_t ms) {
#pragma unroll
    for (int u = 0; u < XV; ++u) {
      const int v = tid + 256 * u;
      const int r = v / (BP / 8);
      const int c = (v % (BP / 8)) * 8;
      const int64_t gm = ms + r;
      int valid = static_cast<int>(P - (p0 + c));
      valid = (gm < mend) ? (valid < 0 ? 0 : (valid > 8 ? 8 : valid)) : 0;
      xr[u] = load8(X + (gm < mend ? gm : mbeg) * ldx + p0 + c, valid, x_al);
    }
#pragma unroll
    for (int u = 0; u < YV; ++u) {
      const int v = tid + 256 * u;
      const int r = v / (BQ / 8);
      const int c = (v % (BQ / 8)) * 8;
      const int64_t gm = ms + r;
      int valid = static_cast<int>(Q - (q0 + c));
      valid = (gm < mend) ? (valid < 0 ? 0 : (valid > 8 ? 8 : valid)) : 0;
      yr[u] = load8(Y + (gm < mend ? gm : mbeg) * ldy + q0 + c, valid, y_al);
    }
  };

  load_step(mbeg);
  for (int64_t ms = mbeg; ms < mend; ms += TS) {
    __syncthreads();  // every wave is done reading the previous step
#pragma unroll
    for (int u = 0; u < XV; ++u) {
      const int v = tid + 256 * u;
      u32x4_t xv = xr[u];
      if (a.round_x) xv = scale_round8(xv, a.x_scale);
      *reinterpret_cast<u32x4_t*>(&sX[v / (BP / 8)][(v % (BP / 8)) * 8]) = xv;
    }
#pragma unroll
    for (int u = 0; u < YV; ++u) {
      const int v = tid + 256 * u;
      *reinterpret_cast<u32x4_t*>(&sY[v / (BQ / 8)][(v % (BQ / 8)) * 8]) = yr[u];
    }
    __syncthreads();
    if (ms + TS < mend) load_step(ms + TS);
    const int steps = static_cast<int>((mend - ms + 31) / 32 < TS / 32 ? (mend - ms + 31) / 32 : TS / 32);
    for (int st = 0; st < steps; ++st) {
#pragma unroll
      for (int b = 0; b < PER_WAVE; ++b) {
        const int blk = wave + 4 * b;
        if (blk < NB) {
          const int bp = blk / (BQ / 16);
          const int bq = blk % (BQ / 16);
          const bf16x8_t xf = tr_frag(&sX[0][0], BP + PP, st * 32, bp * 16, lane);
          const bf16x8_t yf = tr_frag(&sY[0][0], BQ + PP, st * 32, bq * 16, lane);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf, yf, acc[b], 0, 0, 0);
        }
      }
    }
  }
  float* part = a.partials + bz * P * Q;
#pragma unroll
  for (int b = 0; b < PER_WAVE; ++b) {
    const int blk = wave + 4 * b;
    if (blk >= NB) continue;
    const int bp = blk / (BQ / 16);
    const int bq = blk % (BQ / 16);
    const int64_t q = q0 + bq * 16 + (lane & 15);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t p = p0 + bp * 16 + 4 * (lane >> 4) + v;
      if (p < P && q < Q) part[p * Q + q] = acc[b][v];
    }
  }
}

__device__ __forceinline__ void rank_tn_dispatch(const RankTnArgs& a, int64_t b, uint16_t* lds) {
  const int64_t per = a.gp * a.gq;
  const int64_t bz = b / per;
  const int64_t r = b - bz * per;
  if (a.wide_p)
    rank_tn_body<64, 16>(a, r % a.gp, r / a.gp, bz, lds);
  else
    rank_tn_body<16, 64>(a, r % a.gp, r / a.gp, bz, lds);
}

// Up to two token-reduction products in one launch: blocks [0, a0.blocks)
// take the first, the rest the second.
__global__ void __launch_bounds__(256) k_rank_tn(RankTnArgs a0, RankTnArgs a1) {
  __shared__ __align__(16) uint16_t lds[kRankLds];
  const int64_t b = blockIdx.x;
  if (b < a0.blocks)
    rank_tn_dispatch(a0, b, lds);
  else
    rank_tn_dispatch(a1, b - a0.blocks, lds);
}

// out = f32(bf16(sum over splits, in split order)) of [J, P] partials,
// stored as out[j * P + p]; two problems in one launch (the second's
// elements follow the first's in the grid-stride range).
struct ReduceArgs {
  const float* partials;
  int64_t splits, count;
  float* out;
};

// The splits' loads of an element are issued 16 at a time before any add,
// and summed in split order.
__device__ __forceinline__ void reduce_one(const ReduceArgs& a, int64_t e) {
  constexpr int kBatch = 16;
  float s = 0.0f;
  for (int64_t i0 = 0; i0 < a.splits; i0 += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int t = 0; t < kBatch; ++t)
      v[t] = i0 + t < a.splits ? a.partials[(i0 + t) * a.count + e] : 0.0f;
#pragma unroll
    for (int t = 0; t < kBatch; ++t)
      if (i0 + t < a.splits) s += v[t];
  }
  a.out[e] = round_bf16(s);
}

__global__ void __launch_bounds__(256) k_reduce_partials(ReduceArgs a0, ReduceArgs a1) {
  const int64_t total = a0.count + a1.count;
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (e < a0.count)
      reduce_one(a0, e);
    else
      reduce_one(a1, e - a0.count);
  }
}

struct TiledPlan {
  int64_t gp, gq, splits, chunk;
  bool wide_p;
};

TiledPlan plan_tiled(int64_t m, int64_t p, int64_t q) {
  TiledPlan pl;
  pl.wide_p = p >= q;  // <64,16> when P is the long side, else <16,64>
  const int64_t bp = pl.wide_p ? 64 : 16;
  const int64_t bq = pl.wide_p ? 16 : 64;
  pl.gp = ceil_div(p, bp);
  pl.gq = ceil_div(q, bq);
  // 384 workgroups per product: at 4096 tokens (768 -> 3072, r 16) the dA + dB
  // launch fits one round of three workgroups per CU (bwd 60.7 -> 56.9 us);
  // the train-step shapes are unchanged within run-to-run noise
  const int target = tune(kTuneRankBlocks) > 0 ? tune(kTuneRankBlocks) : 384;
  int64_t want = ceil_div(target, pl.gp * pl.gq);
  const int64_t max_splits = ceil_div(m, 64);
  if (want > max_splits) want = max_splits;
  if (want < 1) want = 1;
  pl.chunk = ceil_div(ceil_div(m, want), 32) * 32;
  if (pl.chunk < 32) pl.chunk = 32;
  pl.splits = ceil_div(m, pl.chunk);
  if (pl.splits < 1) pl.splits = 1;
  return pl;
}

// ---------------------------------------------------------------------------
// Generic strided GEMM (any shape/dtype), fp32 accumulate and output.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float load_elem(const void* p, int dtype, int64_t idx) {
  if (dtype == kBF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[idx]);
  return static_cast<const float*>(p)[idx];
}

__device__ __forceinline__ float int4_elem(const Int4Operand& w, int64_t row, int64_t col) {
  const uint32_t byte = w.packed[row * w.packed_cols + col / 2];
  const uint32_t nib = (col & 1) ? (byte >> 4) : (byte & 0xFu);
  const float s = bf16_to_f32(w.scales[row * w.n_groups + col / w.group]);
  const float q = static_cast<float>(static_cast<int>(nib ^ 8u) - 8);
  return round_bf16(q * s);
}

// B(n, k) is B[n * b_sn + k * b_sk], or, for a packed INT4 operand,
// W_b[n, k] (int4_mode 1) or W_b[k, n] (int4_mode 2).
__global__ void __launch_bounds__(256)
    k_generic_gemm(const void* __restrict__ A, int a_dtype, int64_t a_sm, int64_t a_sk,
                   const void* __restrict__ B, int b_dtype, int64_t b_sn, int64_t b_sk,
                   Int4Operand w, int int4_mode, int64_t M, int64_t N, int64_t K,
                   float* __restrict__ out) {
  __shared__ float sa[16][17];
  __shared__ float sb[16][17];
  const int tx = threadIdx.x % 16;
  const int ty = threadIdx.x / 16;
  const int64_t m = static_cast<int64_t>(blockIdx.y) * 16 + ty;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 16 + tx;
  float acc = 0.0f;
  for (int64_t k0 = 0; k0 < K; k0 += 16) {
    const int64_t ka = k0 + tx;
    sa[ty][tx] = (m < M && ka < K) ? load_elem(A, a_dtype, m * a_sm + ka * a_sk) : 0.0f;
    const int64_t nb = static_cast<int64_t>(blockIdx.x) * 16 + ty;
    const int64_t kb = k0 + tx;
    float bv = 0.0f;
    if (nb < N && kb < K) {
      if (int4_mode != 0) {
        bv = (int4_mode == 1) ? int4_elem(w, nb, kb) : int4_elem(w, kb, nb);
      } else {
        bv = load_elem(B, b_dtype, nb * b_sn + kb * b_sk);
      }
    }
    sb[ty][tx] = bv;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) acc = __builtin_fmaf(sa[ty][kk], sb[tx][kk], acc);
    __syncthreads();
  }
  if (m < M && n < N) out[m * N + n] = acc;
}

__global__ void __launch_bounds__(256)
    k_round_store(const float* __restrict__ in, int64_t n, int dtype, void* __restrict__ out) {
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (dtype == kBF16)
      static_cast<uint16_t*>(out)[e] = f32_to_bf16(in[e]);
    else
      static_cast<float*>(out)[e] = in[e];
  }
}

__global__ void __launch_bounds__(256)
    k_transpose_bf16(const uint16_t* __restrict__ in, int64_t rows, int64_t cols, int64_t ld_in,
                     uint16_t* __restrict__ out, int64_t ld_out) {
  __shared__ uint16_t tile[32][33];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int tx = threadIdx.x % 32;
  const int ty = threadIdx.x / 32;  // 0..7
  for (int i = ty; i < 32; i += 8) {
    const int64_t r = r0 + i;
    const int64_t c = c0 + tx;
    tile[i][tx] = (r < rows && c < cols) ? in[r * ld_in + c] : 0;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int64_t c = c0 + i;
    const int64_t r = r0 + tx;
    if (c < cols && r < rows) out[c * ld_out + r] = tile[tx][i];
  }
}

__global__ void __launch_bounds__(256)
    k_f32_to_bf16(const float* __restrict__ in, uint16_t* __restrict__ out, int64_t n) {
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x)
    out[e] = f32_to_bf16(in[e]);
}

__global__ void __launch_bounds__(256) k_fill_f32(float* __restrict__ out, int64_t n, float v) {
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x)
    out[e] = v;
}

int grid1d(int64_t work) {
  int64_t g = ceil_div(work, 256);
  if (g > 8192) g = 8192;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

}  // namespace

// Row groups per workgroup: 4 (64 rows) unless RPX_RANK_NT_G=1 asks for the
// 16-row form; fewer when that leaves under 512 workgroups.
int rank_nt_groups(int64_t m) {
  static const int forced = [] {
    const char* env = std::getenv("RPX_RANK_NT_G");
    return env == nullptr ? 0 : std::atoi(env);
  }();
  if (forced == 1 || forced == 2 || forced == 4) return forced;
  if (ceil_div(m, 64) >= 512) return 4;
  if (ceil_div(m, 32) >= 512) return 2;
  return 1;
}

template <int G, int U>
hipError_t launch_rank_nt_gu(const uint16_t* a, int64_t lda, const RankNtBlocks& blk, int nblk,
                             int64_t m, int64_t k, int ra, float a_scale, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ceil_div(m, 16 * G)));
  switch (nblk) {
    case 1:
      hipLaunchKernelGGL((k_rank_nt<1, G, U>), grid, dim3(256), 0, stream, a, lda, blk, m, k, ra,
                         a_scale);
      break;
    case 2:
      hipLaunchKernelGGL((k_rank_nt<2, G, U>), grid, dim3(256), 0, stream, a, lda, blk, m, k, ra,
                         a_scale);
      break;
    case 3:
      hipLaunchKernelGGL((k_rank_nt<3, G, U>), grid, dim3(256), 0, stream, a, lda, blk, m, k, ra,
                         a_scale);
      break;
    case 4:
      hipLaunchKernelGGL((k_rank_nt<4, G, U>), grid, dim3(256), 0, stream, a, lda, blk, m, k, ra,
                         a_scale);
      break;
    case 5:
    case 6:
    case 7:
    case 8:
      // 5-8 blocks (several adapters of one input); not with all of a long K
      // in flight, whose registers would spill
      if constexpr (U <= 8) {
        if (nblk <= 6)
          hipLaunchKernelGGL((k_rank_nt<6, G, U>), grid, dim3(256), 0, stream, a, lda, blk, m, k,
                             ra, a_scale);
        else
          hipLaunchKernelGGL((k_rank_nt<8, G, U>), grid, dim3(256), 0, stream, a, lda, blk, m, k,
                             ra, a_scale);
        break;
      }
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Steps (128 columns each, over the four waves) in flight per round: the
// whole K range in one round when it is short and a workgroup holds one row
// group (h = x A^T at K = 768: one memory round trip instead of two).
template <int G>
hipError_t launch_rank_nt_g(const uint16_t* a, int64_t lda, const RankNtBlocks& blk, int nblk,
                            int64_t m, int64_t k, int ra, float a_scale, hipStream_t stream) {
  if constexpr (G == 1) {
    const int u = tune(kTuneRankNtU);
    if (u == 16 && nblk <= 4)
      return launch_rank_nt_gu<1, 16>(a, lda, blk, nblk, m, k, ra, a_scale, stream);
    if (u == 4) return launch_rank_nt_gu<1, 4>(a, lda, blk, nblk, m, k, ra, a_scale, stream);
    if (u == 8 || ceil_div(k, 128) > 4)
      return launch_rank_nt_gu<1, 8>(a, lda, blk, nblk, m, k, ra, a_scale, stream);
  }
  return launch_rank_nt_gu<G, (G >= 4 ? 2 : 4)>(a, lda, blk, nblk, m, k, ra, a_scale, stream);
}

hipError_t launch_rank_nt_blocks(const uint16_t* a, int64_t lda, const RankNtBlocks& blk, int nblk,
                                 int64_t m, int64_t k, int ra, float a_scale, hipStream_t stream) {
  switch (rank_nt_groups(m)) {
    case 4: return launch_rank_nt_g<4>(a, lda, blk, nblk, m, k, ra, a_scale, stream);
    case 2: return launch_rank_nt_g<2>(a, lda, blk, nblk, m, k, ra, a_scale, stream);
    default: return launch_rank_nt_g<1>(a, lda, blk, nblk, m, k, ra, a_scale, stream);
  }
}

// Adds the 16-rank column blocks of one product (R [rank, K], out columns
// [0, rank)) to blk; false when they do not fit.
bool add_rank_blocks(RankNtBlocks& blk, int& nblk, const uint16_t* r_mat, int64_t ldr, int64_t rank,
                     uint16_t* out, int64_t ldo) {
  for (int64_t j0 = 0; j0 < rank; j0 += 16) {
    if (nblk == kRankNtMaxBlocks) return false;
    blk.r[nblk] = r_mat + j0 * ldr;
    blk.ldr[nblk] = ldr;
    blk.out[nblk] = out + j0;
    blk.ldo[nblk] = ldo;
    blk.valid[nblk] = static_cast<int>(rank - j0 < 16 ? rank - j0 : 16);
    ++nblk;
  }
  return true;
}

hipError_t launch_rank_nt(const uint16_t* a, int64_t lda, const uint16_t* r_mat, int64_t ldr,
                          int64_t m, int64_t rank, int64_t k, bool round_a, float a_scale,
                          uint16_t* out, int64_t ldo, hipStream_t stream) {
  if (m == 0 || rank == 0) return hipSuccess;
  RankNtBlocks blk{};
  int nblk = 0;
  if (!add_rank_blocks(blk, nblk, r_mat, ldr, rank, out, ldo)) return hipErrorInvalidValue;
  return launch_rank_nt_blocks(a, lda, blk, nblk, m, k, round_a ? 1 : 0, a_scale, stream);
}

int rank_nt_blocks_of(int64_t rank) { return static_cast<int>(ceil_div(rank, 16)); }

hipError_t launch_rank_nt_multi(const uint16_t* a, int64_t lda, int64_t m, int64_t k, int count,
                                const uint16_t* const* r_mats, const int64_t* ranks,
                                uint16_t* const* outs, hipStream_t stream) {
  if (m == 0) return hipSuccess;
  RankNtBlocks blk{};
  int nblk = 0;
  for (int i = 0; i < count; ++i)
    if (!add_rank_blocks(blk, nblk, r_mats[i], k, ranks[i], outs[i], ranks[i]))
      return hipErrorInvalidValue;
  return launch_rank_nt_blocks(a, lda, blk, nblk, m, k, 0, 1.0f, stream);
}

int64_t rank_tn_workspace_floats(int64_t m, int64_t p, int64_t q) {
  const TiledPlan pl = plan_tiled(m, p, q);
  return pl.splits * p * q;
}

namespace {
RankTnArgs rank_tn_args(const uint16_t* x, int64_t ldx, const uint16_t* y, int64_t ldy, int64_t m,
                        int64_t p, int64_t q, bool round_x, float x_scale, float* partials) {
  const TiledPlan pl = plan_tiled(m, p, q);
  RankTnArgs a;
  a.X = x;
  a.ldx = ldx;
  a.Y = y;
  a.ldy = ldy;
  a.M = m;
  a.P = p;
  a.Q = q;
  a.round_x = round_x ? 1 : 0;
  a.x_scale = x_scale;
  a.chunk = pl.chunk;
  a.partials = partials;
  a.gp = pl.gp;
  a.gq = pl.gq;
  a.blocks = pl.gp * pl.gq * pl.splits;
  a.wide_p = pl.wide_p ? 1 : 0;
  return a;
}
}  // namespace

hipError_t launch_rank_tn2(const uint16_t* x0, int64_t ldx0, const uint16_t* y0, int64_t ldy0,
                           int64_t m0, int64_t p0, int64_t q0, bool round_x0, float x_scale0,
                           float* partials0, float* out0, const uint16_t* x1, int64_t ldx1,
                           const uint16_t* y1, int64_t ldy1, int64_t m1, int64_t p1, int64_t q1,
                           bool round_x1, float x_scale1, float* partials1, float* out1,
                           hipStream_t stream) {
  // empty problems: nothing, or a zero fill for an empty token range
  RankTnArgs a0{}, a1{};
  ReduceArgs r0{nullptr, 0, 0, out0}, r1{nullptr, 0, 0, out1};
  if (p0 > 0 && q0 > 0) {
    if (m0 == 0) {
      hipError_t e = launch_fill_f32(out0, p0 * q0, 0.0f, stream);
      if (e != hipSuccess) return e;
    } else {
      a0 = rank_tn_args(x0, ldx0, y0, ldy0, m0, p0, q0, round_x0, x_scale0, partials0);
      r0 = ReduceArgs{partials0, plan_tiled(m0, p0, q0).splits, p0 * q0, out0};
    }
  }
  if (x1 != nullptr && p1 > 0 && q1 > 0) {
    if (m1 == 0) {
      hipError_t e = launch_fill_f32(out1, p1 * q1, 0.0f, stream);
      if (e != hipSuccess) return e;
    } else {
      a1 = rank_tn_args(x1, ldx1, y1, ldy1, m1, p1, q1, round_x1, x_scale1, partials1);
      r1 = ReduceArgs{partials1, plan_tiled(m1, p1, q1).splits, p1 * q1, out1};
    }
  }
  if (a0.blocks + a1.blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rank_tn, dim3(static_cast<unsigned>(a0.blocks + a1.blocks)), dim3(256), 0,
                     stream, a0, a1);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_reduce_partials, dim3(grid1d(r0.count + r1.count)), dim3(256), 0, stream,
                     r0, r1);
  return hipGetLastError();
}

hipError_t launch_rank_tn(const uint16_t* x, int64_t ldx, const uint16_t* y, int64_t ldy,
                          int64_t m, int64_t p, int64_t q, bool round_x, float x_scale,
                          float* partials, float* out, hipStream_t stream) {
  return launch_rank_tn2(x, ldx, y, ldy, m, p, q, round_x, x_scale, partials, out, nullptr, 0,
                         nullptr, 0, 0, 0, 0, false, 1.0f, nullptr, nullptr, stream);
}

hipError_t launch_fill_f32(float* out, int64_t n, float v, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_f32, dim3(grid1d(n)), dim3(256), 0, stream, out, n, v);
  return hipGetLastError();
}

hipError_t launch_transpose_bf16(const uint16_t* in, int64_t rows, int64_t cols, int64_t ld_in,
                                 uint16_t* out, int64_t ld_out, hipStream_t stream) {
  if (rows == 0 || cols == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(ceil_div(cols, 32)), static_cast<unsigned>(ceil_div(rows, 32)));
  hipLaunchKernelGGL(k_transpose_bf16, grid, dim3(256), 0, stream, in, rows, cols, ld_in, out,
                     ld_out);
  return hipGetLastError();
}

hipError_t launch_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_f32_to_bf16, dim3(grid1d(n)), dim3(256), 0, stream, in, out, n);
  return hipGetLastError();
}

hipError_t launch_generic_gemm(const void* a, int a_dtype, int64_t a_sm, int64_t a_sk,
                               const void* b, int b_dtype, int64_t b_sn, int64_t b_sk,
                               const Int4Operand* b_int4, bool int4_transposed, int64_t m,
                               int64_t n, int64_t k, float* out, hipStream_t stream) {
  if (m == 0 || n == 0) return hipSuccess;
  Int4Operand w;
  int mode = 0;
  if (b_int4 != nullptr) {
    w = *b_int4;
    mode = int4_transposed ? 2 : 1;
  }
  const dim3 grid(static_cast<unsigned>(ceil_div(n, 16)), static_cast<unsigned>(ceil_div(m, 16)));
  hipLaunchKernelGGL(k_generic_gemm, grid, dim3(256), 0, stream, a, a_dtype, a_sm, a_sk, b,
                     b_dtype, b_sn, b_sk, w, mode, m, n, k, out);
  return hipGetLastError();
}

hipError_t launch_round_store(const float* in, int64_t n, int dtype, void* out,
                              hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_round_store, dim3(grid1d(n)), dim3(256), 0, stream, in, n, dtype, out);
  return hipGetLastError();
}

}  // namespace rpx
