// fp8 "NT" GEMM for gfx950: out[m, n] = ((sum_k A[m, k] * B[n, k]) * s_a) * s_b
// with A [M, K] and B [N, K] row-major fp8 codes (e4m3fn or e5m2 each), fp32
// accumulation on the 32x32x64 f8f6f4 MFMA, bf16 (round-to-nearest-even) or
// fp32 output. This is the dot_general + rescale of _scaled_fp8_dot
// (representax/precision.py:154-170): the scaling is applied after the
// fp32 dot as (acc * s_a) * s_b, in that order.
#include <atomic>
#include <cstdlib>
#include <cstring>

#include "common.h"
#include "kernels.h"
#include "lds_pipeline.h"
#include "tuning.h"

namespace rpx {
namespace {

constexpr int kBK = 128;  // k bytes (= fp8 elements) per pipeline slice

template <int FA, int FB>
__device__ __forceinline__ f32x16_t mfma_f8(i32x8_t a, i32x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, FA, FB, 0, 0, 0, 0);
}

// Direct-to-LDS loads of one K-slice: this wave's LPW segments (1 KB: 8 rows
// x 128 bytes each; lane l writes bytes [16 l, 16 l + 16) of its segment).
template <int LPW, int NW>
__device__ __forceinline__ void dma_slice(uint8_t* stage, const uint8_t* const* src, int64_t koff,
                                          int wave) {
#pragma unroll
  for (int i = 0; i < LPW; ++i)
    __builtin_amdgcn_global_load_lds(
        src[i] + koff,
        reinterpret_cast<lds_void_t*>(reinterpret_cast<uintptr_t>(stage) + (wave + i * NW) * 1024),
        16, 0, 0);
}

// Fragment of the 32x32x64 MFMA: lane l holds row (l & 31) of a 32-row block,
// k bytes [32 (l >> 5), +32) of the 64-deep step kk.
__device__ __forceinline__ i32x8_t load_frag(const uint8_t* stage, int row, int kk, int half) {
  const int c0 = 4 * kk + 2 * half;
  const int s = swz(row);
  const uint8_t* r = stage + row * kBK;
  const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(r + ((c0 ^ s) << 4));
  const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(r + (((c0 + 1) ^ s) << 4));
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                 (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2_t lds_i32x2_t;

// The same fragment from a K-row tile (LDS row k holds the 128 code bytes of
// columns [0, 128) at reduction index k, 16-byte chunks swizzled by swz(k)):
// lane l needs column col0 + (l & 31) at k = 64 kk + 32 (l >> 5) + [0, 32).
// ds_read_b64_tr_b8 gives lane i of each 16-lane group byte i & 7 of the
// 8-byte pieces that lanes (i >> 3) + 2 e of the group address (e = 0..7),
// as byte e: lane j of the group addresses row k0 + (j >> 1) at column
// c0 + 8 (j & 1), so lane i receives column c0 + i at rows k0 .. k0 + 7.
// Four reads give the 32 reduction bytes, in order.
__device__ __forceinline__ i32x8_t load_frag_krows(const uint8_t* stage, int col0, int kk,
                                                   int lane) {
  const int g = lane >> 4;
  const int j = lane & 15;
  const int col = col0 + 16 * (g & 1) + 8 * (j & 1);
  const int k0 = 64 * kk + 32 * (g >> 1) + (j >> 1);
  i32x8_t f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int k = k0 + 8 * r;
    const uint8_t* q = stage + k * kBK + ((((col >> 4) ^ swz(k))) << 4) + (col & 15);
    const i32x2_t v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t*)q);
    f[2 * r] = v[0];
    f[2 * r + 1] = v[1];
  }
  return f;
}

// Pipelined fp8 GEMM. A workgroup of WM x WN waves computes a BM x BN tile
// (each wave a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks) over the
// K-range of its split. K-slices of 128 bytes of A and B move global -> LDS
// with direct-to-LDS loads into NS rotating stages, NS - 1 slices ahead of
// the one being multiplied. Per slice each wave issues the MFMAs of the first
// 64-deep step, reads the fragments of the second while they run, issues
// those, then waits for the next slice and the barrier while the MFMA pipe is
// still busy. bf16 results go through LDS so each global store writes whole
// 128-byte row segments; fp32 results and split-K partials are stored from
// registers (16 bytes per lane).
// Block `bid` of the `nblk` that run this product (a launch may hold other
// products' blocks too; see k_fp8_gemm_pair).
//
// KROWS: both operands are stored with the reduction index as their row, A
// as [K, M] and B as [K, N] row-major codes (out = A^T B, the weight
// gradient from the tokens-major codes of the gradient and the input, with
// no transposed copies). A slice is then 128 rows of 128 code bytes of each
// operand (128 x 128 tiles only), loaded by the same direct-to-LDS segments
// and read back through transposing LDS reads (load_frag_krows). Columns
// past the edge re-read the last 16 bytes of their row (M, N multiples of
// 16), which only feeds outputs that are never stored.
template <int BM, int BN, int WM, int WN, int NS, int FA, int FB, bool KROWS = false>
__device__ __forceinline__ void fp8_gemm_block(
    int bid, int nblk, const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, int64_t M,
    int64_t N, int64_t K, int64_t k_per_split, const float* __restrict__ s_a,
    const float* __restrict__ s_b, void* __restrict__ out, int out_dtype, int64_t ldc,
    float* __restrict__ partials, int tiles_m, int tiles_n, int band) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM;
  constexpr int TN = BN / WN;
  constexpr int FM = TM / 32;
  constexpr int FN = TN / 32;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be made of 32x32 blocks");
  constexpr int A_SEGS = BM / 8;
  constexpr int SEGS = (BM + BN) / 8;
  static_assert(SEGS % NW == 0, "DMA segments must split evenly over the waves");
  constexpr int LPW = SEGS / NW;
  static_assert(NS >= 2 && NS <= 4 && LPW * (NS - 1) < 64, "vmcnt range");
  constexpr int STAGE = (BM + BN) * kBK;
  static_assert(!KROWS || (BM == kBK && BN == kBK), "K-row operands need 128 x 128 tiles");
  extern __shared__ __align__(16) uint8_t smem[];

  // the scales are needed only by the epilogue; their load is issued first so
  // its latency hides under the main loop
  const float sa = s_a[0];
  const float sb = s_b[0];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM;
  const int wn = wave / WM;

  // Tiles are dealt to the 8 XCDs in contiguous ranges of a banded order
  // (bands of `band` row-blocks walked column by column), so the tiles an
  // XCD holds share few A row-blocks and B column-blocks in its L2; split-K
  // slices are outermost. Partial tiles are stored by the row-major id.
  const int tiles = tiles_m * tiles_n;
  const int b = xcd_block(bid, nblk);
  const int split = b / tiles;
  int tile_m, tile_n;
  band_tile(b % tiles, tiles_m, tiles_n, band, tile_m, tile_n);
  const int tile = tile_m * tiles_n + tile_n;
  const int64_t m0 = static_cast<int64_t>(tile_m) * BM;
  const int64_t n0 = static_cast<int64_t>(tile_n) * BN;
  const int64_t kbeg = static_cast<int64_t>(split) * k_per_split;
  int64_t kend = kbeg + k_per_split;
  if (kend > K) kend = K;
  const int nk = static_cast<int>((kend - kbeg) / kBK);

  // Per-lane DMA sources: segment j = wave + i * NW covers tile rows 8j..8j+7
  // of A (j < A_SEGS) or of B; rows past the edge re-read the last row. With
  // KROWS a segment is 8 reduction rows of the operand's 128-column block,
  // and a K offset moves by whole rows (kstep[i] bytes per unit).
  const int seg_row = lane >> 3;
  const uint8_t* src[LPW];
  int64_t kstep[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int j = wave + i * NW;
    const bool is_a = j < A_SEGS;
    const int trow = (is_a ? 8 * j : 8 * (j - A_SEGS)) + seg_row;
    const int64_t lim = is_a ? M : N;
    if constexpr (KROWS) {
      int64_t c = (is_a ? m0 : n0) + (((lane & 7) ^ swz(trow)) << 4);
      c = c + 16 <= lim ? c : lim - 16;
      src[i] = (is_a ? A : B) + (kbeg + trow) * lim + c;
      kstep[i] = lim;
    } else {
      int64_t r = (is_a ? m0 : n0) + trow;
      r = r < lim ? r : lim - 1;
      src[i] = (is_a ? A : B) + r * K + kbeg + (((lane & 7) ^ swz(trow)) << 4);
      kstep[i] = 1;
    }
  }

  f32x16_t acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[fn][fm][v] = 0.0f;

  const int frow = lane & 31;
  const int half = lane >> 5;
  i32x8_t a_cur[FM], b_cur[FN], a_nxt[FM], b_nxt[FN];
  auto frag = [&](const uint8_t* st, int row0, int kk) {
    if constexpr (KROWS)
      return load_frag_krows(st, row0, kk, lane);
    else
      return load_frag(st, row0 + frow, kk, half);
  };
  auto load_all = [&](const uint8_t* st, int kk, i32x8_t* af, i32x8_t* bf) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) af[fm] = frag(st, wm * TM + fm * 32, kk);
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) bf[fn] = frag(st + BM * kBK, wn * TN + fn * 32, kk);
  };
  // Main loop, branch-free. Slice t lives in stage t % NS. Per slice:
  //   A: MFMAs of 64-deep step 0, each followed by DS reads of step 1's
  //      fragments
  //   barrier: step-1 fragments in registers, slice t + 1 landed (its DMA was
  //            issued NS - 1 slices ago); every wave is done with stage t
  //   B: MFMAs of step 1, each followed by part of the DMA of slice t + NS
  //      into stage t and of the DS reads of slice t + 1's step-0 fragments
  // The fixed order (sched_barrier fences) keeps the DMA and LDS traffic
  // under the MFMAs and the barrier wait under the queued step-0 MFMAs.
  // Refills past the last slice re-read slice nk - 1 into a stage nothing
  // reads again, which keeps the vmcnt accounting constant (LPW per slice).
  constexpr int NMF = FM * FN;
  constexpr int NFR = FM + FN;
  auto mma_one = [&](int i, const i32x8_t* af, const i32x8_t* bf) {
    acc[i / FM][i % FM] = mfma_f8<FB, FA>(bf[i / FM], af[i % FM], acc[i / FM][i % FM]);
  };
  auto frag_one = [&](const uint8_t* st, int kk, int j, i32x8_t* af, i32x8_t* bf) {
    if (j < FM)
      af[j] = frag(st, wm * TM + j * 32, kk);
    else
      bf[j - FM] = frag(st + BM * kBK, wn * TN + (j - FM) * 32, kk);
  };
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int64_t koff = static_cast<int64_t>(s < nk ? s : nk - 1) * kBK;
    if constexpr (KROWS) {
#pragma unroll
      for (int i = 0; i < LPW; ++i) dma_seg(smem + s * STAGE, src[i], koff * kstep[i], wave + i * NW);
    } else {
      dma_slice<LPW, NW>(smem + s * STAGE, src, koff, wave);
    }
  }
  wait_sync<(NS - 1) * LPW>();
  load_all(smem, 0, a_cur, b_cur);
  int stage = 0;
  for (int t = 0; t < nk; ++t) {
    const int next = stage + 1 == NS ? 0 : stage + 1;
    const uint8_t* st = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < NMF; ++i) {
      mma_one(i, a_cur, b_cur);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = i * NFR / NMF; j < (i + 1) * NFR / NMF; ++j) frag_one(st, 1, j, a_nxt, b_nxt);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_sync<(NS - 2) * LPW>();
    const int64_t refill = static_cast<int64_t>(t + NS < nk ? t + NS : nk - 1) * kBK;
    uint8_t* fill = smem + stage * STAGE;
    const uint8_t* nst = smem + next * STAGE;
#pragma unroll
    for (int i = 0; i < NMF; ++i) {
      mma_one(i, a_nxt, b_nxt);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int d = i * LPW / NMF; d < (i + 1) * LPW / NMF; ++d)
        dma_seg(fill, src[d], KROWS ? refill * kstep[d] : refill, wave + d * NW);
#pragma unroll
      for (int j = i * NFR / NMF; j < (i + 1) * NFR / NMF; ++j) frag_one(nst, 0, j, a_cur, b_cur);
      __builtin_amdgcn_sched_barrier(0);
    }
    stage = next;
  }
  // no LDS DMA may still be in flight when the waves go on to the epilogue
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const int64_t mw = m0 + wm * TM;  // first row of this wave's sub-tile
  const int64_t nw = n0 + wn * TN;  // first column
  // D layout (src0 = B fragment): lane holds row m = lane & 31 of the block
  // and columns 8 vg + 4 half + e, e = 0..3, in acc[..][4 vg + e].
  if (partials != nullptr) {
    // Split-K partial tile in fragment order: for each (wave, fn, fm, vg)
    // the 64 lanes store 64 consecutive 16-byte chunks, so every store
    // instruction writes one contiguous kilobyte.
    f32x4_t* dst = reinterpret_cast<f32x4_t*>(
        partials + (static_cast<int64_t>(split) * tiles + tile) * (BM * BN));
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int vg = 0; vg < 4; ++vg) {
          const f32x16_t& a = acc[fn][fm];
          dst[(((wave * FN + fn) * FM + fm) * 4 + vg) * 64 + lane] =
              f32x4_t{a[4 * vg], a[4 * vg + 1], a[4 * vg + 2], a[4 * vg + 3]};
        }
    return;
  }
  if (out_dtype != kBF16) {
    float* o = static_cast<float*>(out);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int64_t m = mw + fm * 32 + frow;
      if (m >= M) continue;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
        for (int vg = 0; vg < 4; ++vg) {
          const int64_t nb = nw + fn * 32 + 8 * vg + 4 * half;
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = (acc[fn][fm][4 * vg + e] * sa) * sb;
          float* d = o + m * ldc + nb;
          if (nb + 3 < N && (ldc & 3) == 0) {
            *reinterpret_cast<f32x4_t*>(d) = f32x4_t{y[0], y[1], y[2], y[3]};
          } else {
            for (int e = 0; e < 4; ++e)
              if (nb + e < N) d[e] = y[e];
          }
        }
      }
    }
    return;
  }

  // bf16: stage this wave's sub-tile in LDS (row pitch TN*2 + 16 bytes), then
  // write whole row segments.
  constexpr int P = TN * 2 + 16;
  wait_sync<0>();  // every wave is done reading the pipeline stages
  uint8_t* reg = smem + wave * (TM * P);
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        const int ml = fm * 32 + frow;
        const int nl = fn * 32 + 8 * vg + 4 * half;
        const f32x16_t& a = acc[fn][fm];
        *reinterpret_cast<u32x2_t*>(reg + ml * P + nl * 2) =
            u32x2_t{pack_bf16x2((a[4 * vg] * sa) * sb, (a[4 * vg + 1] * sa) * sb),
                    pack_bf16x2((a[4 * vg + 2] * sa) * sb, (a[4 * vg + 3] * sa) * sb)};
      }
  constexpr int CPR = TN / 8;  // 16-byte chunks per row
  constexpr int ITS = TM * CPR / 64;
  uint16_t* o = static_cast<uint16_t*>(out);
  const bool vec_ok = (ldc & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  if (vec_ok && mw + TM <= M && nw + TN <= N) {
    // interior sub-tile: all LDS reads, then all 16-byte stores
    u32x4_t v[ITS];
#pragma unroll
    for (int it = 0; it < ITS; ++it) {
      const int idx = it * 64 + lane;
      v[it] = *reinterpret_cast<const u32x4_t*>(reg + (idx / CPR) * P + (idx % CPR) * 16);
    }
#pragma unroll
    for (int it = 0; it < ITS; ++it) {
      const int idx = it * 64 + lane;
      *reinterpret_cast<u32x4_t*>(o + (mw + idx / CPR) * ldc + nw + 8 * (idx % CPR)) = v[it];
    }
    return;
  }
  for (int it = 0; it < ITS; ++it) {
    const int idx = it * 64 + lane;
    const int r = idx / CPR;
    const int c = idx % CPR;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(reg + r * P + c * 16);
    const int64_t m = mw + r;
    const int64_t n = nw + 8 * c;
    if (m >= M) continue;
    uint16_t* d = o + m * ldc + n;
    if (vec_ok && n + 7 < N) {
      *reinterpret_cast<u32x4_t*>(d) = v;
    } else {
      for (int e = 0; e < 8; ++e)
        if (n + e < N) d[e] = static_cast<uint16_t>((v[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
    }
  }
}

template <int BM, int BN, int WM, int WN, int NS, int WPE, int FA, int FB, bool KROWS = false>
__global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
    k_fp8_gemm(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, int64_t M, int64_t N,
               int64_t K, int64_t k_per_split, const float* __restrict__ s_a,
               const float* __restrict__ s_b, void* __restrict__ out, int out_dtype, int64_t ldc,
               float* __restrict__ partials, int tiles_m, int tiles_n, int band) {
  fp8_gemm_block<BM, BN, WM, WN, NS, FA, FB, KROWS>(static_cast<int>(blockIdx.x),
                                                    static_cast<int>(gridDim.x), A, B, M, N, K,
                                                    k_per_split, s_a, s_b, out, out_dtype, ldc,
                                                    partials, tiles_m, tiles_n, band);
}

// Sums the split-K partial tiles written by k_fp8_gemm<BM, BN, WM, WN, ...>
// in split order, scales as (acc * s_a) * s_b and writes bf16 or fp32. One
// thread per 16-byte chunk of the fragment-ordered tile: consecutive threads
// read consecutive chunks of every split.
template <int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(256)
    k_fp8_split_reduce(const float* __restrict__ partials, int splits, int64_t M, int64_t N,
                       int tiles_n, int64_t tiles, const float* __restrict__ s_a,
                       const float* __restrict__ s_b, void* __restrict__ out, int out_dtype,
                       int64_t ldc) {
  constexpr int TM = BM / WM;
  constexpr int TN = BN / WN;
  constexpr int FM = TM / 32;
  constexpr int FN = TN / 32;
  constexpr int CHUNKS = BM * BN / 4;  // per tile
  const float sa = s_a[0];
  const float sb = s_b[0];
  const int64_t total = tiles * CHUNKS;
  const int64_t split_stride = tiles * (BM * BN / 4);
  const f32x4_t* p = reinterpret_cast<const f32x4_t*>(partials);
  for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    f32x4_t s = p[q];
    for (int i = 1; i < splits; ++i) s += p[i * split_stride + q];
    const int64_t tile = q / CHUNKS;
    int r = static_cast<int>(q % CHUNKS);
    const int lane = r & 63;
    r >>= 6;
    const int vg = r & 3;
    r >>= 2;
    const int fm = r % FM;
    r /= FM;
    const int fn = r % FN;
    const int wave = r / FN;
    const int64_t m = (tile / tiles_n) * BM + (wave % WM) * TM + fm * 32 + (lane & 31);
    const int64_t n = (tile % tiles_n) * BN + (wave / WM) * TN + fn * 32 + 8 * vg + 4 * (lane >> 5);
    if (m >= M) continue;
    float y[4];
    for (int e = 0; e < 4; ++e) y[e] = (s[e] * sa) * sb;
    if (out_dtype == kBF16) {
      uint16_t* d = static_cast<uint16_t*>(out) + m * ldc + n;
      if (n + 3 < N && (ldc & 3) == 0) {
        *reinterpret_cast<u32x2_t*>(d) = u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
      } else {
        for (int e = 0; e < 4; ++e)
          if (n + e < N) d[e] = f32_to_bf16(y[e]);
      }
    } else {
      float* d = static_cast<float*>(out) + m * ldc + n;
      for (int e = 0; e < 4; ++e)
        if (n + e < N) d[e] = y[e];
    }
  }
}

// Tile configurations: id, BM, BN, waves along M, waves along N, pipeline
// stages, waves per SIMD the registers are budgeted for.
#define RPX_FP8_CONFIGS(X)     \
  X(1, 128, 128, 2, 2, 2, 2)   \
  X(2, 256, 128, 4, 2, 2, 2)   \
  X(3, 256, 192, 4, 2, 2, 2)   \
  X(4, 128, 192, 2, 2, 2, 2)   \
  X(5, 256, 256, 4, 2, 2, 2)   \
  X(6, 128, 128, 2, 2, 4, 1)   \
  X(7, 128, 192, 2, 2, 3, 1)   \
  X(8, 256, 96, 4, 1, 3, 1)    \
  X(9, 128, 128, 2, 2, 3, 2)   \
  X(10, 256, 128, 2, 2, 3, 1)  \
  X(11, 256, 256, 2, 2, 2, 1)

constexpr int fp8_lds_bytes(int bm, int bn, int wm, int wn, int ns) {
  return ns * (bm + bn) * kBK > wm * wn * (bm / wm) * ((bn / wn) * 2 + 16)
             ? ns * (bm + bn) * kBK
             : wm * wn * (bm / wm) * ((bn / wn) * 2 + 16);
}
constexpr int fp8_blocks_per_cu(int bm, int bn, int wm, int wn, int ns, int wpe) {
  return (160 * 1024 / fp8_lds_bytes(bm, bn, wm, wn, ns)) < (4 * wpe) / (wm * wn)
             ? 160 * 1024 / fp8_lds_bytes(bm, bn, wm, wn, ns)
             : (4 * wpe) / (wm * wn);
}
constexpr int kNumCfg = 12;
#define RPX_CFG_BM(id, bm, bn, wm, wn, ns, wpe) bm,
#define RPX_CFG_BN(id, bm, bn, wm, wn, ns, wpe) bn,
#define RPX_CFG_SLOTS(id, bm, bn, wm, wn, ns, wpe) 256 * fp8_blocks_per_cu(bm, bn, wm, wn, ns, wpe),
constexpr int kCfgBM[kNumCfg] = {0, RPX_FP8_CONFIGS(RPX_CFG_BM)};
constexpr int kCfgBN[kNumCfg] = {0, RPX_FP8_CONFIGS(RPX_CFG_BN)};
constexpr int kCfgSlots[kNumCfg] = {0, RPX_FP8_CONFIGS(RPX_CFG_SLOTS)};

struct Fp8Plan {
  int cfg;
  int64_t splits, k_per_split;
};

// Estimated cycles of a plan on 256 CUs. Per round of resident blocks a CU
// runs `per_cu` blocks whose MFMA work (8192 fp8 flops per clock per CU) and
// global->LDS fill (about 64 bytes per clock per CU when every CU of an XCD
// streams from its L2) overlap, plus a fixed pipeline fill/drain. Split-K adds
// the partial tiles' write and read-back at `partial_rate` bytes per clock
// chip-wide and one more launch.
double plan_cycles(int cfg, int64_t m, int64_t n, int64_t kslices, int64_t kps, int64_t splits,
                   double partial_rate) {
  const double bm = kCfgBM[cfg], bn = kCfgBN[cfg];
  const int64_t tiles = ceil_div(m, kCfgBM[cfg]) * ceil_div(n, kCfgBN[cfg]);
  const int64_t blocks = tiles * splits;
  const int64_t slots = kCfgSlots[cfg];
  const double per_cu = static_cast<double>(slots) / 256.0;
  const double rounds = static_cast<double>(ceil_div(blocks, slots));
  // a last partial round only occupies the CUs it has blocks for
  const double k = static_cast<double>(kps) * kBK;
  const double mfma = per_cu * bm * bn * k * 2.0 / 8192.0;
  const double fill = per_cu * (bm + bn) * k / 64.0;
  const double round = (mfma > fill ? mfma : fill) + 2500.0;
  double cyc = rounds * round;
  if (splits > 1)
    cyc += static_cast<double>(splits + 1) * tiles * bm * bn * 4.0 / partial_rate + 4000.0;
  (void)kslices;
  return cyc;
}

// Cheapest split count for one tile configuration under plan_cycles, with
// the partial tiles priced at 2 KB per clock.
constexpr double kPartialRate = 2048.0;
Fp8Plan plan_for(int cfg, int64_t m, int64_t n, int64_t kslices, double* cost_out,
                 double partial_rate = kPartialRate) {
  Fp8Plan best{cfg, 1, kslices * kBK};
  double best_cost = -1.0;
  const int64_t tiles = ceil_div(m, kCfgBM[cfg]) * ceil_div(n, kCfgBN[cfg]);
  const int64_t forced = tune(kTuneFp8Splits);
  if (forced > 0 && forced <= kslices) {
    const int64_t kps = ceil_div(kslices, forced);
    if (ceil_div(kslices, kps) == forced) {
      if (cost_out != nullptr) *cost_out = plan_cycles(cfg, m, n, kslices, kps, forced, partial_rate);
      return Fp8Plan{cfg, forced, kps * kBK};
    }
  }
  for (int64_t s = 1; s <= 32 && s <= kslices; ++s) {
    if (s > 1 && tiles * s > 2 * kCfgSlots[cfg]) break;
    const int64_t kps = ceil_div(kslices, s);
    const int64_t splits = ceil_div(kslices, kps);
    if (splits != s) continue;
    const double cost = plan_cycles(cfg, m, n, kslices, kps, splits, partial_rate);
    if (best_cost < 0.0 || cost < best_cost) {
      best_cost = cost;
      best = Fp8Plan{cfg, splits, kps * kBK};
    }
  }
  if (cost_out != nullptr) *cost_out = best_cost;
  return best;
}

// The three-stage 128 x 128 tile for long reductions over few tiles (the
// weight gradients, K = tokens). Its split count aims for about 21 128-deep
// slices per split, within one round of blocks (at most 256): a block that
// runs alone on its CU takes ~770 clocks per slice (latency, not the
// MFMA or fill rate plan_cycles assumes), and each split's partial tiles and
// reduce cost about as much as three slices. Measured on the 768 x 768
// weight gradient (36 tiles, graph-timed per call): 4096 tokens, 2-3 splits
// 13.8 us against 14.7 unsplit; 8192 tokens, 3 splits 16.1 us against 17.1
// for 4 and 16.9 for 5; 16384 tokens, 6 splits 19.5 us against 20.0 for 5
// and 20.9 for 4. Wider outputs (144 tiles of 3072 x 768) stay unsplit, and
// unsplit reductions of 16 or more slices gain from the third stage
// (3072 x 768 x 4096: 17.0 us against 23.5 with two stages).
Fp8Plan split_tile_plan(int64_t m, int64_t n, int64_t kslices) {
  const int64_t tiles = ceil_div(m, kCfgBM[9]) * ceil_div(n, kCfgBN[9]);
  int64_t s = (kslices + 10) / 21;
  const int64_t cap = 256 / tiles;
  if (s > cap) s = cap;
  if (s > kslices) s = kslices;
  if (s < 1) s = 1;
  const int64_t forced = tune(kTuneFp8Splits);
  if (forced > 0 && forced <= kslices) s = forced;
  const int64_t kps = ceil_div(kslices, s);
  return Fp8Plan{9, ceil_div(kslices, kps), kps * kBK};
}

Fp8Plan plan_fp8(int64_t m, int64_t n, int64_t k) {
  const int64_t kslices = k / kBK;
  const int forced = tune(kTuneFp8Tile);
  if (forced != 0) return plan_for(forced, m, n, kslices, nullptr);
  Fp8Plan best{1, 1, k};
  double best_cost = -1.0;
  for (int cfg = 1; cfg <= 5; ++cfg) {
    double cost;
    const Fp8Plan p = plan_for(cfg, m, n, kslices, &cost);
    if (best_cost < 0.0 || cost < best_cost) {
      best_cost = cost;
      best = p;
    }
  }
  static const bool model_only = [] {
    const char* env = std::getenv("RPX_FP8_PLAN");
    return env != nullptr && std::strcmp(env, "model") == 0;
  }();
  if (best.cfg == 1 && !model_only) {
    // RPX_FP8_PLAN=model keeps the model's choice (for comparisons).
    // Measured on the BERT-base shapes (tokens 8192, widths 768 / 3072),
    // where the model above does not see pipeline depth: split-K tiles run
    // long K ranges and gain from a third stage (768 x 768 x 8192: 17.6 us
    // against 22.6); unsplit products with >= 16 K slices (K >= 2048) prefer 128 x 192
    // tiles with three stages (8192 x 768 x 3072: 21.9 us against 23.3), and
    // short ones 128 x 192 tiles with two (8192 x 768 x 768: 10.4-11.1 us
    // against 11.1-11.7) when those fill one or two rounds of CUs. Each keeps
    // its own split count.
    const int64_t tiles192 = ceil_div(m, kCfgBM[4]) * ceil_div(n, kCfgBN[4]);
    if (best.splits == 1 && kslices >= 16 && tiles192 >= 200 && tiles192 <= 512) {
      best = plan_for(7, m, n, kslices, nullptr);
    } else if (best.splits > 1 || kslices >= 16) {
      best = split_tile_plan(m, n, kslices);
    } else if (tiles192 >= 256 && tiles192 <= 512) {
      best = plan_for(4, m, n, kslices, nullptr);
    }
  }
  return best;
}

// Rows per band of the tile order. The XCD that runs t = blocks / 8
// consecutive tiles of a b-row band order holds about `rows` A row-blocks and
// `cols` B column-blocks (both fp8, over the same K range), and streams
// rows * BM + cols * BN bytes per unit of K through its L2; b minimizes that
// (ties keep the smaller b, row-major order at b = 1). The kTuneBand knob
// forces a band.
int fp8_band(int tiles_m, int tiles_n, int64_t blocks, int bm, int bn) {
  const int forced = tune(kTuneBand);
  if (forced > 0) return forced < tiles_m ? forced : tiles_m;
  const int64_t t = blocks / 8 > 0 ? blocks / 8 : 1;
  int best = 1;
  int64_t best_cost = -1;
  for (int b = 1; b <= tiles_m && b <= 64; ++b) {
    const int64_t band_tiles = static_cast<int64_t>(b) * tiles_n;
    int64_t rows, cols;
    if (t <= band_tiles) {
      rows = t < b ? t : b;
      cols = ceil_div(t, b);
    } else {
      const int64_t full = t / band_tiles;
      const int64_t rem = t - full * band_tiles;
      rows = full * b + (rem < b ? rem : b);
      cols = tiles_n;
    }
    const int64_t cost = rows * bm + cols * bn;
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = b;
    }
  }
  return best;
}

template <int BM, int BN, int WM, int WN, int NS, int WPE, int FA, int FB, bool KROWS = false>
hipError_t run_fp8(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                   const Fp8Plan& plan, const float* s_a, const float* s_b, void* out,
                   int out_dtype, int64_t ldc, float* partials, hipStream_t stream) {
  constexpr int kLds = fp8_lds_bytes(BM, BN, WM, WN, NS);
  static_assert(kLds <= 160 * 1024, "LDS budget");
  const int tiles_m = static_cast<int>(ceil_div(m, BM));
  const int tiles_n = static_cast<int>(ceil_div(n, BN));
  auto kern = k_fp8_gemm<BM, BN, WM, WN, NS, WPE, FA, FB, KROWS>;
  static std::atomic<unsigned> lds_set{0};
  hipError_t le = ensure_lds_limit(reinterpret_cast<const void*>(kern), kLds, lds_set);
  if (le != hipSuccess) return le;
  const unsigned blocks = static_cast<unsigned>(tiles_m) * tiles_n * plan.splits;
  const int band = fp8_band(tiles_m, tiles_n, blocks, BM, BN);
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * WM * WN), kLds, stream, a, b, m, n, k,
                     plan.k_per_split, s_a, s_b, out, out_dtype, ldc,
                     plan.splits > 1 ? partials : nullptr, tiles_m, tiles_n, band);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || plan.splits == 1) return e;
  const int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
  int64_t g = ceil_div(tiles * (BM * BN / 4), 256);
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL((k_fp8_split_reduce<BM, BN, WM, WN>), dim3(static_cast<unsigned>(g)), dim3(256),
                     0, stream, partials, static_cast<int>(plan.splits), m, n, tiles_n, tiles, s_a,
                     s_b, out, out_dtype, ldc);
  return hipGetLastError();
}

template <int FA, int FB>
hipError_t dispatch_fp8(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                        const float* s_a, const float* s_b, void* out, int out_dtype, int64_t ldc,
                        float* partials, hipStream_t stream) {
  const Fp8Plan p = plan_fp8(m, n, k);
  switch (p.cfg) {
#define RPX_CFG_CASE(id, bm, bn, wm, wn, ns, wpe)                                                 \
  case id:                                                                                        \
    return run_fp8<bm, bn, wm, wn, ns, wpe, FA, FB>(a, b, m, n, k, p, s_a, s_b, out, out_dtype, \
                                                    ldc, partials, stream);
    RPX_FP8_CONFIGS(RPX_CFG_CASE)
#undef RPX_CFG_CASE
    default:
      return hipErrorInvalidValue;
  }
}

// Plans of the K-row form (128 x 128 tiles only): the three-stage split-K
// tile for long reductions, as for the weight gradients of the row-major
// form, else the two-stage tile; a forced 128 x 128 configuration is kept.
Fp8Plan plan_fp8_krows(int64_t m, int64_t n, int64_t k) {
  const int64_t kslices = k / kBK;
  const int forced = tune(kTuneFp8Tile);
  if (forced == 1 || forced == 6 || forced == 9) return plan_for(forced, m, n, kslices, nullptr);
  if (kslices >= 16) return split_tile_plan(m, n, kslices);
  return plan_for(1, m, n, kslices, nullptr);
}

template <int FA, int FB>
hipError_t dispatch_fp8_krows(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                              const float* s_a, const float* s_b, void* out, int out_dtype,
                              int64_t ldc, float* partials, hipStream_t stream) {
  const Fp8Plan p = plan_fp8_krows(m, n, k);
  switch (p.cfg) {
    case 1:
      return run_fp8<128, 128, 2, 2, 2, 2, FA, FB, true>(a, b, m, n, k, p, s_a, s_b, out,
                                                        out_dtype, ldc, partials, stream);
    case 6:
      return run_fp8<128, 128, 2, 2, 4, 1, FA, FB, true>(a, b, m, n, k, p, s_a, s_b, out,
                                                        out_dtype, ldc, partials, stream);
    case 9:
      return run_fp8<128, 128, 2, 2, 3, 2, FA, FB, true>(a, b, m, n, k, p, s_a, s_b, out,
                                                        out_dtype, ldc, partials, stream);
    default:
      return hipErrorInvalidValue;
  }
}

// One product of a paired launch.
struct Fp8Part {
  const uint8_t* a;
  const uint8_t* b;
  int64_t m, n, k, k_per_split;
  const float* s_a;
  const float* s_b;
  void* out;
  int64_t ldc;
  float* partials;  // split-K partial tiles, nullptr when unsplit
  int tiles_m, tiles_n, band, blocks;
};

#define RPX_CFG_WM(id, bm, bn, wm, wn, ns, wpe) wm,
#define RPX_CFG_WN(id, bm, bn, wm, wn, ns, wpe) wn,
#define RPX_CFG_NS(id, bm, bn, wm, wn, ns, wpe) ns,
#define RPX_CFG_WPE(id, bm, bn, wm, wn, ns, wpe) wpe,
constexpr int kCfgWM[kNumCfg] = {0, RPX_FP8_CONFIGS(RPX_CFG_WM)};
constexpr int kCfgWN[kNumCfg] = {0, RPX_FP8_CONFIGS(RPX_CFG_WN)};
constexpr int kCfgNS[kNumCfg] = {0, RPX_FP8_CONFIGS(RPX_CFG_NS)};
constexpr int kCfgWPE[kNumCfg] = {0, RPX_FP8_CONFIGS(RPX_CFG_WPE)};
template <int ID>
struct Fp8Cfg {
  static constexpr int BM = kCfgBM[ID], BN = kCfgBN[ID], WM = kCfgWM[ID], WN = kCfgWN[ID],
                       NS = kCfgNS[ID], WPE = kCfgWPE[ID];
};

template <int ID, int FA, int FB, bool KROWS>
__device__ __forceinline__ void fp8_part_block(int bid, int nblk, const Fp8Part& p, int out_dtype) {
  using C = Fp8Cfg<ID>;
  fp8_gemm_block<C::BM, C::BN, C::WM, C::WN, C::NS, FA, FB, KROWS>(
      bid, nblk, p.a, p.b, p.m, p.n, p.k, p.k_per_split, p.s_a, p.s_b, p.out, out_dtype, p.ldc,
      p.partials, p.tiles_m, p.tiles_n, p.band);
}

// The weight and input gradients of one fp8 linear in one launch (both
// e5m2 x e4m3, four-wave tiles): blocks [0, w.blocks) run the weight
// gradient's tiles (K-row form, from the tokens-major codes of the gradient
// and the input), the long reductions over the tokens, which leave most CUs
// idle on their own (36 tiles x 3 splits for a 768 x 768 weight); the input
// gradient's tiles, dispatched after them, fill those CUs.
template <int CW, int CX, int WPE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
    k_fp8_gemm_pair(Fp8Part w, Fp8Part x, int out_dtype) {
  const int b = static_cast<int>(blockIdx.x);
  if (b < w.blocks)
    fp8_part_block<CW, 1, 0, true>(b, w.blocks, w, out_dtype);
  else
    fp8_part_block<CX, 1, 0, false>(b - w.blocks, x.blocks, x, out_dtype);
}

template <int CW, int CX>
hipError_t run_fp8_pair(Fp8Part w, Fp8Part x, int w_splits, int out_dtype, hipStream_t stream) {
  using W = Fp8Cfg<CW>;
  using X = Fp8Cfg<CX>;
  static_assert(W::WM * W::WN == 4 && X::WM * X::WN == 4, "paired tiles have four waves");
  constexpr int kW = fp8_lds_bytes(W::BM, W::BN, W::WM, W::WN, W::NS);
  constexpr int kX = fp8_lds_bytes(X::BM, X::BN, X::WM, X::WN, X::NS);
  constexpr int kLds = kW > kX ? kW : kX;
  constexpr int kWpe = W::WPE < X::WPE ? W::WPE : X::WPE;
  static_assert(kLds <= 160 * 1024, "LDS budget");
  auto kern = k_fp8_gemm_pair<CW, CX, kWpe>;
  static std::atomic<unsigned> lds_set{0};
  hipError_t le = ensure_lds_limit(reinterpret_cast<const void*>(kern), kLds, lds_set);
  if (le != hipSuccess) return le;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(w.blocks + x.blocks)), dim3(256), kLds,
                     stream, w, x, out_dtype);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || w_splits == 1) return e;
  const int64_t tiles = static_cast<int64_t>(w.tiles_m) * w.tiles_n;
  int64_t g = ceil_div(tiles * (W::BM * W::BN / 4), 256);
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL((k_fp8_split_reduce<W::BM, W::BN, W::WM, W::WN>), dim3(static_cast<unsigned>(g)),
                     dim3(256), 0, stream, w.partials, w_splits, w.m, w.n, w.tiles_n, tiles, w.s_a,
                     w.s_b, w.out, out_dtype, w.ldc);
  return hipGetLastError();
}

Fp8Part make_part(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                  const Fp8Plan& p, const float* s_a, const float* s_b, void* out, int64_t ldc,
                  float* partials) {
  Fp8Part q;
  q.a = a;
  q.b = b;
  q.m = m;
  q.n = n;
  q.k = k;
  q.k_per_split = p.k_per_split;
  q.s_a = s_a;
  q.s_b = s_b;
  q.out = out;
  q.ldc = ldc;
  q.partials = p.splits > 1 ? partials : nullptr;
  q.tiles_m = static_cast<int>(ceil_div(m, kCfgBM[p.cfg]));
  q.tiles_n = static_cast<int>(ceil_div(n, kCfgBN[p.cfg]));
  q.blocks = q.tiles_m * q.tiles_n * static_cast<int>(p.splits);
  q.band = fp8_band(q.tiles_m, q.tiles_n, q.blocks, kCfgBM[p.cfg], kCfgBN[p.cfg]);
  return q;
}

}  // namespace

int fp8_tile_count() { return kNumCfg; }

int64_t fp8_gemm_workspace_floats(int64_t m, int64_t n, int64_t k) {
  const Fp8Plan p = plan_fp8(m, n, k);
  if (p.splits <= 1) return 0;
  return p.splits * ceil_div(m, kCfgBM[p.cfg]) * ceil_div(n, kCfgBN[p.cfg]) * kCfgBM[p.cfg] *
         kCfgBN[p.cfg];
}

hipError_t launch_fp8_gemm(const uint8_t* a, int fmt_a, const float* s_a, const uint8_t* b,
                           int fmt_b, const float* s_b, int64_t m, int64_t n, int64_t k,
                           void* out, int out_dtype, int64_t ldc, float* split_ws,
                           int64_t split_ws_floats, hipStream_t stream) {
  if (m == 0 || n == 0) return hipSuccess;
  if (k % kBK != 0 || split_ws_floats < fp8_gemm_workspace_floats(m, n, k))
    return hipErrorInvalidValue;
  // MFMA format codes: 0 = fp8 (e4m3), 1 = bf8 (e5m2)
  if (fmt_a == kE4M3FN && fmt_b == kE4M3FN)
    return dispatch_fp8<0, 0>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
  if (fmt_a == kE5M2 && fmt_b == kE4M3FN)
    return dispatch_fp8<1, 0>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
  if (fmt_a == kE4M3FN && fmt_b == kE5M2)
    return dispatch_fp8<0, 1>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
  return dispatch_fp8<1, 1>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
}

// Each product keeps its own plan (the 512-thread 256 x 192 input-gradient
// tile becomes 128 x 192, which sums every output in the same order), so the
// outputs equal the two separate launches' bit for bit. The BERT-base fp8
// step at 8192 tokens (graph replays, one process): 0.5455 ms with two
// launches per backward, 0.5240 with only the split-K weight gradients
// (768 -> 768) paired, 0.5150 with every backward paired. Kernel traces
// put the gain in the 768 -> 768 backward (31.2 -> 23.7 us, its weight
// gradient runs 108 latency-bound blocks); the FFN backwards look even
// under the profiler, which serializes the graph's nodes.
hipError_t launch_fp8_backward_pair(const uint8_t* g, const uint8_t* right_codes,
                                    const uint8_t* left_codes, const float* s_g,
                                    const float* s_right, const float* s_left, int64_t m,
                                    int64_t k, int64_t n, void* d_left, void* d_right_t,
                                    int out_dtype, float* split_ws, int64_t split_ws_floats,
                                    hipStream_t stream, bool* launched) {
  *launched = false;
  if (tune(kTuneFp8Pair) == 0) return hipSuccess;
  if (n % kBK != 0 || m % kBK != 0 || k % 16 != 0) return hipSuccess;
  // d_left [m, k] = g [m, n] . right^T; d_right^T [n, k] = g^T . left, from
  // g [m, n] and left [m, k] as K-row operands
  Fp8Plan px = plan_fp8(m, k, n);
  const Fp8Plan pw = plan_fp8_krows(n, k, m);
  if (px.cfg == 3 && px.splits == 1) px = Fp8Plan{4, 1, n};
  if (px.splits != 1 || pw.cfg != 9) return hipSuccess;
  if (pw.splits > 1 &&
      pw.splits * ceil_div(n, kCfgBM[9]) * ceil_div(k, kCfgBN[9]) * kCfgBM[9] * kCfgBN[9] >
          split_ws_floats)
    return hipSuccess;
  const Fp8Part x = make_part(g, right_codes, m, k, n, px, s_g, s_right, d_left, k, nullptr);
  // d_right^T = ((g^T . left) * s_left) * s_g, the separate launch's order
  const Fp8Part w = make_part(g, left_codes, n, k, m, pw, s_left, s_g, d_right_t, k, split_ws);
  hipError_t e;
  if (px.cfg == 4)
    e = run_fp8_pair<9, 4>(w, x, static_cast<int>(pw.splits), out_dtype, stream);
  else if (px.cfg == 7)
    e = run_fp8_pair<9, 7>(w, x, static_cast<int>(pw.splits), out_dtype, stream);
  else
    return hipSuccess;
  *launched = e == hipSuccess;
  return e;
}

int64_t fp8_gemm_krows_workspace_floats(int64_t m, int64_t n, int64_t k) {
  const Fp8Plan p = plan_fp8_krows(m, n, k);
  if (p.splits <= 1) return 0;
  return p.splits * ceil_div(m, kCfgBM[p.cfg]) * ceil_div(n, kCfgBN[p.cfg]) * kCfgBM[p.cfg] *
         kCfgBN[p.cfg];
}

hipError_t launch_fp8_gemm_krows(const uint8_t* a, int fmt_a, const float* s_a, const uint8_t* b,
                                 int fmt_b, const float* s_b, int64_t m, int64_t n, int64_t k,
                                 void* out, int out_dtype, int64_t ldc, float* split_ws,
                                 int64_t split_ws_floats, hipStream_t stream) {
  if (m == 0 || n == 0) return hipSuccess;
  if (k % kBK != 0 || m % 16 != 0 || n % 16 != 0 ||
      split_ws_floats < fp8_gemm_krows_workspace_floats(m, n, k))
    return hipErrorInvalidValue;
  if (fmt_a == kE4M3FN && fmt_b == kE4M3FN)
    return dispatch_fp8_krows<0, 0>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
  if (fmt_a == kE5M2 && fmt_b == kE4M3FN)
    return dispatch_fp8_krows<1, 0>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
  if (fmt_a == kE4M3FN && fmt_b == kE5M2)
    return dispatch_fp8_krows<0, 1>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
  return dispatch_fp8_krows<1, 1>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
}

}  // namespace rpx
