// bf16 MFMA "NT" GEMM for gfx950: C[M, N] = A[M, K] . B[N, K]^T with both
// operands K-contiguous. B is either bf16 rows or packed INT4 rows (two
// nibbles per byte, per-row or per-group bf16 scales) that are dequantized
// exactly, bf16(q * s), from LDS into the MFMA fragments.
//
// Pipeline: K-slices of 64 elements. A (and bf16 B) rows move global -> LDS
// as 128-byte swizzled rows, packed B rows as 32 bytes, all with direct-to-LDS
// loads into NS rotating stages. Within a slice a lane covers 32 consecutive
// k of each row: MFMA step j takes k = 32 h + 8 j + [0, 8) from lane half h
// (the same permutation for both operands), so one 16-byte LDS read per
// packed B fragment serves the whole slice.
//
// A third B form serves the input gradient of the INT4 + LoRA linear,
// dx = g . W_b: B[n, k] = W_b[k, n], read straight from the packed weight
// ([K rows, N / 2 bytes], the reduction running over packed rows). Each
// 64-row slice of packed bytes and its scales land in LDS by DMA one slice
// ahead of A; during the previous slice the workgroup dequantizes it once,
// bf16(q * s) as above, into a bf16 [64 k][BN n] buffer, and the MFMA
// fragments come from that buffer through transposing LDS reads
// (ds_read_b64_tr_b16). No bf16 copy of W_b^T is written to memory. It is
// bit-identical to the bf16 W_b^T form but slower (the INT4 + LoRA backward
// at 16384 x 2048 <- 6144: 790 against 535 us; at 4096 x 768 <- 3072: 90
// against 62 us): the dequantized slice's LDS stores, its scale and packed
// reads and two transposing reads per fragment about double the LDS
// instructions per slice of a loop whose LDS traffic is already close to its
// MFMA time. The backward uses it only on request (RPX_DX_PACKED=1).
//
// Accumulator orientation: the MFMA's first operand is the B (weight) row
// fragment, so lane l of a 32x32 block owns output row m = l % 32 and the
// registers v = 0..15 hold output columns n = 8*(v/4) + 4*(l/32) + v%4,
// which lets each lane store 4 consecutive bf16 outputs at once.
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "act.h"
#include "lds_pipeline.h"
#include "tuning.h"

namespace rpx {

namespace {

constexpr int kBK = 64;  // k elements per slice

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// Number of the 8 ranks starting at j that exist (0..8).
__device__ __forceinline__ int valid8(int64_t rank, int64_t j) {
  const int64_t v = rank - j;
  return static_cast<int>(v < 0 ? 0 : (v > 8 ? 8 : v));
}

// 8 bf16 at base[e * stride], e < valid (zero beyond); one 16-byte load when
// contiguous, complete and aligned.
__device__ __forceinline__ bf16x8_t load8_j(const uint16_t* base, int64_t stride, int valid) {
  if (stride == 1 && valid == 8 && (reinterpret_cast<uintptr_t>(base) & 15) == 0)
    return *reinterpret_cast<const bf16x8_t*>(base);
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t lo = (2 * e < valid) ? base[(2 * e) * stride] : 0u;
    const uint32_t hi = (2 * e + 1 < valid) ? base[(2 * e + 1) * stride] : 0u;
    w[e] = lo | (hi << 16);
  }
  return as_bf16x8(u32x4_t{w[0], w[1], w[2], w[3]});
}

// Byte B of v as a float. Written as uint -> float of (v >> 8B) & 0xFF, which
// the backend selects as one v_cvt_f32_ubyte<B>.
template <int B>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
  return static_cast<float>((v >> (8 * B)) & 0xFFu);
}

// Nibble pair b (columns 2b, 2b + 1) of a packed dword as one bf16 pair,
// exact: with u = nibble ^ 8 (the two's complement value plus 8),
// q * s = fma(float(u), s, -8 s) is exact in f32 (q has 4 bits, s 8), and
// v_cvt_pk_bf16_f32 rounds it once. lo / hi are the dword's low / high
// nibbles after the xor, one per byte.
template <int B>
__device__ __forceinline__ uint32_t dequant_pair(uint32_t lo, uint32_t hi, float s, float m8s) {
  return pack_bf16x2(__builtin_fmaf(ubyte_f32<B>(lo), s, m8s),
                     __builtin_fmaf(ubyte_f32<B>(hi), s, m8s));
}

// Rounds a and b to the nearest bf16 values (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ void round2(float& a, float& b) {
  const uint32_t p = pack_bf16x2(a, b);
  a = __builtin_bit_cast(float, p << 16);
  b = __builtin_bit_cast(float, p & 0xFFFF0000u);
}

// Packed-B rows are 32 bytes per slice; the two 16-byte halves of rows 8..15
// of every 16 swap places so a fragment read (16 lanes on 16 rows, one half)
// is conflict-free.
__device__ __forceinline__ int pswz(int row) { return (row >> 3) & 1; }

// B operand forms of k_gemm_nt.
constexpr int kBBf16 = 0;   // bf16 rows [N, K]
constexpr int kBInt4 = 1;   // packed INT4 rows [N, K / 2] (the forward)
constexpr int kBInt4T = 2;  // packed INT4 [K, N / 2], B[n, k] = W_b[k, n] (dx)
constexpr int kBInt4L = 3;  // packed INT4 rows [N, K / 2], dequantized once per workgroup
                            // into a bf16 slice buffer in LDS (the forward, 256-row tiles)

// One direct-to-LDS load of 16 bytes per lane: lane l writes dst + 16 l.
// (A device function: the LDS address-space cast must stay out of code the
// host pass also parses, such as lambdas in a kernel body.)
__device__ __forceinline__ void dma16(const uint8_t* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<lds_void_t*>(reinterpret_cast<uintptr_t>(dst)),
                                   16, 0, 0);
}

// One direct-to-LDS load of 4 bytes per lane: lane l writes dst + 4 l.
__device__ __forceinline__ void dma_dword(uint8_t* dst, const uint8_t* src) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<lds_void_t*>(reinterpret_cast<uintptr_t>(dst)),
                                   4, 0, 0);
}

// s_waitcnt as an instruction the compiler's own wait insertion accounts
// for (an inline-asm wait is opaque to it): at most VM vector-memory
// operations pending, LGKM LDS operations (15: no wait on them).
template <int VM, int LGKM>
__device__ __forceinline__ void waitcnt() {
  static_assert(VM >= 0 && VM < 64 && LGKM >= 0 && LGKM < 16, "waitcnt range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (LGKM << 8));
  asm volatile("" ::: "memory");
}

// waitcnt<N, 0>, then the workgroup barrier (memory clobber: no memory
// access moves across it).
template <int N>
__device__ __forceinline__ void wait_sync_c() {
  waitcnt<N, 0>();
  asm volatile("s_barrier" ::: "memory");
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// kBInt4T's bf16 slice buffer: 64 rows (k) of BN columns (n), 16-bit
// elements, rows of 2 BN bytes whose 64-byte blocks are XOR-swizzled by the
// row's low two bits, so the four rows of a transposing read (64 contiguous
// bytes each for a 32-lane half) fall on distinct banks.
__device__ __forceinline__ int t4_off(int row, int byte) { return row * 256 + (byte ^ ((row & 3) << 6)); }

template <int BM, int BN, int WM, int WN, int NS, int WPE, int BK, int JB, int ACT>
__global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
    k_gemm_nt(const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ B,
              int64_t ldb, Int4Operand w, int group_shift, int64_t M, int64_t N, int64_t K,
              uint16_t* __restrict__ out, int64_t ldc, LowRankEpilogue epi, int tiles_m,
              int tiles_n, int band) {
  constexpr bool INT4 = BK == kBInt4;
  constexpr bool T4 = BK == kBInt4T;
  constexpr bool I4L = BK == kBInt4L;
  constexpr int NW = WM * WN;
  constexpr int NT = 64 * NW;
  constexpr int TM = BM / WM;
  constexpr int TN = BN / WN;
  constexpr int FM = TM / 32;
  constexpr int FN = TN / 32;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be made of 32x32 blocks");
  constexpr int A_BYTES = BM * 128;
  constexpr int B_ROW = INT4 ? 32 : 128;
  // kBInt4T: the stages hold A only; packed slices (64 rows of BN / 2 bytes)
  // and their scales (one dword per row) rotate through NS + 1 stages of
  // their own, one slice ahead of A, and two bf16 slice buffers follow
  // kBInt4L: the stages hold A only; two bf16 B slice buffers (BN rows of
  // 128 bytes, swizzled like the A rows) follow them
  constexpr int STAGE = (T4 || I4L) ? A_BYTES : A_BYTES + BN * B_ROW;
  constexpr int P_BYTES = T4 ? 64 * (BN / 2) : 0;
  constexpr int P_SEGS = P_BYTES / 1024;
  constexpr int A_SEGS = BM / 8;
  // kBInt4T slots: A segments, packed segments, then the scale load (slots
  // past it repeat the scale load, which rewrites the same bytes)
  constexpr int SEGS = T4 ? A_SEGS + P_SEGS + 1 : (I4L ? A_SEGS : A_SEGS + BN * B_ROW / 1024);
  static_assert(T4 || ((BN * B_ROW) % 1024 == 0 && SEGS % NW == 0), "DMA segments must split evenly");
  static_assert(!T4 || (BN == 128 && BM % 64 == 0), "kBInt4T: 128-column tiles");
  static_assert(!I4L || (NS == 3 && (BN * 8) % NT == 0 && A_SEGS % NW == 0),
                "kBInt4L: three stages, whole packed dwords and A segments per thread");
  // LDS the epilogue may stage the output tile in
  constexpr int LDS_ALL = I4L ? NS * STAGE + 2 * BN * 128 : NS * STAGE;
  constexpr int LPW = (SEGS + NW - 1) / NW;
  static_assert(NS >= 2 && NS <= 4 && LPW * NS < 64, "vmcnt range");
  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* const t4_p = smem + NS * STAGE;             // packed stages
  uint8_t* const t4_s = t4_p + (NS + 1) * P_BYTES;     // scale stages, 256 bytes each
  uint8_t* const t4_b = t4_s + (NS + 1) * 256;         // two bf16 slices of 64 x 256 bytes

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM;
  const int wn = wave / WM;
  int tile_m, tile_n;
  band_tile(xcd_block(blockIdx.x, static_cast<int>(gridDim.x)), tiles_m, tiles_n, band, tile_m,
            tile_n);
  const int64_t m0 = static_cast<int64_t>(tile_m) * BM;
  const int64_t n0 = static_cast<int64_t>(tile_n) * BN;
  const int nk = static_cast<int>(K / kBK);
  const int half = lane >> 5;
  const int frow = lane & 31;

  // INT4 scales of this block's B rows for every group, copied to LDS after
  // the stages ([row][group], 16-byte vectors); the first chunk's loads go
  // out before the prologue DMA and its LDS stores after it.
  constexpr int SC_CAP = INT4 ? 8 : 1;
  uint16_t* sc = reinterpret_cast<uint16_t*>(smem + NS * STAGE);
  const int ng = INT4 ? static_cast<int>(w.n_groups) : 0;
  const int sc_total = INT4 ? static_cast<int>(((N - n0) < BN ? (N - n0) : BN) * ng) : 0;
  const int sc_vecs = sc_total / 8;
  const u32x4_t* sc_src = reinterpret_cast<const u32x4_t*>(INT4 ? w.scales + n0 * ng : nullptr);
  u32x4_t sc_reg[SC_CAP];
  if constexpr (INT4) {
#pragma unroll
    for (int c = 0; c < SC_CAP; ++c) {
      const int v = tid + c * NT;
      if (v < sc_vecs) sc_reg[c] = sc_src[v];
    }
  }

  // DMA sources. Segment j = wave + i * NW: A rows 8j..8j+7 (128 B each), or
  // B rows (8 per segment of bf16 rows, 32 per segment of packed rows). Rows
  // past the edge re-read the last row.
  const uint8_t* src[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int j = wave + i * NW;
    if (j < A_SEGS) {
      const int trow = 8 * j + (lane >> 3);
      int64_t r = m0 + trow;
      r = r < M ? r : M - 1;
      src[i] = reinterpret_cast<const uint8_t*>(A + r * lda) + (((lane & 7) ^ swz(trow)) << 4);
    } else if constexpr (T4) {
      if (j < A_SEGS + P_SEGS) {
        // packed rows 16 p + lane / 4 of the slice, 16 bytes each of the
        // tile's BN / 2
        const int trow = 16 * (j - A_SEGS) + (lane >> 2);
        src[i] = w.packed + trow * w.packed_cols + n0 / 2 + ((lane & 3) << 4);
      } else if (w.n_groups == 1) {
        // per-row scales: lane l loads the dword holding rows l & ~1, l | 1
        src[i] = reinterpret_cast<const uint8_t*>(w.scales + (lane & ~1));
      } else {
        // 64-column groups: lane l loads row l's two groups of the tile
        src[i] = reinterpret_cast<const uint8_t*>(w.scales + lane * w.n_groups + n0 / 64);
      }
    } else if constexpr (INT4) {
      const int trow = 32 * (j - A_SEGS) + (lane >> 1);
      int64_t r = n0 + trow;
      r = r < N ? r : N - 1;
      src[i] = w.packed + r * w.packed_cols + (((lane & 1) ^ pswz(trow)) << 4);
    } else {
      const int trow = 8 * (j - A_SEGS) + (lane >> 3);
      int64_t r = n0 + trow;
      r = r < N ? r : N - 1;
      src[i] = reinterpret_cast<const uint8_t*>(B + r * ldb) + (((lane & 7) ^ swz(trow)) << 4);
    }
  }
  // byte offset of slice s in the source rows
  auto koff = [&](int s, int i) -> int64_t {
    const int j = wave + i * NW;
    if constexpr (T4) {
      if (j >= A_SEGS + P_SEGS) return static_cast<int64_t>(s) * kBK * w.n_groups * 2;
      if (j >= A_SEGS) return static_cast<int64_t>(s) * kBK * w.packed_cols;
    }
    return (INT4 && j >= A_SEGS) ? static_cast<int64_t>(s) * (kBK / 2)
                                 : static_cast<int64_t>(s) * (kBK * 2);
  };
  // kBInt4T: slot i's load of A slice `as` into A stage `ast`, or of packed
  // (or scale) slice `ps` into stage `pst` of its own
  auto dma_t4 = [&](int i, int ast, int as, int pst, int ps) {
    const int j = wave + i * NW;
    if (j < A_SEGS)
      dma_seg(smem + ast * STAGE, src[i], koff(as, i), j);
    else if (j < A_SEGS + P_SEGS)
      dma_seg(t4_p + pst * P_BYTES, src[i], koff(ps, i), j - A_SEGS);
    else
      dma_dword(t4_s + pst * 256, src[i] + koff(ps, i));
  };

  f32x16_t acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[fn][fm][v] = 0.0f;

  // Fragments, double-buffered by 16-deep step: a[kk & 1][fm], b[kk & 1][fn]
  // for bf16 B; for INT4 B the packed bytes of the whole slice (bp, one
  // 16-byte read per fragment) are dequantized unit by unit into bq[kk].
  bf16x8_t af[2][FM];
  bf16x8_t bfr[2][FN];
  u32x4_t bp[FN];
  float bs[FN];
  uint32_t bq[4][FN][4];
  auto read_a = [&](const uint8_t* st, int kk, int buf) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
      af[buf][fm] = as_bf16x8(lds_chunk(st, wm * TM + fm * 32 + frow, 4 * half + kk));
  };
  auto read_b = [&](const uint8_t* st, int kk, int buf) {
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
      bfr[buf][fn] = as_bf16x8(lds_chunk(st + A_BYTES, wn * TN + fn * 32 + frow, 4 * half + kk));
  };
  // kBInt4T: B fragments of step kk from a bf16 slice buffer through
  // transposing reads. Lane l needs B[n][k] for its row n = l % 32 of the
  // 32-column block and the 8 k of step kk in its half (32 half + 8 kk +
  // [0, 8), the order A uses); ds_read_b64_tr_b16 hands lane i of a 16-lane
  // group element i % 4 of the 8-byte pieces that lanes 4 e + i / 4 address,
  // so lane j addresses row 8 kk + 32 half + j / 4 (then + 4) at columns
  // 4 (j % 4) of its 16-column half, and lane i receives 4 consecutive k of
  // column i.
  auto read_bt = [&](const uint8_t* bt, int kk, int buf) {
    const int j = lane & 15;
    const int row = 32 * half + 8 * kk + (j >> 2);
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int col = wn * TN + fn * 32 + 16 * ((lane >> 4) & 1) + 4 * (j & 3);
      const i16x4_t lo =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(bt + t4_off(row, 2 * col)));
      const i16x4_t hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(bt + t4_off(row + 4, 2 * col)));
      bfr[buf][fn] =
          __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };
  // kBInt4T dequantization of a packed slice into a bf16 slice buffer, once
  // per workgroup: item q = tid + it * NT is packed row q / 8 of the slice
  // and its 16 columns 16 (q % 8). t4_read loads every item's 8 packed bytes
  // and scale, t4_pair(u) turns column pair u % 8 of item u / 8 into bf16,
  // t4_write stores the items' 32-byte row pieces (odd rows write their
  // second 16 bytes first, which spreads a 16-lane store over all banks).
  constexpr int T4_IPT = T4 ? 64 * (BN / 16) / NT : 1;
  static_assert(!T4 || (64 * (BN / 16)) % NT == 0, "kBInt4T items must split evenly");
  uint32_t t4_raw[T4_IPT][2];
  float t4_sc[T4_IPT];
  uint32_t t4_out[T4_IPT][8];
  auto t4_read = [&](int pst) {
#pragma unroll
    for (int it = 0; it < T4_IPT; ++it) {
      const int q = tid + it * NT;
      const int r = q >> 3;
      const int c = (q & 7) * 16;
      const u32x2_t v = *reinterpret_cast<const u32x2_t*>(t4_p + pst * P_BYTES + r * (BN / 2) + c / 2);
      t4_raw[it][0] = v[0];
      t4_raw[it][1] = v[1];
      const uint16_t* s16 = reinterpret_cast<const uint16_t*>(t4_s + pst * 256);
      t4_sc[it] = bf16_to_f32(s16[2 * r + (w.n_groups == 1 ? (r & 1) : (c >> 6))]);
    }
  };
  auto t4_pair = [&](int u) {
    const int it = u / 8;
    const int pr = u % 8;
    const uint32_t x = t4_raw[it][pr / 4] ^ 0x88888888u;
    uint32_t lo = x & 0x0F0F0F0Fu;
    uint32_t hi = (x >> 4) & 0x0F0F0F0Fu;
    asm("" : "+v"(lo), "+v"(hi));
    const float sv = t4_sc[it];
    const float m8s = -8.0f * sv;
    uint32_t r;
    switch (pr % 4) {
      case 0: r = dequant_pair<0>(lo, hi, sv, m8s); break;
      case 1: r = dequant_pair<1>(lo, hi, sv, m8s); break;
      case 2: r = dequant_pair<2>(lo, hi, sv, m8s); break;
      default: r = dequant_pair<3>(lo, hi, sv, m8s); break;
    }
    t4_out[it][pr] = r;
  };
  auto t4_write = [&](int bi) {
    uint8_t* bt = t4_b + bi * (64 * 256);
#pragma unroll
    for (int it = 0; it < T4_IPT; ++it) {
      const int q = tid + it * NT;
      const int r = q >> 3;
      const int c = (q & 7) * 16;
      const u32x4_t lo4{t4_out[it][0], t4_out[it][1], t4_out[it][2], t4_out[it][3]};
      const u32x4_t hi4{t4_out[it][4], t4_out[it][5], t4_out[it][6], t4_out[it][7]};
      const bool odd = (r & 1) != 0;
      *reinterpret_cast<u32x4_t*>(bt + t4_off(r, 2 * c + (odd ? 16 : 0))) = odd ? hi4 : lo4;
      *reinterpret_cast<u32x4_t*>(bt + t4_off(r, 2 * c + (odd ? 0 : 16))) = odd ? lo4 : hi4;
    }
  };
  // slot gs (0 .. 3 NS1 - 1) of steps 0-2: the next slice's dequantization,
  // read first, pairs spread over the middle slots, stores last
  auto t4_slot = [&](int gs, int pst, int bi) {
    constexpr int SL = 3 * FM * FN;
    constexpr int U = 8 * T4_IPT;
    constexpr int F = SL >= 4 ? 2 : 1;
    if (gs == 0) t4_read(pst);
    if (gs >= F && gs < SL - 1) {
#pragma unroll
      for (int u = (gs - F) * U / (SL - 1 - F); u < (gs - F + 1) * U / (SL - 1 - F); ++u) t4_pair(u);
    }
    if (gs == SL - 1) t4_write(bi);
  };
  auto read_bp = [&](const uint8_t* st) {
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int r = wn * TN + fn * 32 + frow;
      bp[fn] = *reinterpret_cast<const u32x4_t*>(st + A_BYTES + r * 32 + ((half ^ pswz(r)) << 4));
    }
  };
  auto read_bs = [&](int s) {
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int r = wn * TN + fn * 32 + frow;
      const int g = ng == 1 ? 0 : ((s * kBK + 32 * half) >> group_shift);
      bs[fn] = bf16_to_f32(sc[r * ng + g]);
    }
  };
  // unit u (0 .. 4 FN - 1) of step kk: fragment u / 4, bf16 pair u % 4
  auto dq_unit = [&](int kk, int u) {
    const int fn = u / 4;
    const uint32_t x = bp[fn][kk] ^ 0x88888888u;
    uint32_t lo = x & 0x0F0F0F0Fu;
    uint32_t hi = (x >> 4) & 0x0F0F0F0Fu;
    // opaque to the optimizer: keeps the per-byte conversions from being
    // narrowed to bit-field extracts (one instruction instead of two)
    asm("" : "+v"(lo), "+v"(hi));
    const float m8s = -8.0f * bs[fn];
    uint32_t r;
    switch (u % 4) {
      case 0: r = dequant_pair<0>(lo, hi, bs[fn], m8s); break;
      case 1: r = dequant_pair<1>(lo, hi, bs[fn], m8s); break;
      case 2: r = dequant_pair<2>(lo, hi, bs[fn], m8s); break;
      default: r = dequant_pair<3>(lo, hi, bs[fn], m8s); break;
    }
    bq[kk][fn][u % 4] = r;
  };
  auto mma = [&](int i, int kk) {
    const int fn = i / FM;
    const int fm = i % FM;
    bf16x8_t bv;
    if constexpr (INT4)
      bv = as_bf16x8(u32x4_t{bq[kk][fn][0], bq[kk][fn][1], bq[kk][fn][2], bq[kk][fn][3]});
    else
      bv = bfr[kk & 1][fn];
    acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bv, af[kk & 1][fm], acc[fn][fm], 0, 0, 0);
  };

  // prologue: NS slices in flight (refills past the end re-read the last
  // slice into a stage nothing reads again: LPW loads per slice always);
  // kBInt4L has its own, with its main loop below
  if constexpr (I4L) {
  } else if constexpr (T4) {
    // packed slice 0 and its scales first, then A slice s with packed
    // slice s + 1 (the loop's grouping); vmcnt counts the groups from the
    // newest, so the extra first load needs no count of its own
#pragma unroll
    for (int i = 0; i < LPW; ++i)
      if (wave + i * NW >= A_SEGS) dma_t4(i, 0, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int i = 0; i < LPW; ++i)
        dma_t4(i, s, s < nk ? s : nk - 1, (s + 1) % (NS + 1), s + 1 < nk ? s + 1 : nk - 1);
  } else {
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int i = 0; i < LPW; ++i)
        dma_seg(smem + s * STAGE, src[i], koff(s < nk ? s : nk - 1, i), wave + i * NW);
  }
  if constexpr (INT4) {
#pragma unroll
    for (int c = 0; c < SC_CAP; ++c) {
      const int v = tid + c * NT;
      if (v < sc_vecs) reinterpret_cast<u32x4_t*>(sc)[v] = sc_reg[c];
    }
    for (int v = tid + SC_CAP * NT; v < sc_vecs; v += NT)
      reinterpret_cast<u32x4_t*>(sc)[v] = sc_src[v];
    for (int i = 8 * sc_vecs + tid; i < sc_total; i += NT) sc[i] = w.scales[n0 * ng + i];
  }
  if constexpr (!I4L) wait_sync<(NS - 1) * LPW>();
  if constexpr (T4) {
    // slice 0 dequantized before the loop, visible to every wave
    t4_read(0);
#pragma unroll
    for (int u = 0; u < 8 * T4_IPT; ++u) t4_pair(u);
    t4_write(0);
    wait_sync<(NS - 1) * LPW>();
  }
  if constexpr (!I4L) read_a(smem, 0, 0);
  if constexpr (I4L) {
  } else if constexpr (T4) {
    read_bt(t4_b, 0, 0);
  } else if constexpr (INT4) {
    read_bp(smem);
    read_bs(0);
#pragma unroll
    for (int u = 0; u < 4 * FN; ++u) dq_unit(0, u);
  } else {
    read_b(smem, 0, 0);
  }

  // Main loop, one 16-deep step at a time. Slice t lives in stage t % NS.
  // Each step issues its FM x FN MFMAs, each followed by its share of the
  // step-ahead work: the DS reads of the next step's fragments and, for
  // INT4, the dequantization of the next step's B (one unit per slot). The
  // barrier sits before step 3 (steps 0-3 of the slice have been read by
  // then, slice t + 1 has landed and stage t is free); step 3 then also
  // carries the DMA of slice t + NS into stage t and the reads of slice
  // t + 1's packed rows, scales and step-0 fragments. sched_barrier fences
  // keep the order.
  constexpr int NS1 = FM * FN;  // MFMA slots per step
  constexpr int NU = 4 * FN;    // dequantization units per step
  // Activation operands ([M, N], the output's row stride) for the backward
  // epilogues of the bf16 (dx) tiles, loaded as 16-byte row segments (segment
  // idx = it * NT + tid of the tile) before the last K slice so that their
  // latency overlaps it; that slice runs outside the loop so the loop itself
  // does not carry their registers.
  constexpr bool AUX_OPS = ACT != kActNone && ACT != kActGeluFwd;
  constexpr bool TWO_OPS = ACT == kActSiluMulBwd;
  constexpr bool PREFETCH = AUX_OPS && !INT4 && !I4L;
  constexpr int SEG_ROW = BN / 8;  // 8-column segments per tile row
  constexpr int SEG_ITS = BM * SEG_ROW / NT;
  static_assert(ACT == kActNone || (BM * SEG_ROW) % NT == 0,
                "tile segments must split evenly over the threads");
  const uintptr_t act_ptrs = reinterpret_cast<uintptr_t>(out) |
                             reinterpret_cast<uintptr_t>(epi.aux) |
                             reinterpret_cast<uintptr_t>(epi.aux2) |
                             reinterpret_cast<uintptr_t>(epi.pre_out) |
                             reinterpret_cast<uintptr_t>(epi.out2);
  const bool act_vec = ACT != kActNone && m0 + BM <= M && n0 + BN <= N && (ldc & 7) == 0 &&
                       (act_ptrs & 15) == 0;
  u32x4_t av[AUX_OPS ? SEG_ITS : 1], a2v[TWO_OPS ? SEG_ITS : 1];
  auto load_aux = [&]() {
#pragma unroll
    for (int it = 0; it < SEG_ITS; ++it) {
      const int idx = it * NT + tid;
      const int64_t off = (m0 + idx / SEG_ROW) * ldc + n0 + 8 * (idx % SEG_ROW);
      if constexpr (AUX_OPS) av[it] = *reinterpret_cast<const u32x4_t*>(epi.aux + off);
      if constexpr (TWO_OPS) a2v[it] = *reinterpret_cast<const u32x4_t*>(epi.aux2 + off);
    }
  };

  int stage = 0;
  if constexpr (I4L) {
    // Packed B through registers, dequantized once per workgroup. Thread
    // tid owns dword d = tid % 8 of a slice's 32 packed bytes (k = 8 d ..
    // 8 d + 7) in rows tid / 8 + i (NT / 8), i < PD; each dword becomes one
    // 16-byte chunk of its row in a bf16 slice buffer, with the swizzle of
    // the A rows, from which the B fragments are read as in the bf16 form.
    //
    // Slice t: A[t] in stage t % 3, its B in buffer t & 1. Packed slice t + 1
    // (register set (t + 1) & 1) is dequantized into buffer (t + 1) & 1
    // during step 3 of slice t - 1 and steps 0-2 of slice t, one unit (a
    // bf16 pair) per two MFMA slots. The barrier before step 3 then hands
    // over A[t + 1] and buffer (t + 1) & 1; step 3 waits for packed slice
    // t + 2, issues packed slice t + 3 (registers) and A[t + 3] (into stage
    // t % 3, free after the barrier), starts dequantizing slice t + 2 into
    // buffer t & 1 (free as well) and reads the step-0 fragments of slice
    // t + 1. Per thread and slice: E = 2 PD loads of packed dwords and
    // scales, then LPW A segments, in that order, so vmcnt counts groups.
    constexpr int PD = BN * 8 / NT;
    constexpr int U = 4 * PD;        // dequantization units per slice
    constexpr int SLOTS = 4 * NS1;   // MFMA slots they spread over
    constexpr int E = 2 * PD;
    constexpr int LA = LPW;
    constexpr int BQ = BN * 128;     // bytes of one bf16 slice buffer
    const int ngq = static_cast<int>(w.n_groups);
    const int pdw = tid & 7;
    // Loop-invariant per-lane offsets; the per-slice advance of every global
    // address is uniform (a scalar base), and every LDS address is a
    // per-lane offset plus a compile-time stage or buffer base (the slice
    // loop is unrolled over the 3 A stages x 2 buffer parities), so the loop
    // spends no vector instructions on addresses. The host keeps A and the
    // packed weight under 4 GB for the 32-bit offsets.
    uint32_t poff[PD], soff[PD], qoff[PD];
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      const int lr = (tid >> 3) + i * (NT / 8);
      int64_t r = n0 + lr;
      r = r < N ? r : N - 1;
      poff[i] = static_cast<uint32_t>(r * w.packed_cols + 4 * pdw);
      soff[i] = static_cast<uint32_t>(r * ngq + (ngq == 1 ? 0 : ((8 * pdw) >> group_shift)));
      qoff[i] = static_cast<uint32_t>(lr * 128 + ((pdw ^ swz(lr)) << 4));
    }
    uint32_t aoff[LA];
#pragma unroll
    for (int d = 0; d < LA; ++d) {
      const int trow = 8 * (wave + d * NW) + (lane >> 3);
      int64_t r = m0 + trow;
      r = r < M ? r : M - 1;
      aoff[d] = static_cast<uint32_t>(r * lda * 2 + (((lane & 7) ^ swz(trow)) << 4));
    }
    uint32_t a_off[FM][4], b_off[FN][4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int row = wm * TM + fm * 32 + frow;
        a_off[fm][kk] = row * 128 + (((4 * half + kk) ^ swz(row)) << 4);
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int row = wn * TN + fn * 32 + frow;
        b_off[fn][kk] = NS * STAGE + row * 128 + (((4 * half + kk) ^ swz(row)) << 4);
      }
    }
    uint32_t pk[2][PD], ps[2][PD];
    auto p_load = [&](auto set_c, int s) {
      constexpr int set = decltype(set_c)::value;
      const int sl = s < nk ? s : nk - 1;
      const uint8_t* pb = w.packed + static_cast<int64_t>(sl) * (kBK / 2);
      const uint16_t* sb = w.scales + (ngq == 1 ? 0 : ((sl * kBK) >> group_shift));
#pragma unroll
      for (int i = 0; i < PD; ++i) pk[set][i] = *reinterpret_cast<const uint32_t*>(pb + poff[i]);
#pragma unroll
      for (int i = 0; i < PD; ++i) ps[set][i] = sb[soff[i]];
    };
    uint32_t ulo[PD], uhi[PD], uo[PD][4];
    float us[PD], um[PD];
    // unit u: item u / 4, bf16 pair u % 4 (k = 8 d + 2 (u % 4) + {0, 1});
    // the item's first unit unpacks it
    auto p_unit = [&](auto set_c, int u) {
      constexpr int set = decltype(set_c)::value;
      const int i = u / 4;
      const int pr = u % 4;
      if (pr == 0) {
        const uint32_t x = pk[set][i] ^ 0x88888888u;
        uint32_t lo = x & 0x0F0F0F0Fu;
        uint32_t hi = (x >> 4) & 0x0F0F0F0Fu;
        asm("" : "+v"(lo), "+v"(hi));
        ulo[i] = lo;
        uhi[i] = hi;
        us[i] = __builtin_bit_cast(float, ps[set][i] << 16);
        um[i] = -8.0f * us[i];
      }
      switch (pr) {
        case 0: uo[i][0] = dequant_pair<0>(ulo[i], uhi[i], us[i], um[i]); break;
        case 1: uo[i][1] = dequant_pair<1>(ulo[i], uhi[i], us[i], um[i]); break;
        case 2: uo[i][2] = dequant_pair<2>(ulo[i], uhi[i], us[i], um[i]); break;
        default: uo[i][3] = dequant_pair<3>(ulo[i], uhi[i], us[i], um[i]); break;
      }
    };
    // units of slot g (0 .. SLOTS - 1; slot g of step 3 is g < NS1)
    auto p_units = [&](auto set_c, int g) {
#pragma unroll
      for (int u = g * U / SLOTS; u < (g + 1) * U / SLOTS; ++u) p_unit(set_c, u);
    };
    // The chunk stores of the items finished by the end of step q (0: step 3
    // of the previous slice, 1-3: steps 0-2), issued early in step q + 1 so
    // that no LDS store is in flight at a step boundary (the compiler waits
    // for every LDS operation there); the last ones go out before the barrier.
    auto done_items = [](int q) { return (q + 1) * PD / 4; };
    auto p_store = [&](auto buf_c, int i0, int i1) {
      constexpr int buf = decltype(buf_c)::value;
#pragma unroll
      for (int i = i0; i < i1; ++i)
        *reinterpret_cast<u32x4_t*>(smem + NS * STAGE + buf * BQ + qoff[i]) =
            u32x4_t{uo[i][0], uo[i][1], uo[i][2], uo[i][3]};
    };
    // B fragments double-buffered like A: all of the next step's fragments
    // are read early in the step (at most three 32-column blocks per wave:
    // a fourth would not fit the two-waves-per-SIMD register budget)
    static_assert(FN <= 3, "kBInt4L: at most three B fragments per wave");
    auto read_ac = [&](auto stg_c, int kk) {
      constexpr int stg = decltype(stg_c)::value;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        af[kk & 1][fm] = *reinterpret_cast<const bf16x8_t*>(smem + stg * STAGE + a_off[fm][kk]);
    };
    auto read_bq = [&](auto buf_c, int kk) {
      constexpr int buf = decltype(buf_c)::value;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        bfr[kk & 1][fn] = *reinterpret_cast<const bf16x8_t*>(smem + buf * BQ + b_off[fn][kk]);
    };
    auto mma_l = [&](int i, int kk) {
      const int fn = i / FM;
      const int fm = i % FM;
      acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[kk & 1][fn], af[kk & 1][fm],
                                                            acc[fn][fm], 0, 0, 0);
    };
    // next-step fragment reads in slot i of a step (kk: the next step)
    auto frag_reads = [&](auto stg_c, auto buf_c, int kk, int i) {
      if (i == 0) read_ac(stg_c, kk);
      if (i == 1) read_bq(buf_c, kk);
    };
    // A slice s into stage stg: segments d0 .. d1 - 1 of this wave
    auto dma_a = [&](auto stg_c, int s, int d0, int d1) {
      constexpr int stg = decltype(stg_c)::value;
      const uint8_t* ab = reinterpret_cast<const uint8_t*>(A) +
                          static_cast<int64_t>(s < nk ? s : nk - 1) * (kBK * 2);
#pragma unroll
      for (int d = d0; d < d1; ++d) dma16(ab + aoff[d], smem + stg * STAGE + (wave + d * NW) * 1024);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;

    // prologue: packed slices 0, 1, 2 and A slices 0, 1, 2 in flight;
    // slice 0 dequantized whole, slice 1 its step-3 share
    p_load(I0{}, 0);
    dma_a(I0{}, 0, 0, LA);
    p_load(I1{}, 1);
    dma_a(I1{}, 1, 0, LA);
    waitcnt<LA + E + LA, 15>();
#pragma unroll
    for (int u = 0; u < U; ++u) p_unit(I0{}, u);
    p_store(I0{}, 0, PD);
    p_load(I0{}, 2);
    dma_a(I2{}, 2, 0, LA);
    wait_sync_c<LA + E + LA>();
#pragma unroll
    for (int i = 0; i < NS1; ++i) frag_reads(I0{}, I0{}, 0, i);
#pragma unroll
    for (int g = 0; g < NS1; ++g) p_units(I1{}, g);

    // slice t: A in stage STG = t % 3, B in buffer PAR = t % 2
    auto slice = [&](auto stg_c, auto par_c, int t) {
      constexpr int STG = decltype(stg_c)::value;
      constexpr int PAR = decltype(par_c)::value;
      const std::integral_constant<int, (STG + 1) % 3> nstg{};
      const std::integral_constant<int, 1 - PAR> cur{};  // packed slice t + 1, buffer of t + 1
      const std::integral_constant<int, PAR> nxt{};      // packed slice t + 2, buffer of t
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 3; ++kk) {
#pragma unroll
        for (int i = 0; i < NS1; ++i) {
          mma_l(i, kk);
          __builtin_amdgcn_sched_barrier(0);
          frag_reads(stg_c, par_c, kk + 1, i);
          if (i == 2) p_store(cur, done_items(kk - 1), done_items(kk));
          p_units(cur, NS1 * (kk + 1) + i);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      p_store(cur, done_items(2), PD);
      __builtin_amdgcn_sched_barrier(0);
      wait_sync_c<E + LA>();
#pragma unroll
      for (int i = 0; i < NS1; ++i) {
        mma_l(i, 3);
        __builtin_amdgcn_sched_barrier(0);
        if (i == 0) {
          waitcnt<LA, 15>();
          p_load(cur, t + 3);
        }
        dma_a(stg_c, t + 3, i * LA / NS1, (i + 1) * LA / NS1);
        frag_reads(nstg, cur, 0, i);
        p_units(nxt, i);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    int t = 0;
    for (; t + 6 <= nk; t += 6) {
      slice(I0{}, I0{}, t);
      slice(I1{}, I1{}, t + 1);
      slice(I2{}, I0{}, t + 2);
      slice(I0{}, I1{}, t + 3);
      slice(I1{}, I0{}, t + 4);
      slice(I2{}, I1{}, t + 5);
    }
    if (t < nk) slice(I0{}, I0{}, t);
    if (t + 1 < nk) slice(I1{}, I1{}, t + 1);
    if (t + 2 < nk) slice(I2{}, I0{}, t + 2);
    if (t + 3 < nk) slice(I0{}, I1{}, t + 3);
    if (t + 4 < nk) slice(I1{}, I0{}, t + 4);
  } else if constexpr (PREFETCH) {
    auto slice = [&](int t) {
      const int next = stage + 1 == NS ? 0 : stage + 1;
      const uint8_t* st = smem + stage * STAGE;
      // kBInt4T: bf16 buffers of slices t and t + 1, packed stage of t + 1
      [[maybe_unused]] const uint8_t* bt_cur = t4_b + (t & 1) * (64 * 256);
      [[maybe_unused]] const uint8_t* bt_next = t4_b + ((t + 1) & 1) * (64 * 256);
      [[maybe_unused]] const int p_next = (t + 1) % (NS + 1);
      __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
      for (int kk = 0; kk < 3; ++kk) {
  #pragma unroll
        for (int i = 0; i < NS1; ++i) {
          mma(i, kk);
          __builtin_amdgcn_sched_barrier(0);
          if (i == 0) read_a(st, kk + 1, (kk + 1) & 1);
          if constexpr (INT4) {
  #pragma unroll
            for (int u = i * NU / NS1; u < (i + 1) * NU / NS1; ++u) dq_unit(kk + 1, u);
          } else if constexpr (T4) {
            if (i == NS1 / 2) read_bt(bt_cur, kk + 1, (kk + 1) & 1);
            t4_slot(kk * NS1 + i, p_next, (t + 1) & 1);
          } else {
            if (i == NS1 / 2) read_b(st, kk + 1, (kk + 1) & 1);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      wait_sync<(NS - 2) * LPW>();
      const int refill = t + NS < nk ? t + NS : nk - 1;
      uint8_t* fill = smem + stage * STAGE;
      const uint8_t* nst = smem + next * STAGE;
      // INT4: packed rows and scales first, their units in the last half
      constexpr int U0 = NS1 / 2;
  #pragma unroll
      for (int i = 0; i < NS1; ++i) {
        mma(i, 3);
        __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
        for (int d = i * LPW / NS1; d < (i + 1) * LPW / NS1; ++d)
          if constexpr (T4)
            dma_t4(d, stage, refill, t % (NS + 1), t + NS + 1 < nk ? t + NS + 1 : nk - 1);
          else
            dma_seg(fill, src[d], koff(refill, d), wave + d * NW);
        if constexpr (INT4) {
          if (i == 0) {
            read_bp(nst);
            read_bs(t + 1 < nk ? t + 1 : t);
          }
          if (i == 1) read_a(nst, 0, 0);
          if (i >= U0) {
  #pragma unroll
            for (int u = (i - U0) * NU / (NS1 - U0); u < (i - U0 + 1) * NU / (NS1 - U0); ++u)
              dq_unit(0, u);
          }
        } else {
          if (i == 0) read_a(nst, 0, 0);
          if constexpr (T4) {
            if (i == NS1 / 2) read_bt(bt_next, 0, 0);
          } else {
            if (i == NS1 / 2) read_b(nst, 0, 0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      stage = next;
    };
    for (int t = 0; t + 1 < nk; ++t) slice(t);
    if (act_vec) load_aux();
    slice(nk - 1);
  } else {
    for (int t = 0; t < nk; ++t) {
      const int next = stage + 1 == NS ? 0 : stage + 1;
      const uint8_t* st = smem + stage * STAGE;
      // kBInt4T: bf16 buffers of slices t and t + 1, packed stage of t + 1
      [[maybe_unused]] const uint8_t* bt_cur = t4_b + (t & 1) * (64 * 256);
      [[maybe_unused]] const uint8_t* bt_next = t4_b + ((t + 1) & 1) * (64 * 256);
      [[maybe_unused]] const int p_next = (t + 1) % (NS + 1);
      __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
      for (int kk = 0; kk < 3; ++kk) {
  #pragma unroll
        for (int i = 0; i < NS1; ++i) {
          mma(i, kk);
          __builtin_amdgcn_sched_barrier(0);
          if (i == 0) read_a(st, kk + 1, (kk + 1) & 1);
          if constexpr (INT4) {
  #pragma unroll
            for (int u = i * NU / NS1; u < (i + 1) * NU / NS1; ++u) dq_unit(kk + 1, u);
          } else if constexpr (T4) {
            if (i == NS1 / 2) read_bt(bt_cur, kk + 1, (kk + 1) & 1);
            t4_slot(kk * NS1 + i, p_next, (t + 1) & 1);
          } else {
            if (i == NS1 / 2) read_b(st, kk + 1, (kk + 1) & 1);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      wait_sync<(NS - 2) * LPW>();
      const int refill = t + NS < nk ? t + NS : nk - 1;
      uint8_t* fill = smem + stage * STAGE;
      const uint8_t* nst = smem + next * STAGE;
      // INT4: packed rows and scales first, their units in the last half
      constexpr int U0 = NS1 / 2;
  #pragma unroll
      for (int i = 0; i < NS1; ++i) {
        mma(i, 3);
        __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
        for (int d = i * LPW / NS1; d < (i + 1) * LPW / NS1; ++d)
          if constexpr (T4)
            dma_t4(d, stage, refill, t % (NS + 1), t + NS + 1 < nk ? t + NS + 1 : nk - 1);
          else
            dma_seg(fill, src[d], koff(refill, d), wave + d * NW);
        if constexpr (INT4) {
          if (i == 0) {
            read_bp(nst);
            read_bs(t + 1 < nk ? t + 1 : t);
          }
          if (i == 1) read_a(nst, 0, 0);
          if (i >= U0) {
  #pragma unroll
            for (int u = (i - U0) * NU / (NS1 - U0); u < (i - U0 + 1) * NU / (NS1 - U0); ++u)
              dq_unit(0, u);
          }
        } else {
          if (i == 0) read_a(nst, 0, 0);
          if constexpr (T4) {
            if (i == NS1 / 2) read_bt(bt_next, 0, 0);
          } else {
            if (i == NS1 / 2) read_b(nst, 0, 0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      stage = next;
    }
  }
  // no LDS DMA may still be in flight when the waves leave the loop
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue --------------------------------------------------------------
  // y = bf16(bf16(acc) + bf16(bf16(t) * scale)) (+ bias, rounded again), the
  // reference's rounding points, where t = C R^T is one more 32x32x16 MFMA
  // per 16 ranks. Values are rounded in pairs (one v_cvt_pk_bf16_f32 per
  // two), staged as bf16 in LDS and written as whole row segments of the
  // workgroup tile.
  constexpr int kMaxJB = JB > 0 ? JB : 1;  // ceil(rank / 16), rank <= 16 * JB
  const int jblocks = JB > 0 ? static_cast<int>((epi.rank + 15) / 16) : 0;
  const int64_t mw = m0 + wm * TM;  // first row of this wave's sub-tile
  const int64_t nw = n0 + wn * TN;  // first column
  const bool inside = mw + TM <= M && nw + TN <= N;
  // low-rank operands with unit rank stride, whole 16-rank blocks and
  // 16-byte aligned rows: every fragment is one plain 16-byte load
  const bool lr_vec =
      inside && epi.rows_sj == 1 && epi.cols_sj == 1 && (epi.rank & 15) == 0 &&
      (epi.rows_sn & 7) == 0 && (epi.cols_sm & 7) == 0 &&
      ((reinterpret_cast<uintptr_t>(epi.rows) | reinterpret_cast<uintptr_t>(epi.cols)) & 15) == 0;
  bf16x8_t cf[kMaxJB][FM];
  bf16x8_t rf[kMaxJB][FN];
  if (jblocks > 0) {
#pragma unroll
    for (int jb = 0; jb < kMaxJB; ++jb) {
      if (jb >= jblocks) break;
      const int64_t jl = jb * 16 + half * 8;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int64_t m = mw + fm * 32 + frow;
        cf[jb][fm] = lr_vec ? *reinterpret_cast<const bf16x8_t*>(epi.cols + m * epi.cols_sm + jl)
                            : load8_j(epi.cols + m * epi.cols_sm + jl * epi.cols_sj, epi.cols_sj,
                                      m < M ? valid8(epi.rank, jl) : 0);
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int64_t n = nw + fn * 32 + frow;
        rf[jb][fn] = lr_vec ? *reinterpret_cast<const bf16x8_t*>(epi.rows + n * epi.rows_sn + jl)
                            : load8_j(epi.rows + n * epi.rows_sn + jl * epi.rows_sj, epi.rows_sj,
                                      n < N ? valid8(epi.rank, jl) : 0);
      }
    }
  }
  // bias of this lane's columns nw + 32 fn + 8 vg + 4 half + e
  const bool has_bias = epi.bias != nullptr;
  float bias4[FN][4][4];
  if (has_bias) {
    const bool bvec = inside && (reinterpret_cast<uintptr_t>(epi.bias) & 7) == 0;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        const int64_t nb = nw + fn * 32 + 8 * vg + 4 * half;
        if (bvec) {
          const u32x2_t w2 = *reinterpret_cast<const u32x2_t*>(epi.bias + nb);
          bias4[fn][vg][0] = bf16lo_to_f32(w2[0]);
          bias4[fn][vg][1] = bf16hi_to_f32(w2[0]);
          bias4[fn][vg][2] = bf16lo_to_f32(w2[1]);
          bias4[fn][vg][3] = bf16hi_to_f32(w2[1]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            bias4[fn][vg][e] = nb + e < N ? bf16_to_f32(epi.bias[nb + e]) : 0.0f;
        }
      }
  }
  // bf16(t) * scale is already a bf16 value when scale = 2^k, k >= 0 (the
  // product only shifts the exponent; overflow gives inf either way)
  const uint32_t sbits = __builtin_bit_cast(uint32_t, epi.scale);
  const bool scale_exact = (sbits & 0x807FFFFFu) == 0 && sbits >= 0x3F800000u && sbits < 0x7F800000u;

  uint32_t ypk[FN][FM][8];  // bf16 pairs (columns 8 (v / 4) + 4 half + v % 4, v even)
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      f32x16_t t;
#pragma unroll
      for (int v = 0; v < 16; ++v) t[v] = 0.0f;
#pragma unroll
      for (int jb = 0; jb < kMaxJB; ++jb) {
        if (jb >= jblocks) break;
        t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rf[jb][fn], cf[jb][fm], t, 0, 0, 0);
      }
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        float a0 = acc[fn][fm][v];
        float a1 = acc[fn][fm][v + 1];
        if (jblocks > 0) {
          round2(a0, a1);
          float t0 = t[v];
          float t1 = t[v + 1];
          round2(t0, t1);
          t0 *= epi.scale;
          t1 *= epi.scale;
          if (!scale_exact) round2(t0, t1);
          a0 += t0;
          a1 += t1;
        }
        if (has_bias) {
          round2(a0, a1);
          a0 += bias4[fn][v / 4][v % 4];
          a1 += bias4[fn][v / 4][v % 4 + 1];
        }
        ypk[fn][fm][v / 2] = pack_bf16x2(a0, a1);
      }
    }
  }

  constexpr int P = BN * 2 + 16;  // LDS row pitch of the staged tile
  if constexpr (ACT == kActNone) {
    const bool vec_out = (ldc & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    if constexpr (BM * P <= LDS_ALL) {
      wait_sync<0>();  // every wave is done reading the pipeline stages
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int vg = 0; vg < 4; ++vg) {
            const int ml = wm * TM + fm * 32 + frow;
            const int nl = wn * TN + fn * 32 + 8 * vg + 4 * half;
            *reinterpret_cast<u32x2_t*>(smem + ml * P + nl * 2) =
                u32x2_t{ypk[fn][fm][2 * vg], ypk[fn][fm][2 * vg + 1]};
          }
      __syncthreads();
      constexpr int CPR = BN / 8;  // 16-byte chunks per tile row
      constexpr int ITS = BM * CPR / NT;
      static_assert((BM * CPR) % NT == 0, "tile chunks must split evenly over the threads");
      if (vec_out && m0 + BM <= M && n0 + BN <= N) {
        u32x4_t v[ITS];
#pragma unroll
        for (int it = 0; it < ITS; ++it) {
          const int idx = it * NT + tid;
          v[it] = *reinterpret_cast<const u32x4_t*>(smem + (idx / CPR) * P + (idx % CPR) * 16);
        }
#pragma unroll
        for (int it = 0; it < ITS; ++it) {
          const int idx = it * NT + tid;
          *reinterpret_cast<u32x4_t*>(out + (m0 + idx / CPR) * ldc + n0 + 8 * (idx % CPR)) = v[it];
        }
        return;
      }
      for (int it = 0; it < ITS; ++it) {
        const int idx = it * NT + tid;
        const int64_t m = m0 + idx / CPR;
        const int64_t n = n0 + 8 * (idx % CPR);
        if (m >= M || n >= N) continue;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(smem + (idx / CPR) * P + (idx % CPR) * 16);
        uint16_t* d = out + m * ldc + n;
        if (vec_out && n + 7 < N) {
          *reinterpret_cast<u32x4_t*>(d) = v;
        } else {
          for (int e = 0; e < 8; ++e)
            if (n + e < N) d[e] = static_cast<uint16_t>((v[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
        }
      }
    } else {
      // tile too large to stage in the pipeline's LDS: 8-byte stores per lane
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          const int64_t m = mw + fm * 32 + frow;
          if (m >= M) continue;
#pragma unroll
          for (int vg = 0; vg < 4; ++vg) {
            const int64_t nb = nw + fn * 32 + 8 * vg + 4 * half;
            uint16_t* dst = out + m * ldc + nb;
            if (vec_out && nb + 3 < N) {
              *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{ypk[fn][fm][2 * vg], ypk[fn][fm][2 * vg + 1]};
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (nb + e < N)
                  dst[e] = static_cast<uint16_t>((ypk[fn][fm][2 * vg + e / 2] >> (16 * (e & 1))) & 0xFFFFu);
            }
          }
        }
    }
  } else {
    // Activation epilogue on the rounded outputs v: f32 from bf16 operands,
    // rounded once (act.h). The tile of v is staged in LDS and every thread
    // then transforms whole 8-column row segments, with the auxiliary
    // operands' 16-byte loads issued before the staging. Forward modes also
    // store v itself.
    static_assert(BM * P <= LDS_ALL, "activation epilogues stage the tile in LDS");
    constexpr bool FWD = ACT == kActGeluFwd || ACT == kActSiluMulFwd;
    constexpr bool AUX = AUX_OPS;
    constexpr bool TWO = TWO_OPS;
    constexpr int CPR = SEG_ROW;
    constexpr int ITS = SEG_ITS;
    const bool vec = act_vec;
    if constexpr (AUX && !PREFETCH) {
      if (vec) load_aux();
    }
    wait_sync<0>();  // every wave is done reading the pipeline stages
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int vg = 0; vg < 4; ++vg) {
          const int ml = wm * TM + fm * 32 + frow;
          const int nl = wn * TN + fn * 32 + 8 * vg + 4 * half;
          *reinterpret_cast<u32x2_t*>(smem + ml * P + nl * 2) =
              u32x2_t{ypk[fn][fm][2 * vg], ypk[fn][fm][2 * vg + 1]};
        }
    __syncthreads();
    auto bf16_at = [](const u32x4_t& q, int e) {
      return (e & 1) ? bf16hi_to_f32(q[e >> 1]) : bf16lo_to_f32(q[e >> 1]);
    };
#pragma unroll
    for (int it = 0; it < ITS; ++it) {
      const int idx = it * NT + tid;
      const int64_t m = m0 + idx / CPR;
      const int64_t n = n0 + 8 * (idx % CPR);
      if (m >= M || n >= N) continue;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(smem + (idx / CPR) * P + (idx % CPR) * 16);
      const int64_t off = m * ldc + n;
      float r[8], r2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a0 = 0.0f, a1 = 0.0f;
        if (vec) {
          if constexpr (AUX) a0 = bf16_at(av[it], e);
          if constexpr (TWO) a1 = bf16_at(a2v[it], e);
        } else if (n + e < N) {
          if constexpr (AUX) a0 = bf16_to_f32(epi.aux[off + e]);
          if constexpr (TWO) a1 = bf16_to_f32(epi.aux2[off + e]);
        }
        r[e] = act_apply<ACT>(bf16_at(v, e), a0, a1, &r2[e]);
      }
      const u32x4_t o{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]), pack_bf16x2(r[4], r[5]),
                      pack_bf16x2(r[6], r[7])};
      u32x4_t o2{0u, 0u, 0u, 0u};
      if constexpr (TWO)
        o2 = u32x4_t{pack_bf16x2(r2[0], r2[1]), pack_bf16x2(r2[2], r2[3]),
                     pack_bf16x2(r2[4], r2[5]), pack_bf16x2(r2[6], r2[7])};
      if (vec) {
        *reinterpret_cast<u32x4_t*>(out + off) = o;
        if constexpr (FWD) *reinterpret_cast<u32x4_t*>(epi.pre_out + off) = v;
        if constexpr (TWO) *reinterpret_cast<u32x4_t*>(epi.out2 + off) = o2;
      } else {
        for (int e = 0; e < 8 && n + e < N; ++e) {
          const int sh = 16 * (e & 1);
          out[off + e] = static_cast<uint16_t>((o[e >> 1] >> sh) & 0xFFFFu);
          if constexpr (FWD) epi.pre_out[off + e] = static_cast<uint16_t>((v[e >> 1] >> sh) & 0xFFFFu);
          if constexpr (TWO) epi.out2[off + e] = static_cast<uint16_t>((o2[e >> 1] >> sh) & 0xFFFFu);
        }
      }
    }
  }
}

constexpr int gemm_lds_bytes(int bm, int bn, int ns, bool int4) {
  return ns * (bm * 128 + bn * (int4 ? 32 : 128));
}

// kBInt4T (BN = 128): A stages, NS + 1 packed stages of 4 KB and scale
// stages of 256 bytes, two bf16 slices of 16 KB
constexpr int gemm_lds_bytes_t4(int bm, int ns) {
  return ns * bm * 128 + (ns + 1) * (64 * 64 + 256) + 2 * 64 * 256;
}

// kBInt4L: A stages and two bf16 B slice buffers
constexpr int gemm_lds_bytes_i4l(int bm, int bn, int ns) { return ns * bm * 128 + 2 * bn * 128; }

// The kTuneBand knob's band (at most tiles_m rows) when it is set, else
// `otherwise`.
int forced_band(int tiles_m, int otherwise) {
  const int forced = tune(kTuneBand);
  if (forced <= 0) return otherwise;
  return forced < tiles_m ? forced : (tiles_m > 0 ? tiles_m : 1);
}

// Rows per band of the banded tile order (band_tile). An XCD runs its tiles
// `resident` at a time (32 CUs x workgroups per CU); with b-row bands such a
// set spans about `rows` A row-blocks and `cols` B column-blocks, which it
// streams through the XCD's L2 at rows * a_bytes + cols * b_bytes per unit
// of K (BM or BN rows times the operand's bytes per element). b minimizes
// that (ties keep the smaller b; b = 1 is row-major order). Measured on the
// bf16 input-gradient GEMMs alone (two runs each, alternating): 16384 x 2048
// <- 6144 344-349 -> 319-323 us, 16384 x 6144 <- 2048 395-402 -> 378-382 us,
// 32768 x 3072 <- 768 163-164 -> 154-159 us, while 768-wide outputs, whose
// row-major sets already span ~10 row blocks, are unchanged. The kTuneBand
// knob forces a band.
int gemm_band(int tiles_m, int tiles_n, int64_t resident, int64_t a_bytes, int64_t b_bytes) {
  if (tune(kTuneBand) > 0) return forced_band(tiles_m, 1);
  const int64_t per_xcd = ceil_div(static_cast<int64_t>(tiles_m) * tiles_n, 8);
  const int64_t t = resident < per_xcd ? resident : per_xcd;
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
    const int64_t cost = rows * a_bytes + cols * b_bytes;
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = b;
    }
  }
  return best;
}

template <int BM, int BN, int WM, int WN, int NS, int WPE, int BK, int JB, int ACT>
hipError_t run_gemm_act(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                        const Int4Operand& w, int64_t m, int64_t n, int64_t k, uint16_t* out,
                        int64_t ldc, const LowRankEpilogue& epi, hipStream_t stream) {
  constexpr bool INT4 = BK == kBInt4;
  constexpr bool T4 = BK == kBInt4T;
  constexpr bool I4L = BK == kBInt4L;
  const int tiles_m = static_cast<int>(ceil_div(m, BM));
  const int tiles_n = static_cast<int>(ceil_div(n, BN));
  const size_t scale_bytes = INT4 ? static_cast<size_t>(BN) * w.n_groups * 2 : 0;
  const size_t lds = T4    ? static_cast<size_t>(gemm_lds_bytes_t4(BM, NS))
                     : I4L ? static_cast<size_t>(gemm_lds_bytes_i4l(BM, BN, NS))
                           : gemm_lds_bytes(BM, BN, NS, INT4) + ((scale_bytes + 15) & ~size_t{15});
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  auto kern = k_gemm_nt<BM, BN, WM, WN, NS, WPE, BK, JB, ACT>;
  static std::atomic<unsigned> lds_set{0};
  hipError_t e = ensure_lds_limit(reinterpret_cast<const void*>(kern), 160 * 1024, lds_set);
  if (e != hipSuccess) return e;
  int group_shift = 0;
  if ((INT4 || I4L) && w.n_groups > 1) {
    while ((int64_t{1} << group_shift) < w.group) ++group_shift;
  }
  // workgroups per CU: waves per SIMD (WPE) x 4 SIMDs over the block's
  // waves, or fewer when LDS runs out
  int64_t per_cu = (4 * WPE) / (WM * WN);
  if (per_cu * static_cast<int64_t>(lds) > 160 * 1024) per_cu = (160 * 1024) / static_cast<int64_t>(lds);
  if (per_cu < 1) per_cu = 1;
  // bf16 operands on both sides. The INT4 GEMMs keep row-major order (a
  // forced band aside): their packed B is a quarter of the bytes, and bands
  // measured within run-to-run noise of row-major on every train-step shape.
  const int band = INT4 || T4 || I4L ? forced_band(tiles_m, 1)
                        : gemm_band(tiles_m, tiles_n, 32 * per_cu, int64_t{2} * BM,
                                    int64_t{2} * BN);
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles_m) * tiles_n), dim3(64 * WM * WN),
                     lds, stream, a, lda, b, ldb, w, group_shift, m, n, k, out, ldc, epi, tiles_m,
                     tiles_n, band);
  return hipGetLastError();
}

// Activation epilogues: the forward modes on the INT4 GEMM (the FFN's up
// projection), the backward modes on the bf16 dx GEMM (the down projection's
// input gradient), for the default tile shapes.
template <int BM, int BN, int WM, int WN, int NS, int WPE, int BK, int JB>
hipError_t run_gemm_jb(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                       const Int4Operand& w, int64_t m, int64_t n, int64_t k, uint16_t* out,
                       int64_t ldc, const LowRankEpilogue& epi, hipStream_t stream) {
#define RPX_RUN_ACT(ACT) \
  run_gemm_act<BM, BN, WM, WN, NS, WPE, BK, JB, ACT>(a, lda, b, ldb, w, m, n, k, out, ldc, epi, stream)
  if (epi.act == kActNone) return RPX_RUN_ACT(kActNone);
  if constexpr (JB > 0 && !(BM == 256 && BN == 256)) {
    if constexpr (BK == kBInt4 || BK == kBInt4L) {
      if (epi.act == kActGeluFwd) return RPX_RUN_ACT(kActGeluFwd);
      if (epi.act == kActSiluMulFwd) return RPX_RUN_ACT(kActSiluMulFwd);
    } else {
      if (epi.act == kActGeluBwd) return RPX_RUN_ACT(kActGeluBwd);
      if (epi.act == kActSiluMulBwd) return RPX_RUN_ACT(kActSiluMulBwd);
      if (epi.act == kActAddBwd) return RPX_RUN_ACT(kActAddBwd);
    }
  }
#undef RPX_RUN_ACT
  return hipErrorInvalidValue;
}

template <int BM, int BN, int WM, int WN, int NS, int WPE, int BK>
hipError_t run_gemm(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                    const Int4Operand& w, int64_t m, int64_t n, int64_t k, uint16_t* out,
                    int64_t ldc, const LowRankEpilogue& epi, hipStream_t stream) {
  if (epi.rank <= 0)
    return run_gemm_jb<BM, BN, WM, WN, NS, WPE, BK, 0>(a, lda, b, ldb, w, m, n, k, out, ldc,
                                                         epi, stream);
  if (epi.rank <= 16)
    return run_gemm_jb<BM, BN, WM, WN, NS, WPE, BK, 1>(a, lda, b, ldb, w, m, n, k, out, ldc,
                                                         epi, stream);
  if (epi.rank <= 32)
    return run_gemm_jb<BM, BN, WM, WN, NS, WPE, BK, 2>(a, lda, b, ldb, w, m, n, k, out, ldc,
                                                         epi, stream);
  return run_gemm_jb<BM, BN, WM, WN, NS, WPE, BK, 4>(a, lda, b, ldb, w, m, n, k, out, ldc, epi,
                                                       stream);
}

// INT4 B: one wave row (WM = 1) so every packed row is dequantized by a
// single wave. bf16 B: 2 x 2 or 4 x 2 waves.
hipError_t dispatch_int4(const uint16_t* a, int64_t lda, const Int4Operand& w, int64_t m,
                         int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                         const LowRankEpilogue& epi, hipStream_t stream) {
  // scales are copied in 16-byte vectors from a 16-byte aligned base, and the
  // packed rows are read in 16-byte chunks
  if ((reinterpret_cast<uintptr_t>(w.scales) & 15) != 0 || (w.packed_cols & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(w.packed) & 15) != 0)
    return hipErrorInvalidValue;
  int cfg = tune(kTuneInt4Tile);
  // kBInt4L addresses A and the packed weight with 32-bit per-lane offsets
  const bool i4l_ok = m * lda * 2 < (int64_t{1} << 32) && n * w.packed_cols < (int64_t{1} << 32);
  if (cfg == kTileI4L_256x192 && i4l_ok)
    return run_gemm<256, 192, 4, 2, 3, 2, kBInt4L>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                   stream);
  if (cfg == kTileI4_256x256)
    return run_gemm<256, 256, 2, 2, 3, 1, kBInt4>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                stream);
  if (cfg == kTileI4_128x128s2)
    return run_gemm<128, 128, 1, 4, 2, 3, kBInt4>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                stream);
  if (cfg == kTileI4_128x128s3)
    return run_gemm<128, 128, 1, 4, 3, 2, kBInt4>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                stream);
  if (cfg == kTileI4_256x128s2)
    return run_gemm<256, 128, 1, 4, 2, 2, kBInt4>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                stream);
  if (cfg < kTileI4_256x128 || cfg > kTileI4_64x128) {
    // Long reductions over outputs that split into whole 192-column tiles,
    // at least one round of them: the 256 x 192 tile that dequantizes each
    // packed element once per 256 rows into LDS (BERT FFN down, 32768 x 768
    // <- 3072: 195 against 214 us). The K = 768 products, ragged column
    // tiles and the Qwen3-2B shapes measured as fast or faster on the
    // 128-row tiles below.
    if (i4l_ok && k >= 3072 && n % 192 == 0 && ceil_div(m, 256) * (n / 192) >= 256)
      return run_gemm<256, 192, 4, 2, 3, 2, kBInt4L>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                     stream);
    // 128 x 32 wave tiles, two or three workgroups (8 or 12 waves) per CU:
    // each dequantized B fragment feeds four MFMAs, and a CU's waves keep
    // the LDS fragment reads and the dequantization VALU work under the MFMAs.
    // Wide outputs with at least two rounds of 256-row tiles take 256 x 32
    // wave tiles at two workgroups per CU instead: every dequantized B
    // fragment then feeds eight MFMAs, which halves the dequantization VALU
    // per MFMA (measured: BERT FFN up at 32,768 tokens 212 -> 198 us, the
    // Qwen3-2B projections at 16,384 tokens 5-9% faster; 768-wide outputs and
    // 4096-token batches keep the 128-row tile, whose rounds divide evenly)
    const int64_t scale_bytes = 256 * w.n_groups * 2;
    if (n >= 2048 && ceil_div(m, 256) * ceil_div(n, 128) >= 512 &&
        gemm_lds_bytes(256, 128, 2, true) + scale_bytes <= 160 * 1024)
      return run_gemm<256, 128, 1, 4, 2, 2, kBInt4>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                  stream);
    cfg = ceil_div(m, 128) * ceil_div(n, 128) >= 128 ? kTileI4_128x128 : kTileI4_64x128;
  }
  if (cfg == kTileI4_128x128) {
    // three workgroups per CU (12 waves) with a two-stage pipeline while the
    // block's scales leave room for them in LDS, else two with three stages;
    // when the scales (many groups) leave room for only one, the 256-row
    // tile of the same LDS budget does twice the work per block
    const int64_t scale_bytes = 128 * w.n_groups * 2;
    if (gemm_lds_bytes(128, 128, 2, true) + scale_bytes <= (160 * 1024) / 3)
      return run_gemm<128, 128, 1, 4, 2, 3, kBInt4>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                  stream);
    if (gemm_lds_bytes(128, 128, 3, true) + scale_bytes > (160 * 1024) / 2 && m >= 256 &&
        gemm_lds_bytes(256, 128, 3, true) + scale_bytes <= 160 * 1024)
      cfg = kTileI4_256x128;
    else
      return run_gemm<128, 128, 1, 4, 3, 2, kBInt4>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                  stream);
  }
  if (cfg == kTileI4_256x128)
    return run_gemm<256, 128, 1, 4, 3, 1, kBInt4>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                stream);
  return run_gemm<64, 128, 1, 4, 3, 2, kBInt4>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                             stream);
}

hipError_t dispatch_bf16(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                         int64_t m, int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                         const LowRankEpilogue& epi, hipStream_t stream) {
  Int4Operand none;
  int cfg = tune(kTuneBf16Tile);
  if (cfg == kTileBf_256x256)
    return run_gemm<256, 256, 2, 2, 2, 1, kBBf16>(a, lda, b, ldb, none, m, n, k, out, ldc, epi,
                                                 stream);
  if (cfg == kTileAuto) {
    // Grids of at least 256 tiles of 256 x 128 take that tile with a
    // three-stage pipeline (one workgroup of 8 waves per CU): the deeper
    // prefetch pays on long reductions (the INT4 + LoRA backward at
    // 16384 x 2048 <- 6144: 538 us against 628 with two stages; 16384 x 6144
    // <- 2048: 597 against 636), except for short reductions (K <= 1024)
    // with many tiles, where 128 x 128 tiles at two workgroups per CU are
    // faster (32768 x 3072 <- 768: 323 against 330-341 us). 128 x 96 tiles
    // when they make one balanced round of 192-256 workgroups where
    // 128 x 128 would leave CUs idle (4096 x 768 outputs: 31 us against 33
    // for two uneven rounds of 64 x 128).
    const int64_t t128 = ceil_div(m, 128) * ceil_div(n, 128);
    const int64_t t96 = ceil_div(m, 128) * ceil_div(n, 96);
    if (ceil_div(m, 256) * ceil_div(n, 128) >= 256)
      cfg = k <= 1024 && t128 >= 512 ? kTileBf_128x128 : kTileBf_256x128s3;
    else
      cfg = t128 >= 256 ? kTileBf_128x128
                        : (t96 >= 192 && t96 <= 256 ? kTileBf_128x96 : kTileBf_64x128);
  }
  if (cfg == kTileBf_128x96)
    return run_gemm<128, 96, 4, 1, 3, 1, kBBf16>(a, lda, b, ldb, none, m, n, k, out, ldc, epi,
                                                stream);
  if (cfg == kTileBf_256x128)
    return run_gemm<256, 128, 4, 2, 2, 2, kBBf16>(a, lda, b, ldb, none, m, n, k, out, ldc, epi,
                                                 stream);
  if (cfg == kTileBf_256x128s3)
    return run_gemm<256, 128, 4, 2, 3, 2, kBBf16>(a, lda, b, ldb, none, m, n, k, out, ldc, epi,
                                                 stream);
  if (cfg == kTileBf_128x128)
    return run_gemm<128, 128, 2, 2, 2, 2, kBBf16>(a, lda, b, ldb, none, m, n, k, out, ldc, epi,
                                                 stream);
  return run_gemm<64, 128, 2, 2, 3, 2, kBBf16>(a, lda, b, ldb, none, m, n, k, out, ldc, epi,
                                              stream);
}

// The packed-weight input gradient: 256 x 128 tiles (8 waves, one workgroup
// per CU) when they make at least one round, else 128 x 128 (4 waves) when
// those do, else 64 x 128 at two workgroups per CU. The bf16 tile knob
// forces one of the three.
hipError_t dispatch_int4t(const uint16_t* a, int64_t lda, const Int4Operand& w, int64_t m,
                          int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                          const LowRankEpilogue& epi, hipStream_t stream) {
  int cfg = tune(kTuneBf16Tile);
  if (cfg != kTileT4_256x128 && cfg != kTileT4_128x128 && cfg != kTileT4_64x128) {
    if (ceil_div(m, 256) * (n / 128) >= 256)
      cfg = kTileT4_256x128;
    else if (ceil_div(m, 128) * (n / 128) >= 256)
      cfg = kTileT4_128x128;
    else
      cfg = kTileT4_64x128;
  }
  if (cfg == kTileT4_256x128)
    return run_gemm<256, 128, 4, 2, 3, 2, kBInt4T>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                   stream);
  if (cfg == kTileT4_128x128)
    return run_gemm<128, 128, 2, 2, 3, 1, kBInt4T>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                   stream);
  return run_gemm<64, 128, 2, 2, 3, 2, kBInt4T>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi,
                                                stream);
}

}  // namespace

bool int4t_gemm_ok(int64_t m, int64_t n, int64_t k, int64_t lda, const void* a,
                   const Int4Operand& w) {
  // 128-column tiles over whole packed bytes; the scale load takes one dword
  // per packed row (a per-row scale pair, or the tile's two 64-column groups)
  const bool scales_ok = w.n_groups == 1 || (w.group == 64 && w.n_groups * 64 == n);
  return m > 0 && n > 0 && n % 128 == 0 && k > 0 && k % kBK == 0 && lda % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(a) & 15) == 0 && w.packed_cols * 2 == n &&
         (reinterpret_cast<uintptr_t>(w.packed) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(w.scales) & 3) == 0 && scales_ok;
}

hipError_t launch_gemm_int4t(const uint16_t* a, int64_t lda, const Int4Operand& w, int64_t m,
                             int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                             const LowRankEpilogue& epi, hipStream_t stream) {
  if (m == 0 || n == 0) return hipSuccess;
  if (!int4t_gemm_ok(m, n, k, lda, a, w)) return hipErrorInvalidValue;
  return dispatch_int4t(a, lda, w, m, n, k, out, ldc, epi, stream);
}

bool gemm_fast_path_ok(int64_t k, int64_t lda, int64_t ldb_elems, const void* a, const void* b,
                       int64_t ldc, const void* out) {
  (void)ldc;
  (void)out;
  return k > 0 && k % kBK == 0 && lda % 8 == 0 && ldb_elems % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(a) & 15) == 0 && (reinterpret_cast<uintptr_t>(b) & 15) == 0;
}

hipError_t launch_gemm_int4(const uint16_t* a, int64_t lda, const Int4Operand& w, int64_t m,
                            int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                            const LowRankEpilogue& epi, hipStream_t stream) {
  if (m == 0 || n == 0) return hipSuccess;
  return dispatch_int4(a, lda, w, m, n, k, out, ldc, epi, stream);
}

hipError_t launch_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                            int64_t m, int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                            const LowRankEpilogue& epi, hipStream_t stream) {
  if (m == 0 || n == 0) return hipSuccess;
  return dispatch_bf16(a, lda, b, ldb, m, n, k, out, ldc, epi, stream);
}

}  // namespace rpx
