// Dynamically scaled OCP fp8 linear for gfx950
// (src/representax/precision.py:127-221).
//
//   amax  : per-block max |t| over ordered f32 bit patterns (NaN sorts above
//           inf, so NaN propagates like XLA's max), then a one-block finalize
//           that writes s = max(amax / fmax, FLT_MIN).
//   cast  : codes = f8(f32(t) / s), IEEE-rounded divide then a direct
//           round-to-nearest-even cast; optional row-major and transposed
//           outputs from one read of t.
//   gemm  : v_mfma_f32_32x32x64_f8f6f4 NT GEMM on fp8 codes, f32 accumulate,
//           epilogue ((acc * s_a) * s_b) rounded once to the output dtype;
//           optional split-K with fp32 partials and a deterministic sum.
#include <cstdlib>
#include <cstring>

#include "common.h"
#include "kernels.h"

namespace rpx {

namespace {

constexpr int kAmaxBlocks = 512;

__device__ __forceinline__ uint32_t abs_bits_f32(float f) {
  return __builtin_bit_cast(uint32_t, f) & 0x7FFFFFFFu;
}

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint32_t block_reduce_max(uint32_t v, uint32_t* sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    v = umax(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64)));
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  uint32_t r = 0;
  const int nw = blockDim.x / 64;
  for (int i = 0; i < nw; ++i) r = umax(r, sh[i]);
  return r;
}

// Dense buffer of numel elements (any logical layout).
__global__ void __launch_bounds__(256)
    k_amax_partial(const void* __restrict__ t, int dtype, int64_t numel,
                   uint32_t* __restrict__ partials) {
  __shared__ uint32_t sh[4];
  uint32_t m = 0;
  const int64_t tid = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  if (dtype == kBF16) {
    const uint16_t* p = static_cast<const uint16_t*>(t);
    const bool al = (reinterpret_cast<uintptr_t>(p) & 15) == 0;
    const int64_t nvec = al ? numel / 8 : 0;
    const u32x4_t* pv = reinterpret_cast<const u32x4_t*>(p);
    int64_t i = tid;
    for (; i + 3 * stride < nvec; i += 4 * stride) {
      u32x4_t w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) w[u] = pv[i + u * stride];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) m = umax(m, umax(w[u][e] & 0x7FFFu, (w[u][e] >> 16) & 0x7FFFu));
    }
    for (; i < nvec; i += stride) {
      const u32x4_t w = pv[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) m = umax(m, umax(w[e] & 0x7FFFu, (w[e] >> 16) & 0x7FFFu));
    }
    for (int64_t j = nvec * 8 + tid; j < numel; j += stride)
      m = umax(m, static_cast<uint32_t>(p[j] & 0x7FFFu));
    m <<= 16;
  } else {
    const float* p = static_cast<const float*>(t);
    const bool al = (reinterpret_cast<uintptr_t>(p) & 15) == 0;
    const int64_t nvec = al ? numel / 4 : 0;
    const u32x4_t* pv = reinterpret_cast<const u32x4_t*>(p);
    for (int64_t i = tid; i < nvec; i += stride) {
      const u32x4_t w = pv[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) m = umax(m, w[e] & 0x7FFFFFFFu);
    }
    for (int64_t i = nvec * 4 + tid; i < numel; i += stride) m = umax(m, abs_bits_f32(p[i]));
  }
  m = block_reduce_max(m, sh);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

__global__ void __launch_bounds__(256)
    k_amax_finalize(const uint32_t* __restrict__ partials, int64_t n, float fmax,
                    float* __restrict__ scale_out) {
  __shared__ uint32_t sh[4];
  uint32_t m = 0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) m = umax(m, partials[i]);
  m = block_reduce_max(m, sh);
  if (threadIdx.x == 0) {
    const float amax = __builtin_bit_cast(float, m);
    float s;
    if (m > 0x7F800000u) {
      s = __builtin_bit_cast(float, 0x7FC00000u);
    } else {
      s = amax / fmax;
      const float tiny = 1.17549435e-38f;
      s = s > tiny ? s : tiny;
    }
    scale_out[0] = s;
  }
}

__device__ __forceinline__ uint32_t encode(float v, int fmt) {
  return fmt == kE4M3FN ? f32_to_e4m3fn(v) : f32_to_e5m2(v);
}

// Two values -> two codes (a in the low byte). Inside the finite range the
// gfx950 packed convert (round to nearest even, OCP encodings) is used; NaN,
// infinities and |v| > fmax take the integer encoder, which has the
// non-saturating overflow behaviour. Agreement with the integer encoder over
// every f32 bit pattern is checked by rpx_fp8_encode_selfcheck.
__device__ __forceinline__ uint32_t encode2(float a, float b, int fmt) {
  uint32_t r;
  float fmax;
  if (fmt == kE4M3FN) {
    r = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xFFFFu;
    fmax = 448.0f;
  } else {
    r = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false)) & 0xFFFFu;
    fmax = 57344.0f;
  }
  if (!(__builtin_fabsf(a) <= fmax)) r = (r & 0xFF00u) | encode(a, fmt);
  if (!(__builtin_fabsf(b) <= fmax)) r = (r & 0x00FFu) | (encode(b, fmt) << 8);
  return r;
}

__device__ __forceinline__ float load_val(const void* t, int dtype, int64_t idx) {
  if (dtype == kBF16) return bf16_to_f32(static_cast<const uint16_t*>(t)[idx]);
  return static_cast<const float*>(t)[idx];
}

// Scale for this launch: the given value, or max(amax / fmax, FLT_MIN) from
// the amax partials (every block reduces them; block 0 also publishes it).
__device__ __forceinline__ float resolve_scale(const float* scale, const uint32_t* partials,
                                               int64_t n_partials, float fmax, float* scale_out,
                                               float* sh) {
  if (partials == nullptr) return scale[0];
  uint32_t m = 0;
  for (int64_t i = threadIdx.x; i < n_partials; i += blockDim.x) m = umax(m, partials[i]);
  __shared__ uint32_t red[4];
  m = block_reduce_max(m, red);
  if (threadIdx.x == 0) {
    float s;
    if (m > 0x7F800000u) {
      s = __builtin_bit_cast(float, 0x7FC00000u);
    } else {
      s = __builtin_bit_cast(float, m) / fmax;
      const float tiny = 1.17549435e-38f;
      s = s > tiny ? s : tiny;
    }
    *sh = s;
    if (scale_out != nullptr && blockIdx.x == 0 && blockIdx.y == 0) scale_out[0] = s;
  }
  __syncthreads();
  return *sh;
}

// Row-major input [rows, cols] (unit column stride, ld % 8 == 0, 16-byte
// aligned): a 64 x 64 tile per block, 2 x 8 contiguous elements per thread.
// All loads are issued before the scale reduction and the conversion.
template <int DT>
__global__ void __launch_bounds__(256)
    k_fp8_cast_rows(const void* __restrict__ t, int64_t rows, int64_t cols, int64_t ld,
                    const float* __restrict__ scale, const uint32_t* __restrict__ partials,
                    int64_t n_partials, float fmax, float* __restrict__ scale_out, int fmt,
                    uint8_t* __restrict__ out, uint8_t* __restrict__ out_t) {
  __shared__ __align__(16) uint8_t tile[64][64 + 16];
  __shared__ float s_sh;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int tid = threadIdx.x;
  const int cl = (tid % 8) * 8;
  float v[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rl = tid / 8 + 32 * i;
    const int64_t r = r0 + rl;
    const int64_t c = c0 + cl;
    const bool ok = (r < rows) && (c < cols);  // cols % 8 == 0: the 8-vector is all in or out
    if constexpr (DT == kBF16) {
      u32x4_t w = ok ? *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(t) + r * ld + c)
                     : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[i][2 * e] = bf16lo_to_f32(w[e]);
        v[i][2 * e + 1] = bf16hi_to_f32(w[e]);
      }
    } else {
      const float* p = static_cast<const float*>(t) + r * ld + c;
      f32x4_t a = ok ? *reinterpret_cast<const f32x4_t*>(p) : f32x4_t{0.f, 0.f, 0.f, 0.f};
      f32x4_t b = ok ? *reinterpret_cast<const f32x4_t*>(p + 4) : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[i][e] = a[e];
        v[i][4 + e] = b[e];
      }
    }
  }
  const float s = resolve_scale(scale, partials, n_partials, fmax, scale_out, &s_sh);
  const float rcp = 1.0f / s;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rl = tid / 8 + 32 * i;
    const int64_t r = r0 + rl;
    const int64_t c = c0 + cl;
    float q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = div_rn(v[i][e], s, rcp);
    const uint32_t lo = encode2(q[0], q[1], fmt) | (encode2(q[2], q[3], fmt) << 16);
    const uint32_t hi = encode2(q[4], q[5], fmt) | (encode2(q[6], q[7], fmt) << 16);
    if (out != nullptr && r < rows && c < cols)
      *reinterpret_cast<u32x2_t*>(out + r * cols + c) = u32x2_t{lo, hi};
    if (out_t != nullptr) *reinterpret_cast<u32x2_t*>(&tile[rl][cl]) = u32x2_t{lo, hi};
  }
  if (out_t == nullptr) return;
  __syncthreads();
  // out_t [cols, rows]: thread -> column c, 16 consecutive rows
  const int cc = tid % 64;
  const int rb = (tid / 64) * 16;
  const int64_t c = c0 + cc;
  const int64_t r = r0 + rb;
  if (c >= cols || r >= rows) return;
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    w[q] = static_cast<uint32_t>(tile[rb + 4 * q][cc]) |
           (static_cast<uint32_t>(tile[rb + 4 * q + 1][cc]) << 8) |
           (static_cast<uint32_t>(tile[rb + 4 * q + 2][cc]) << 16) |
           (static_cast<uint32_t>(tile[rb + 4 * q + 3][cc]) << 24);
  uint8_t* dst = out_t + c * rows + r;
  if (r + 15 < rows && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
    *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{w[0], w[1], w[2], w[3]};
  } else {
    for (int e = 0; e < 16; ++e)
      if (r + e < rows) dst[e] = static_cast<uint8_t>(w[e / 4] >> (8 * (e % 4)));
  }
}

// Any strides: 64 x 64 tile, loads first, then conversion; byte outputs.
__global__ void __launch_bounds__(256)
    k_fp8_cast_any(const void* __restrict__ t, int dtype, int64_t rows, int64_t cols,
                   int64_t s_row, int64_t s_col, const float* __restrict__ scale,
                   const uint32_t* __restrict__ partials, int64_t n_partials, float fmax,
                   float* __restrict__ scale_out, int fmt, uint8_t* __restrict__ out,
                   uint8_t* __restrict__ out_t) {
  __shared__ uint8_t tile[64][64 + 4];
  __shared__ float s_sh;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int tid = threadIdx.x;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rl = tid / 64 + 4 * i;
    const int cl = tid % 64;
    const int64_t r = r0 + rl;
    const int64_t c = c0 + cl;
    v[i] = (r < rows && c < cols) ? load_val(t, dtype, r * s_row + c * s_col) : 0.0f;
  }
  const float s = resolve_scale(scale, partials, n_partials, fmax, scale_out, &s_sh);
  const float rcp = 1.0f / s;
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const uint32_t two = encode2(div_rn(v[i], s, rcp), div_rn(v[i + 1], s, rcp), fmt);
    tile[tid / 64 + 4 * i][tid % 64] = static_cast<uint8_t>(two & 0xFFu);
    tile[tid / 64 + 4 * (i + 1)][tid % 64] = static_cast<uint8_t>(two >> 8);
  }
  __syncthreads();
  for (int i = 0; i < 16; ++i) {
    const int a = tid / 64 + 4 * i;
    const int b = tid % 64;
    if (out != nullptr && r0 + a < rows && c0 + b < cols) out[(r0 + a) * cols + c0 + b] = tile[a][b];
    if (out_t != nullptr && c0 + a < cols && r0 + b < rows)
      out_t[(c0 + a) * rows + r0 + b] = tile[b][a];
  }
}

// ---------------------------------------------------------------------------
// fp8 NT GEMM
// ---------------------------------------------------------------------------
constexpr int kBKb = 128;            // bytes (= fp8 elements) per K slice

template <int FA, int FB>
__device__ __forceinline__ f32x16_t mfma_f8(i32x8_t a, i32x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, FA, FB, 0, 0, 0, 0);
}

// vmcnt(n) with the expcnt / lgkmcnt fields left at "no wait" (gfx9 encoding).
#define RPX_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14))

typedef __attribute__((address_space(3))) void lds_void_t;

// Issues one K-slice of direct-to-LDS loads for this wave: AS A-segments and
// BS B-segments of 8 rows x 128 bytes (kept out of lambdas: the builtin is
// device-only).
template <int BM, int AS, int BS>
__device__ __forceinline__ void dma_stage(uint8_t* st, const uint8_t* const* a_src,
                                          const uint8_t* const* b_src, int64_t koff, int wave) {
#pragma unroll
  for (int i = 0; i < AS; ++i)
    __builtin_amdgcn_global_load_lds(
        a_src[i] + koff,
        reinterpret_cast<lds_void_t*>(reinterpret_cast<uintptr_t>(st) + (wave * AS + i) * 1024),
        16, 0, 0);
#pragma unroll
  for (int i = 0; i < BS; ++i)
    __builtin_amdgcn_global_load_lds(
        b_src[i] + koff,
        reinterpret_cast<lds_void_t*>(reinterpret_cast<uintptr_t>(st) + BM * kBKb +
                                      (wave * BS + i) * 1024),
        16, 0, 0);
}

// Pipelined fp8 NT GEMM. Each K-slice of 128 bytes of A [BM rows] and B [BN
// rows] moves global -> LDS with 16-byte direct-to-LDS loads (no register
// staging) into one of NS stages; NS - 1 slices are in flight while one is
// multiplied. LDS rows are 128 bytes, unpadded, with their eight 16-byte
// chunks XOR-swizzled by (row & 7) so that fragment reads are conflict-free:
// a DMA wave instruction writes 64 x 16 bytes = 8 rows contiguously, lane l
// landing at (row l/8, physical chunk l%8), so lane l fetches logical chunk
// (l%8) ^ (row & 7). Completion is tracked with explicit vmcnt waits and a
// plain s_barrier (a __syncthreads would wait for every load in flight).
template <int BM, int BN, int WM, int WN, int NS, int FA, int FB>
__global__ void __launch_bounds__(64 * WM * WN)
    k_fp8_gemm(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, int64_t M,
               int64_t N, int64_t K, int64_t k_per_split, const float* __restrict__ s_a,
               const float* __restrict__ s_b, void* __restrict__ out, int out_dtype,
               int64_t ldc, float* __restrict__ partials, int tiles_m, int tiles_n) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM;
  constexpr int TN = BN / WN;
  constexpr int FM = TM / 32;
  constexpr int FN = TN / 32;
  constexpr int A_SEGS = BM / 8;  // 1 KB DMA segments (8 rows) per stage
  constexpr int B_SEGS = BN / 8;
  static_assert(A_SEGS % NW == 0 && B_SEGS % NW == 0, "segments must split over waves");
  constexpr int LPW = (A_SEGS + B_SEGS) / NW;  // DMA instructions per wave per stage
  static_assert(LPW * (NS - 2) < 64, "vmcnt range");
  constexpr int STAGE = (BM + BN) * kBKb;
  extern __shared__ __align__(16) uint8_t smem8[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
  // Row-major (n fastest) tiles dealt to the 8 XCDs in contiguous ranges so
  // each XCD's L2 keeps a few A row-blocks; split-K slices are outermost.
  const int tiles = tiles_m * tiles_n;
  const int total = static_cast<int>(gridDim.x);
  int b = blockIdx.x;
  if (total % 8 == 0) b = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
  const int split = b / tiles;
  const int tile = b % tiles;
  const int tm = tile / tiles_n;
  const int tn = tile % tiles_n;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int64_t n0 = static_cast<int64_t>(tn) * BN;
  const int64_t kbeg = static_cast<int64_t>(split) * k_per_split;
  int64_t kend = kbeg + k_per_split;
  if (kend > K) kend = K;
  const int64_t nk = (kend - kbeg) / kBKb;

  // per-lane source rows/chunks for this wave's DMA segments
  const int seg_row = lane >> 3;                        // row within a segment
  const int chunk = (lane & 7) ^ (seg_row & 7);         // logical 16-byte chunk
  const uint8_t* a_src[A_SEGS / NW];
  const uint8_t* b_src[B_SEGS / NW];
#pragma unroll
  for (int i = 0; i < A_SEGS / NW; ++i) {
    int64_t r = m0 + (wave * (A_SEGS / NW) + i) * 8 + seg_row;
    r = r < M ? r : M - 1;
    a_src[i] = A + r * K + chunk * 16;
  }
#pragma unroll
  for (int i = 0; i < B_SEGS / NW; ++i) {
    int64_t r = n0 + (wave * (B_SEGS / NW) + i) * 8 + seg_row;
    r = r < N ? r : N - 1;
    b_src[i] = B + r * K + chunk * 16;
  }
  f32x16_t acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[fn][fm][v] = 0.0f;

  const int frow = lane & 31;        // fragment row within a 32-row block
  const int fhalf = lane >> 5;       // which 32 bytes of the 64-byte k sub-step
  auto frag = [&](const uint8_t* base, int row, int kk) -> i32x8_t {
    const int c0 = 4 * kk + 2 * fhalf;
    const uint8_t* r = base + row * kBKb;
    const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(r + ((c0 ^ (row & 7)) * 16));
    const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(r + (((c0 + 1) ^ (row & 7)) * 16));
    return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                   (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  auto compute = [&](int64_t t) {
    const uint8_t* sa = smem8 + (t % NS) * STAGE;
    const uint8_t* sb = sa + BM * kBKb;
#pragma unroll
    for (int kk = 0; kk < kBKb / 64; ++kk) {
      i32x8_t af[FM];
      i32x8_t bfr[FN];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) af[fm] = frag(sa, wm * TM + fm * 32 + frow, kk);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) bfr[fn] = frag(sb, wn * TN + fn * 32 + frow, kk);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) acc[fn][fm] = mfma_f8<FB, FA>(bfr[fn], af[fm], acc[fn][fm]);
    }
  };

#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk)
      dma_stage<BM, A_SEGS / NW, B_SEGS / NW>(smem8 + (s % NS) * STAGE, a_src, b_src,
                                               kbeg + s * kBKb, wave);
  for (int64_t t = 0; t < nk; ++t) {
    // slice t has landed once at most the later slices' loads are pending
    if (t + NS - 2 < nk) {
      RPX_WAIT_VMCNT(LPW * (NS - 2));
    } else {
      RPX_WAIT_VMCNT(0);
    }
    __builtin_amdgcn_s_barrier();
    if (t + NS - 1 < nk)  // refills the stage read at t - 1
      dma_stage<BM, A_SEGS / NW, B_SEGS / NW>(smem8 + ((t + NS - 1) % NS) * STAGE, a_src, b_src,
                                               kbeg + (t + NS - 1) * kBKb, wave);
    compute(t);
  }

  const float sa = s_a[0];
  const float sb = s_b[0];
  float* part = partials != nullptr ? partials + static_cast<int64_t>(split) * M * N : nullptr;
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int64_t m = m0 + wm * TM + fm * 32 + (lane & 31);
      if (m >= M) continue;
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        const int64_t nb = n0 + wn * TN + fn * 32 + 8 * vg + 4 * (lane >> 5);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = acc[fn][fm][4 * vg + e];
        if (part != nullptr) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (nb + e < N) part[m * N + nb + e] = y[e];
          continue;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (y[e] * sa) * sb;
        if (out_dtype == kBF16) {
          uint16_t* dst = static_cast<uint16_t*>(out) + m * ldc + nb;
          if (nb + 3 < N && (ldc % 4 == 0)) {
            *reinterpret_cast<u32x2_t*>(dst) =
                u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
          } else {
            for (int e = 0; e < 4; ++e)
              if (nb + e < N) dst[e] = f32_to_bf16(y[e]);
          }
        } else {
          float* dst = static_cast<float*>(out) + m * ldc + nb;
          for (int e = 0; e < 4; ++e)
            if (nb + e < N) dst[e] = y[e];
        }
      }
    }
  }
}

__global__ void __launch_bounds__(256)
    k_fp8_split_reduce(const float* __restrict__ partials, int64_t splits, int64_t M, int64_t N,
                       const float* __restrict__ s_a, const float* __restrict__ s_b,
                       void* __restrict__ out, int out_dtype, int64_t ldc) {
  const float sa = s_a[0];
  const float sb = s_b[0];
  const int64_t count = M * N;
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < count;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    float s = 0.0f;
    for (int64_t i = 0; i < splits; ++i) s += partials[i * count + e];
    s = (s * sa) * sb;
    const int64_t m = e / N;
    const int64_t n = e % N;
    if (out_dtype == kBF16)
      static_cast<uint16_t*>(out)[m * ldc + n] = f32_to_bf16(s);
    else
      static_cast<float*>(out)[m * ldc + n] = s;
  }
}

struct Fp8Plan {
  int cfg;  // 1: 256x128 (2x2), 2: 128x128 (2x2), 3: 256x256 (2x2), 4: 256x96 (4x1)
  int bm, bn;
  int64_t splits, k_per_split;
};

int fp8_tile_override() {
  static int cached = -1;
  if (cached < 0) {
    const char* env = std::getenv("RPX_FP8_TILE");
    cached = 0;
    if (env != nullptr) {
      if (std::strcmp(env, "256x128") == 0) cached = 1;
      if (std::strcmp(env, "128x128") == 0) cached = 2;
      if (std::strcmp(env, "256x256") == 0) cached = 3;
      if (std::strcmp(env, "256x96") == 0) cached = 4;
    }
  }
  return cached;
}

Fp8Plan plan_fp8(int64_t m, int64_t n, int64_t k) {
  static const int kBM[5] = {0, 256, 128, 256, 256};
  static const int kBN[5] = {0, 128, 128, 256, 96};
  Fp8Plan p;
  p.cfg = fp8_tile_override();
  if (p.cfg == 0) {
    // biggest tile that still gives one tile per CU, else 128x128 + split-K
    if (ceil_div(m, 256) * ceil_div(n, 256) >= 256)
      p.cfg = 3;
    else if (ceil_div(m, 256) * ceil_div(n, 128) >= 256)
      p.cfg = 1;
    else if (n % 96 == 0 && ceil_div(m, 256) * (n / 96) >= 256)
      p.cfg = 4;
    else
      p.cfg = 2;
  }
  p.bm = kBM[p.cfg];
  p.bn = kBN[p.cfg];
  const int64_t tiles = ceil_div(m, p.bm) * ceil_div(n, p.bn);
  const int64_t kslices = k / kBKb;
  int64_t s = 1;
  while (tiles * s < 256 && s * 2 <= kslices && s < 16) s *= 2;
  p.k_per_split = ceil_div(kslices, s) * kBKb;
  p.splits = ceil_div(k, p.k_per_split);
  return p;
}

template <int BM, int BN, int WM, int WN, int FA, int FB>
hipError_t run_fp8(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                   const Fp8Plan& plan, const float* s_a, const float* s_b, void* out,
                   int out_dtype, int64_t ldc, float* partials, hipStream_t stream) {
  // as many stages as fit in 160 KB of LDS (at most 4)
  constexpr int kStage = (BM + BN) * kBKb;
  constexpr int NS = (160 * 1024 / kStage) >= 4 ? 4 : (160 * 1024 / kStage);
  static_assert(NS >= 2, "tile too large for LDS");
  const int tiles_m = static_cast<int>(ceil_div(m, BM));
  const int tiles_n = static_cast<int>(ceil_div(n, BN));
  const size_t lds = static_cast<size_t>(NS) * kStage;
  auto kern = k_fp8_gemm<BM, BN, WM, WN, NS, FA, FB>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const unsigned blocks = static_cast<unsigned>(tiles_m) * tiles_n * plan.splits;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * WM * WN), lds, stream, a, b, m, n, k,
                     plan.k_per_split, s_a, s_b, out, out_dtype, ldc,
                     plan.splits > 1 ? partials : nullptr, tiles_m, tiles_n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || plan.splits == 1) return e;
  int64_t g = ceil_div(m * n, 256);
  if (g > 8192) g = 8192;
  hipLaunchKernelGGL(k_fp8_split_reduce, dim3(static_cast<unsigned>(g)), dim3(256), 0, stream,
                     partials, plan.splits, m, n, s_a, s_b, out, out_dtype, ldc);
  return hipGetLastError();
}

template <int FA, int FB>
hipError_t dispatch_fp8(const uint8_t* a, const uint8_t* b, int64_t m, int64_t n, int64_t k,
                        const float* s_a, const float* s_b, void* out, int out_dtype, int64_t ldc,
                        float* partials, hipStream_t stream) {
  const Fp8Plan plan = plan_fp8(m, n, k);
  switch (plan.cfg) {
    case 1:
      return run_fp8<256, 128, 2, 2, FA, FB>(a, b, m, n, k, plan, s_a, s_b, out, out_dtype, ldc,
                                             partials, stream);
    case 3:
      return run_fp8<256, 256, 2, 2, FA, FB>(a, b, m, n, k, plan, s_a, s_b, out, out_dtype, ldc,
                                             partials, stream);
    case 4:
      return run_fp8<256, 96, 4, 1, FA, FB>(a, b, m, n, k, plan, s_a, s_b, out, out_dtype, ldc,
                                            partials, stream);
    default:
      return run_fp8<128, 128, 2, 2, FA, FB>(a, b, m, n, k, plan, s_a, s_b, out, out_dtype, ldc,
                                             partials, stream);
  }
}

}  // namespace

int64_t fp8_amax_partials(int64_t numel) {
  int64_t g = ceil_div(numel, 256 * 16);
  if (g > kAmaxBlocks) g = kAmaxBlocks;
  if (g < 1) g = 1;
  return g;
}

hipError_t launch_fp8_amax(const void* t, int dtype, int64_t numel, uint32_t* partials,
                           int64_t n_partials, int fmt, float* scale_out, hipStream_t stream) {
  hipLaunchKernelGGL(k_amax_partial, dim3(static_cast<unsigned>(n_partials)), dim3(256), 0, stream,
                     t, dtype, numel, partials);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || scale_out == nullptr) return e;
  hipLaunchKernelGGL(k_amax_finalize, dim3(1), dim3(256), 0, stream, partials, n_partials,
                     fp8_max(fmt), scale_out);
  return hipGetLastError();
}

hipError_t launch_fp8_cast(const void* t, int dtype, int64_t rows, int64_t cols, int64_t s_row,
                           int64_t s_col, const float* scale, const uint32_t* partials,
                           int64_t n_partials, float* scale_out, int fmt, uint8_t* out,
                           uint8_t* out_t, hipStream_t stream) {
  if (rows == 0 || cols == 0) return hipSuccess;
  // A transposed view of a row-major buffer is cast as that buffer with the
  // two outputs exchanged.
  if (s_row == 1 && s_col != 1) {
    const int64_t tmp = rows;
    rows = cols;
    cols = tmp;
    s_row = s_col;
    s_col = 1;
    uint8_t* o = out;
    out = out_t;
    out_t = o;
  }
  const float fmax = fp8_max(fmt);
  const dim3 grid(static_cast<unsigned>(ceil_div(cols, 64)), static_cast<unsigned>(ceil_div(rows, 64)));
  const size_t esz = dtype == kBF16 ? 2 : 4;
  const bool rows_fast = s_col == 1 && cols % 8 == 0 && s_row % 8 == 0 &&
                         (reinterpret_cast<uintptr_t>(t) % 16 == 0) &&
                         (out == nullptr || reinterpret_cast<uintptr_t>(out) % 8 == 0) && esz > 0;
  if (rows_fast && dtype == kBF16) {
    hipLaunchKernelGGL(k_fp8_cast_rows<kBF16>, grid, dim3(256), 0, stream, t, rows, cols, s_row,
                       scale, partials, n_partials, fmax, scale_out, fmt, out, out_t);
  } else if (rows_fast) {
    hipLaunchKernelGGL(k_fp8_cast_rows<kF32>, grid, dim3(256), 0, stream, t, rows, cols, s_row,
                       scale, partials, n_partials, fmax, scale_out, fmt, out, out_t);
  } else {
    hipLaunchKernelGGL(k_fp8_cast_any, grid, dim3(256), 0, stream, t, dtype, rows, cols, s_row,
                       s_col, scale, partials, n_partials, fmax, scale_out, fmt, out, out_t);
  }
  return hipGetLastError();
}

namespace {
// Compares encode2 (hardware convert in range) with the integer encoder on
// bit patterns [first, first + count); per-block mismatch count and first
// mismatching pattern (0xFFFFFFFF when none) go to plain per-block slots.
__global__ void __launch_bounds__(256)
    k_fp8_encode_selfcheck(int fmt, uint64_t first, uint64_t count, uint32_t* __restrict__ counts,
                           uint32_t* __restrict__ firsts) {
  __shared__ uint32_t sc[256];
  __shared__ uint32_t sf[256];
  const uint64_t per_block = (count + gridDim.x - 1) / gridDim.x;
  const uint64_t b0 = first + per_block * blockIdx.x;
  uint64_t b1 = b0 + per_block;
  if (b1 > first + count) b1 = first + count;
  uint32_t bad = 0;
  uint32_t first_bad = 0xFFFFFFFFu;
  for (uint64_t p = b0 + threadIdx.x; p < b1; p += blockDim.x) {
    const uint32_t bits = static_cast<uint32_t>(p);
    const float a = __builtin_bit_cast(float, bits);
    const float b = __builtin_bit_cast(float, bits ^ 0x80000000u);
    const uint32_t hw = encode2(a, b, fmt);
    const uint32_t sw = encode(a, fmt) | (encode(b, fmt) << 8);
    if (hw != sw) {
      ++bad;
      if (bits < first_bad) first_bad = bits;
    }
  }
  sc[threadIdx.x] = bad;
  sf[threadIdx.x] = first_bad;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t c = 0, f = 0xFFFFFFFFu;
    for (int t = 0; t < 256; ++t) {
      c += sc[t];
      f = sf[t] < f ? sf[t] : f;
    }
    counts[blockIdx.x] = c;
    firsts[blockIdx.x] = f;
  }
}
}  // namespace

hipError_t launch_fp8_encode_selfcheck(int fmt, uint64_t first, uint64_t count, uint32_t* counts,
                                       uint32_t* firsts, int64_t blocks, hipStream_t stream) {
  hipLaunchKernelGGL(k_fp8_encode_selfcheck, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, fmt, first, count, counts, firsts);
  return hipGetLastError();
}

int64_t fp8_gemm_workspace_floats(int64_t m, int64_t n, int64_t k) {
  const Fp8Plan p = plan_fp8(m, n, k);
  return p.splits > 1 ? p.splits * m * n : 0;
}

hipError_t launch_fp8_gemm(const uint8_t* a, int fmt_a, const float* s_a, const uint8_t* b,
                           int fmt_b, const float* s_b, int64_t m, int64_t n, int64_t k,
                           void* out, int out_dtype, int64_t ldc, float* split_ws,
                           int64_t split_ws_floats, hipStream_t stream) {
  if (m == 0 || n == 0) return hipSuccess;
  if (split_ws_floats < fp8_gemm_workspace_floats(m, n, k)) return hipErrorInvalidValue;
  // MFMA format codes: 0 = fp8 (e4m3), 1 = bf8 (e5m2)
  if (fmt_a == kE4M3FN && fmt_b == kE4M3FN)
    return dispatch_fp8<0, 0>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
  if (fmt_a == kE5M2 && fmt_b == kE4M3FN)
    return dispatch_fp8<1, 0>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
  if (fmt_a == kE4M3FN && fmt_b == kE5M2)
    return dispatch_fp8<0, 1>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
  return dispatch_fp8<1, 1>(a, b, m, n, k, s_a, s_b, out, out_dtype, ldc, split_ws, stream);
}

}  // namespace rpx
