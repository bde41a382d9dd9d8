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

}  // namespace rpx
