// INT4 pack / unpack / dequant kernels and the merged-weight export kernel.
//
// Packed layout (identical to the reference's integer leaves):
//   packed     uint8 [N, ceil(K/2)]  low nibble = even column, high = odd
//   scale_bits uint16[N, n_groups]   bf16 bit patterns; n_groups = 1 is the
//                                    reference's per-output-row scheme
// Nibbles are two's-complement int4; the packer emits -7..7.
#include "common.h"
#include "kernels.h"

namespace rpx {

// ---------------------------------------------------------------------------
// Dequant: W_b[n, k] = bf16(f32(q) * f32(s)); the product is exact in f32, so
// the result is one round-to-nearest-even, bit-identical to
// src/representax/models/adapters.py:68-79.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float nibble_value(uint32_t nib) {
  // two's complement 4-bit -> float
  return static_cast<float>(static_cast<int>((nib ^ 8u)) - 8);
}

// Vector path: each thread converts 8 packed bytes (16 values).
// Requires K % 16 == 0 and packed row stride == K / 2.
__global__ void __launch_bounds__(256) k_int4_dequant_vec(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
    uint16_t* __restrict__ out, int64_t n_rows, int64_t k, int64_t n_groups,
    int64_t group) {
  const int64_t chunks_per_row = k / 16;
  const int64_t total = n_rows * chunks_per_row;
  for (int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; c < total;
       c += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = c / chunks_per_row;
    const int64_t col = (c % chunks_per_row) * 16;
    const u32x2_t w = *reinterpret_cast<const u32x2_t*>(packed + row * (k / 2) + col / 2);
    const float s = bf16_to_f32(scales[row * n_groups + col / group]);
    uint32_t o[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t word = w[h];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = nibble_value((word >> (8 * i)) & 0xFu) * s;
        const float hi = nibble_value((word >> (8 * i + 4)) & 0xFu) * s;
        o[h * 4 + i] = pack_bf16x2(lo, hi);
      }
    }
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + row * k + col);
    dst[0] = u32x4_t{o[0], o[1], o[2], o[3]};
    dst[1] = u32x4_t{o[4], o[5], o[6], o[7]};
  }
}

// General path: one thread per output element (any K, any packed stride).
__global__ void __launch_bounds__(256) k_int4_dequant_any(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
    uint16_t* __restrict__ out, int64_t n_rows, int64_t k, int64_t packed_cols,
    int64_t n_groups, int64_t group) {
  const int64_t total = n_rows * k;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = e / k;
    const int64_t col = e % k;
    const uint32_t byte = packed[row * packed_cols + col / 2];
    const uint32_t nib = (col & 1) ? (byte >> 4) : (byte & 0xFu);
    const float s = bf16_to_f32(scales[row * n_groups + col / group]);
    out[e] = f32_to_bf16(nibble_value(nib) * s);
  }
}

// Transposed dequant for groups that are multiples of 32 (and per-row
// scales): out[k, n] = W_b[n, k]. A block takes 64 rows (n) x 128 columns (k):
// the packed bytes arrive in LDS with one 16-byte load per thread; each
// thread then turns one byte column of 8 consecutive rows into two output
// rows (k even / odd) of 8 consecutive n, stored as 16 bytes each.
__device__ __forceinline__ void dequant_t32_tile(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
    uint16_t* __restrict__ out, int64_t n_rows, int64_t k, int64_t packed_cols,
    int64_t n_groups, int64_t group, int64_t ld_out, int64_t bx, int64_t by,
    uint8_t (&pk)[64][80], float (&sc)[64][5]) {
  const int64_t n0 = by * 64;
  const int64_t k0 = bx * 128;
  const int t = threadIdx.x;
  {
    const int r = t >> 2;
    const int c = t & 3;  // 16-byte chunk: columns k0 + 32 c .. + 31
    const int64_t n = n0 + r;
    const int64_t b0 = k0 / 2 + 16 * c;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (n < n_rows) {
      const uint8_t* src = packed + n * packed_cols + b0;
      if (b0 + 16 <= packed_cols && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
        v = *reinterpret_cast<const u32x4_t*>(src);
      } else {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        for (int i = 0; i < 16; ++i)
          if (b0 + i < packed_cols) w[i >> 2] |= static_cast<uint32_t>(src[i]) << (8 * (i & 3));
        v = u32x4_t{w[0], w[1], w[2], w[3]};
      }
    }
    *reinterpret_cast<u32x4_t*>(&pk[r][16 * (c ^ ((r >> 4) & 3))]) = v;
    const int64_t kc = k0 + 32 * c;
    sc[r][c] = (n < n_rows && kc < k) ? bf16_to_f32(scales[n * n_groups + kc / group]) : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int unit = 0; unit < 2; ++unit) {
    const int o = t & 7;                 // n-octet
    const int pb = (t >> 3) + 32 * unit;  // byte column = k pair
    const int64_t ke = k0 + 2 * pb;
    uint32_t lo4[4], hi4[4];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      float ve[2], vo[2];
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int r = 8 * o + i + d;
        const uint32_t byte = pk[r][(((pb >> 4) ^ ((r >> 4) & 3)) << 4) | (pb & 15)] ^ 0x88u;
        const float s = sc[r][pb >> 4];
        ve[d] = __builtin_fmaf(static_cast<float>(byte & 0xFu), s, -8.0f * s);
        vo[d] = __builtin_fmaf(static_cast<float>(byte >> 4), s, -8.0f * s);
      }
      lo4[i >> 1] = pack_bf16x2(ve[0], ve[1]);
      hi4[i >> 1] = pack_bf16x2(vo[0], vo[1]);
    }
    const int64_t n = n0 + 8 * o;
    const bool full = n + 8 <= n_rows && (ld_out & 7) == 0 &&
                      (reinterpret_cast<uintptr_t>(out) & 15) == 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t kk = ke + h;
      if (kk >= k) continue;
      const uint32_t* w = h ? hi4 : lo4;
      uint16_t* dst = out + kk * ld_out + n;
      if (full) {
        *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{w[0], w[1], w[2], w[3]};
      } else {
        for (int e = 0; e < 8; ++e)
          if (n + e < n_rows) dst[e] = static_cast<uint16_t>((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      }
    }
  }
}

__global__ void __launch_bounds__(256) k_int4_dequant_t32(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
    uint16_t* __restrict__ out, int64_t n_rows, int64_t k, int64_t packed_cols,
    int64_t n_groups, int64_t group, int64_t ld_out) {
  // 16-byte chunk c of row r sits at chunk c ^ ((r >> 4) & 3), and scale
  // rows are padded to 5 floats: the byte and scale reads of a wave's eight
  // row-octets then fall in eight different banks.
  __shared__ __align__(16) uint8_t pk[64][80];
  __shared__ float sc[64][5];
  dequant_t32_tile(packed, scales, out, n_rows, k, packed_cols, n_groups, group, ld_out,
                   blockIdx.x, blockIdx.y, pk, sc);
}

// 32 x 32 tile of a bf16 transpose through LDS.
__device__ __forceinline__ void transpose_tile(const uint16_t* __restrict__ in, int64_t rows,
                                               int64_t cols, int64_t ld_in,
                                               uint16_t* __restrict__ out, int64_t ld_out,
                                               int64_t bx, int64_t by, uint16_t (&tile)[32][33]) {
  const int64_t r0 = by * 32;
  const int64_t c0 = bx * 32;
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

// The INT4-LoRA backward's operand preparation in one launch: B^T [r, N]
// (blocks [0, tb)), A^T [K, r] (blocks [tb, tb + ta)) and the dequantized
// W_b^T [K, N] (the rest; groups that are multiples of 32).
struct BwdPrep {
  const uint16_t* b;  // [N, r]
  uint16_t* bt;       // [r, N]
  const uint16_t* a;  // [r, K]
  uint16_t* at;       // [K, r]
  const uint8_t* packed;
  const uint16_t* scales;
  uint16_t* wt;       // [K, N]
  int64_t n, k, rank, packed_cols, n_groups, group;
  int64_t tb_x, tb, ta_x, ta, tw_x;
};

__global__ void __launch_bounds__(256) k_int4lora_bwd_prep(BwdPrep p) {
  __shared__ __align__(16) uint8_t pk[64][80];
  __shared__ float sc[64][5];
  __shared__ uint16_t tile[32][33];
  int64_t b = blockIdx.x;
  if (b < p.tb) {
    transpose_tile(p.b, p.n, p.rank, p.rank, p.bt, p.n, b % p.tb_x, b / p.tb_x, tile);
    return;
  }
  b -= p.tb;
  if (b < p.ta) {
    transpose_tile(p.a, p.rank, p.k, p.k, p.at, p.rank, b % p.ta_x, b / p.ta_x, tile);
    return;
  }
  b -= p.ta;
  dequant_t32_tile(p.packed, p.scales, p.wt, p.n, p.k, p.packed_cols, p.n_groups, p.group, p.n,
                   b % p.tw_x, b / p.tw_x, pk, sc);
}

// Transposed dequant: out[k, n] = W_b[n, k], row stride ld_out (>= N).
// Tile of 64 rows (n) x 64 columns (k) through LDS.
__global__ void __launch_bounds__(256) k_int4_dequant_t(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
    uint16_t* __restrict__ out, int64_t n_rows, int64_t k, int64_t packed_cols,
    int64_t n_groups, int64_t group, int64_t ld_out) {
  __shared__ uint16_t tile[64][64 + 2];
  const int64_t n0 = (int64_t)blockIdx.y * 64;
  const int64_t k0 = (int64_t)blockIdx.x * 64;
  const int t = threadIdx.x;
  // load: 64 rows x 32 bytes; each thread handles 8 bytes? -> 64*32/256 = 8 bytes
  {
    const int r = t / 4;           // 0..63
    const int cb = (t % 4) * 8;    // byte offset within the 32-byte row chunk
    const int64_t n = n0 + r;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int64_t kk = k0 + 2 * (cb + b);
      uint32_t byte = 0;
      if (n < n_rows && kk < k) byte = packed[n * packed_cols + kk / 2];
      float v0 = 0.f, v1 = 0.f;
      if (n < n_rows && kk < k) {
        v0 = nibble_value(byte & 0xFu) * bf16_to_f32(scales[n * n_groups + kk / group]);
      }
      if (n < n_rows && kk + 1 < k) {
        v1 = nibble_value(byte >> 4) * bf16_to_f32(scales[n * n_groups + (kk + 1) / group]);
      }
      const uint32_t p = pack_bf16x2(v0, v1);
      tile[2 * (cb + b)][r] = static_cast<uint16_t>(p & 0xFFFFu);
      tile[2 * (cb + b) + 1][r] = static_cast<uint16_t>(p >> 16);
    }
  }
  __syncthreads();
  // store: 64 k-rows x 64 n-columns; each thread writes 16 values of one row
  {
    const int r = t / 4;
    const int c0 = (t % 4) * 16;
    const int64_t kk = k0 + r;
    if (kk < k) {
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const int64_t n = n0 + c0 + c;
        if (n < n_rows) out[kk * ld_out + n] = tile[r][c0 + c];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Packer (src/representax/models/adapters.py:38-65), one wave per
// (row, group): w_b = bf16(w); m = max|w_b|; s = bf16(m / 7) (1.0 if m is not
// positive); q = clip(rint(bf16(w_b / s)), -7, 7); nibble = q & 0xF.
// Groups hold an even number of columns unless there is a single group.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float load_weight(const void* w, int dtype, int64_t idx) {
  if (dtype == kBF16) return bf16_to_f32(static_cast<const uint16_t*>(w)[idx]);
  return static_cast<const float*>(w)[idx];
}

__global__ void __launch_bounds__(256) k_int4_pack(
    const void* __restrict__ weight, int dtype, uint8_t* __restrict__ packed,
    uint16_t* __restrict__ scales, int64_t n_rows, int64_t k, int64_t packed_cols,
    int64_t n_groups, int64_t group) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
  if (unit >= n_rows * n_groups) return;
  const int64_t row = unit / n_groups;
  const int64_t g = unit % n_groups;
  const int64_t c_begin = g * group;
  const int64_t c_end = c_begin + group;  // group divides k
  const int64_t base = row * k;
  // pass 1: maximum of |bf16(w)| as ordered bit patterns (NaN sorts above inf)
  uint32_t mx = 0;
  for (int64_t c = c_begin + lane; c < c_end; c += 64) {
    const float wb = round_bf16(load_weight(weight, dtype, base + c));
    const uint32_t bits = __builtin_bit_cast(uint32_t, wb) & 0x7FFFFFFFu;
    mx = bits > mx ? bits : mx;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t o = static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), off, 64));
    mx = o > mx ? o : mx;
  }
  const float maximum = __builtin_bit_cast(float, mx);
  const float s = (maximum > 0.0f) ? round_bf16(maximum / 7.0f) : 1.0f;
  if (lane == 0) scales[row * n_groups + g] = f32_to_bf16(s);
  // pass 2: quantize column pairs; a pair never straddles two groups because
  // groups start at even columns.
  for (int64_t c = c_begin + 2 * lane; c < c_end; c += 128) {
    uint32_t nib[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t cc = c + h;
      nib[h] = 0;
      if (cc < c_end) {
        const float wb = round_bf16(load_weight(weight, dtype, base + cc));
        const float t = round_bf16(wb / s);
        float q = __builtin_rintf(t);
        q = q < -7.0f ? -7.0f : (q > 7.0f ? 7.0f : q);
        const int qi = (t != t) ? 0 : static_cast<int>(q);
        nib[h] = static_cast<uint32_t>(qi) & 0xFu;
      }
    }
    packed[row * packed_cols + c / 2] = static_cast<uint8_t>(nib[0] | (nib[1] << 4));
  }
}

// ---------------------------------------------------------------------------
// Merged export weight (adapters.py:150-156):
//   out[n, k] = f32(W_b[n, k]) + f32(sum_j B[n, j] * A[j, k]) * f32(alpha / r)
// with float32 masters A [r, K], B [N, r].
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_int4_merge(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
    const float* __restrict__ lora_a, const float* __restrict__ lora_b,
    float* __restrict__ out, int64_t n_rows, int64_t k, int64_t packed_cols,
    int64_t n_groups, int64_t group, int64_t rank, float scaling) {
  const int64_t total = n_rows * k;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = e / k;
    const int64_t col = e % k;
    const uint32_t byte = packed[row * packed_cols + col / 2];
    const uint32_t nib = (col & 1) ? (byte >> 4) : (byte & 0xFu);
    const float s = bf16_to_f32(scales[row * n_groups + col / group]);
    const float base = round_bf16(nibble_value(nib) * s);
    float acc = 0.0f;
    for (int64_t j = 0; j < rank; ++j) acc = fmaf(lora_b[row * rank + j], lora_a[j * k + col], acc);
    out[e] = base + acc * scaling;
  }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
static int grid_for(int64_t work, int per_block = 256) {
  int64_t g = ceil_div(work, per_block);
  if (g > 65535 * 16) g = 65535 * 16;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

hipError_t launch_int4_dequant(const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                               int64_t n, int64_t k, int64_t packed_cols, int64_t n_groups,
                               int64_t group, hipStream_t stream) {
  if (n == 0 || k == 0) return hipSuccess;
  const bool vec = (k % 16 == 0) && (packed_cols == k / 2) && (group % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(packed) % 8 == 0) &&
                   (reinterpret_cast<uintptr_t>(out) % 16 == 0);
  if (vec) {
    hipLaunchKernelGGL(k_int4_dequant_vec, dim3(grid_for(n * (k / 16))), dim3(256), 0, stream,
                       packed, scales, out, n, k, n_groups, group);
  } else {
    hipLaunchKernelGGL(k_int4_dequant_any, dim3(grid_for(n * k)), dim3(256), 0, stream, packed,
                       scales, out, n, k, packed_cols, n_groups, group);
  }
  return hipGetLastError();
}

hipError_t launch_int4_dequant_t(const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                                 int64_t n, int64_t k, int64_t packed_cols, int64_t n_groups,
                                 int64_t group, int64_t ld_out, hipStream_t stream) {
  if (n == 0 || k == 0) return hipSuccess;
  if (group % 32 == 0) {
    dim3 grid(static_cast<unsigned>(ceil_div(k, 128)), static_cast<unsigned>(ceil_div(n, 64)));
    hipLaunchKernelGGL(k_int4_dequant_t32, grid, dim3(256), 0, stream, packed, scales, out, n, k,
                       packed_cols, n_groups, group, ld_out);
    return hipGetLastError();
  }
  dim3 grid(static_cast<unsigned>(ceil_div(k, 64)), static_cast<unsigned>(ceil_div(n, 64)));
  hipLaunchKernelGGL(k_int4_dequant_t, grid, dim3(256), 0, stream, packed, scales, out, n, k,
                     packed_cols, n_groups, group, ld_out);
  return hipGetLastError();
}

hipError_t launch_int4lora_bwd_prep(const uint16_t* b, uint16_t* bt, const uint16_t* a,
                                   uint16_t* at, const uint8_t* packed, const uint16_t* scales,
                                   uint16_t* wt, int64_t n, int64_t k, int64_t rank,
                                   int64_t packed_cols, int64_t n_groups, int64_t group,
                                   hipStream_t stream) {
  if (group % 32 != 0) return hipErrorInvalidValue;
  BwdPrep p;
  p.b = b;
  p.bt = bt;
  p.a = a;
  p.at = at;
  p.packed = packed;
  p.scales = scales;
  p.wt = wt;
  p.n = n;
  p.k = k;
  p.rank = rank;
  p.packed_cols = packed_cols;
  p.n_groups = n_groups;
  p.group = group;
  p.tb_x = ceil_div(rank, 32);
  p.tb = p.tb_x * ceil_div(n, 32);
  p.ta_x = ceil_div(k, 32);
  p.ta = p.ta_x * ceil_div(rank, 32);
  p.tw_x = ceil_div(k, 128);
  // wt == nullptr: B^T and A^T only (the input gradient reads the packed
  // weight itself)
  const int64_t tw = wt == nullptr ? 0 : p.tw_x * ceil_div(n, 64);
  hipLaunchKernelGGL(k_int4lora_bwd_prep, dim3(static_cast<unsigned>(p.tb + p.ta + tw)), dim3(256),
                     0, stream, p);
  return hipGetLastError();
}

hipError_t launch_int4_pack(const void* weight, int dtype, uint8_t* packed, uint16_t* scales,
                            int64_t n, int64_t k, int64_t packed_cols, int64_t n_groups,
                            int64_t group, hipStream_t stream) {
  const int64_t units = n * n_groups;
  if (units == 0) return hipSuccess;
  hipLaunchKernelGGL(k_int4_pack, dim3(static_cast<unsigned>(ceil_div(units, 4))), dim3(256), 0,
                     stream, weight, dtype, packed, scales, n, k, packed_cols, n_groups, group);
  return hipGetLastError();
}

hipError_t launch_int4_merge(const uint8_t* packed, const uint16_t* scales, const float* lora_a,
                             const float* lora_b, float* out, int64_t n, int64_t k,
                             int64_t packed_cols, int64_t n_groups, int64_t group, int64_t rank,
                             float scaling, hipStream_t stream) {
  if (n == 0 || k == 0) return hipSuccess;
  hipLaunchKernelGGL(k_int4_merge, dim3(grid_for(n * k)), dim3(256), 0, stream, packed, scales,
                     lora_a, lora_b, out, n, k, packed_cols, n_groups, group, rank, scaling);
  return hipGetLastError();
}

}  // namespace rpx
