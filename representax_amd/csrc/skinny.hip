// Skinny-M INT4 + LoRA forward (M <= 64 tokens): the memory-bound inference
// regime where every call streams the whole packed weight for a few rows.
//
// Launch 1 (k_skinny_partials), two kinds of blocks:
//   weight blocks  (64 rows of W x one K chunk): x[:, chunk] staged in LDS,
//                  each wave streams 16 rows with 16-byte loads, dequantizes
//                  exactly (bf16(q*s)) and runs v_mfma_f32_16x16x32_bf16 with
//                  the weights as the row operand; fp32 partial sums go to
//                  part_w[chunk][m][n].
//   adapter blocks (one K chunk of h = x A^T): fp32 partials part_h[chunk][m][j].
// Launch 2 (k_skinny_finish): fixed-order sums of the partials, then the
// reference's rounding points: h = bf16(.), base = bf16(.),
// a = bf16(h B^T), y = bf16(base + bf16(a * c)) (+ bias).
#include "common.h"
#include "kernels.h"

namespace rpx {

namespace {

constexpr int kRowsPerBlock = 64;  // 4 waves x 16 rows
constexpr int kMaxVec = 4;         // 16-byte weight vectors per lane per chunk (kc <= 512)

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// Exact dequant of one packed dword (8 nibbles) into 4 bf16 pairs.
__device__ __forceinline__ void dequant8_exact(uint32_t word, float s, float m8s, uint32_t* o) {
  const uint32_t x = word ^ 0x88888888u;
  const uint32_t lo = x & 0x0F0F0F0Fu;
  const uint32_t hi = (x >> 4) & 0x0F0F0F0Fu;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float fl = static_cast<float>((lo >> (8 * b)) & 0xFFu);
    const float fh = static_cast<float>((hi >> (8 * b)) & 0xFFu);
    o[b] = pack_bf16x2(__builtin_fmaf(fl, s, m8s), __builtin_fmaf(fh, s, m8s));
  }
}

struct SkinnyArgs {
  const uint16_t* x;   // [M, K] bf16
  int64_t m, k, n;
  const uint8_t* packed;  // [N, K/2]
  const uint16_t* scales; // [N, n_groups]
  int64_t n_groups;
  int group_shift;        // log2(group) when n_groups > 1
  const uint16_t* lora_a; // [r, K] bf16
  int64_t rank;
  int64_t kc;             // K chunk (multiple of 128)
  int64_t splits;         // number of K chunks
  int64_t w_blocks_n;     // ceil(N / 64)
  float* part_w;          // [splits][M][N]
  float* part_h;          // [splits][M][r]
};

template <int MB>
__global__ void __launch_bounds__(256) k_skinny_partials(SkinnyArgs a) {
  extern __shared__ __align__(16) uint16_t xs[];  // [MB*16][kc + 8]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t ld = a.kc + 8;
  const int64_t weight_blocks = a.w_blocks_n * a.splits;
  const bool is_weight = blockIdx.x < weight_blocks;
  const int64_t bid = is_weight ? blockIdx.x : blockIdx.x - weight_blocks;
  const int64_t split = is_weight ? bid / a.w_blocks_n : bid;
  const int64_t k0 = split * a.kc;
  int64_t k1 = k0 + a.kc;
  if (k1 > a.k) k1 = a.k;
  const int64_t klen = k1 - k0;

  // stage x[:, k0:k1] (rows >= M are zero)
  const int64_t vecs = static_cast<int64_t>(MB) * 16 * (klen / 8);
  for (int64_t v = tid; v < vecs; v += 256) {
    const int64_t row = v / (klen / 8);
    const int64_t c = (v % (klen / 8)) * 8;
    const u32x4_t val = row < a.m ? *reinterpret_cast<const u32x4_t*>(a.x + row * a.k + k0 + c)
                                  : u32x4_t{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4_t*>(xs + row * ld + c) = val;
  }
  __syncthreads();

  const int rl = lane & 15;
  const int g = lane >> 4;
  if (is_weight) {
    const int64_t n_blk = bid % a.w_blocks_n;
    const int64_t row = n_blk * kRowsPerBlock + wave * 16 + rl;
    const bool row_ok = row < a.n;
    const uint8_t* wrow = a.packed + (row_ok ? row : 0) * (a.k / 2);
    float s_row = 0.0f;
    if (a.n_groups == 1 && row_ok) s_row = bf16_to_f32(a.scales[row]);
    f32x4_t acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int64_t nblk128 = klen / 128;  // <= kMaxVec
    u32x4_t wv[kMaxVec];
    float sv[kMaxVec];
#pragma unroll
    for (int b = 0; b < kMaxVec; ++b) {
      const int64_t kb = k0 + b * 128;
      const bool ok = row_ok && b < nblk128;
      wv[b] = ok ? *reinterpret_cast<const u32x4_t*>(wrow + (kb + 32 * g) / 2)
                 : u32x4_t{0u, 0u, 0u, 0u};
      sv[b] = s_row;
      if (a.n_groups > 1)
        sv[b] = ok ? bf16_to_f32(a.scales[row * a.n_groups + ((kb + 32 * g) >> a.group_shift)])
                   : 0.0f;
    }
#pragma unroll
    for (int b = 0; b < kMaxVec; ++b) {
      if (b >= nblk128) break;
      const int64_t kb = k0 + b * 128;
      const float s = sv[b];
      const float m8s = -8.0f * s;
      uint32_t dq[16];
#pragma unroll
      for (int d = 0; d < 4; ++d) dequant8_exact(wv[b][d], s, m8s, dq + 4 * d);
      const uint16_t* xb = xs + (kb - k0) + 32 * g;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const bf16x8_t af = as_bf16x8(u32x4_t{dq[4 * st], dq[4 * st + 1], dq[4 * st + 2],
                                              dq[4 * st + 3]});
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const bf16x8_t xf =
              *reinterpret_cast<const bf16x8_t*>(xb + (mb * 16 + rl) * ld + 8 * st);
          acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, xf, acc[mb], 0, 0, 0);
        }
      }
    }
    // D[n][m]: lane -> m = 16*mb + (lane & 15), n = 4*(lane >> 4) + v
    float* out = a.part_w + split * a.m * a.n;
    const int64_t nb = n_blk * kRowsPerBlock + wave * 16 + 4 * g;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int64_t mm = mb * 16 + rl;
      if (mm >= a.m) continue;
      float* dst = out + mm * a.n + nb;
      if (nb + 3 < a.n && (a.n % 4 == 0)) {
        *reinterpret_cast<f32x4_t*>(dst) = acc[mb];
      } else {
        for (int v = 0; v < 4; ++v)
          if (nb + v < a.n) dst[v] = acc[mb][v];
      }
    }
    return;
  }
  // adapter block: partial h[m, j] over this chunk; A[:, chunk] is staged in
  // LDS behind x (all loads issued together), wave w handles j in
  // [16 w, 16 w + 16) (rank <= 64)
  uint16_t* as = xs + static_cast<int64_t>(MB) * 16 * ld;
  const int64_t avecs = a.rank * (klen / 8);
  for (int64_t v = tid; v < avecs; v += 256) {
    const int64_t jr = v / (klen / 8);
    const int64_t c = (v % (klen / 8)) * 8;
    *reinterpret_cast<u32x4_t*>(as + jr * ld + c) =
        *reinterpret_cast<const u32x4_t*>(a.lora_a + jr * a.k + k0 + c);
  }
  __syncthreads();
  const int64_t j = wave * 16 + rl;
  f32x4_t acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (wave * 16 < a.rank) {
    for (int64_t kk = 0; kk < klen; kk += 32) {
      u32x4_t av = u32x4_t{0u, 0u, 0u, 0u};
      if (j < a.rank) av = *reinterpret_cast<const u32x4_t*>(as + j * ld + kk + 8 * g);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const bf16x8_t xf = *reinterpret_cast<const bf16x8_t*>(xs + (mb * 16 + rl) * ld + kk + 8 * g);
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), xf, acc[mb], 0, 0, 0);
      }
    }
    float* out = a.part_h + split * a.m * a.rank;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int64_t mm = mb * 16 + rl;
      if (mm >= a.m) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t jj = wave * 16 + 4 * g + v;
        if (jj < a.rank) out[mm * a.rank + jj] = acc[mb][v];
      }
    }
  }
}

// One block per (m, 256-column slab): h row from its partials (fixed order),
// then each thread finishes one output element.
__global__ void __launch_bounds__(256)
    k_skinny_finish(const float* __restrict__ part_w, const float* __restrict__ part_h,
                    int64_t splits, int64_t m_rows, int64_t n, int64_t rank,
                    const uint16_t* __restrict__ lora_b, float scale,
                    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                    uint16_t* __restrict__ h) {
  __shared__ float hrow[64];
  const int64_t mm = blockIdx.y;
  const int tid = threadIdx.x;
  if (tid < rank) {
    float s = 0.0f;
    for (int64_t i = 0; i < splits; ++i) s += part_h[(i * m_rows + mm) * rank + tid];
    const float hb = round_bf16(s);
    hrow[tid] = hb;
    if (blockIdx.x == 0) h[mm * rank + tid] = f32_to_bf16(hb);
  }
  __syncthreads();
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 256 + tid;
  if (col >= n) return;
  float s = 0.0f;
#pragma unroll 8
  for (int64_t i = 0; i < splits; ++i) s += part_w[(i * m_rows + mm) * n + col];
  const float base = round_bf16(s);
  float t = 0.0f;
  for (int64_t jj = 0; jj < rank; ++jj)
    t = __builtin_fmaf(hrow[jj], bf16_to_f32(lora_b[col * rank + jj]), t);
  float out = round_bf16(base + round_bf16(round_bf16(t) * scale));
  if (bias != nullptr) out = round_bf16(out + bf16_to_f32(bias[col]));
  y[mm * n + col] = f32_to_bf16(out);
}

struct SkinnyPlan {
  int64_t kc, splits, w_blocks_n, mb;
};

SkinnyPlan plan_skinny(int64_t m, int64_t n, int64_t k) {
  SkinnyPlan p;
  p.mb = (m + 15) / 16;
  p.w_blocks_n = ceil_div(n, kRowsPerBlock);
  const int64_t k128 = k / 128;
  int64_t want = ceil_div(1024, p.w_blocks_n);  // ~4 blocks per CU
  if (want > k128) want = k128;
  if (want < 1) want = 1;
  // chunk <= kMaxVec * 128 columns (weight vectors held in registers)
  while (ceil_div(k128, want) > kMaxVec) ++want;
  p.kc = ceil_div(k128, want) * 128;
  p.splits = ceil_div(k, p.kc);
  return p;
}

}  // namespace

bool skinny_ok(int64_t m, int64_t k, int64_t rank, int64_t n_groups, int64_t group) {
  if (m < 1 || m > 64 || k % 128 != 0 || rank < 1 || rank > 64) return false;
  if (n_groups > 1 && (group < 32 || (group & (group - 1)) != 0)) return false;
  return true;
}

int64_t skinny_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t rank) {
  const SkinnyPlan p = plan_skinny(m, n, k);
  return p.splits * m * n + p.splits * m * rank + 64;
}

hipError_t launch_skinny_forward(const uint16_t* x, int64_t m, int64_t k, const Int4Operand& w,
                                 int64_t n, const uint16_t* lora_a, const uint16_t* lora_b,
                                 int64_t rank, float scale, const uint16_t* bias, uint16_t* y,
                                 uint16_t* h, float* ws, hipStream_t stream) {
  const SkinnyPlan p = plan_skinny(m, n, k);
  SkinnyArgs a;
  a.x = x;
  a.m = m;
  a.k = k;
  a.n = n;
  a.packed = w.packed;
  a.scales = w.scales;
  a.n_groups = w.n_groups;
  a.group_shift = 0;
  if (w.n_groups > 1)
    while ((int64_t{1} << a.group_shift) < w.group) ++a.group_shift;
  a.lora_a = lora_a;
  a.rank = rank;
  a.kc = p.kc;
  a.splits = p.splits;
  a.w_blocks_n = p.w_blocks_n;
  a.part_w = ws;
  a.part_h = ws + p.splits * m * n;
  const unsigned blocks = static_cast<unsigned>(p.w_blocks_n * p.splits + p.splits);
  // x rows (16 * mb) and, for the adapter blocks, up to 64 rows of A
  const size_t lds = static_cast<size_t>(p.mb * 16 + rank) * (p.kc + 8) * sizeof(uint16_t);
  static bool attr_set[4] = {false, false, false, false};
  const void* kerns[4] = {reinterpret_cast<const void*>(k_skinny_partials<1>),
                          reinterpret_cast<const void*>(k_skinny_partials<2>),
                          reinterpret_cast<const void*>(k_skinny_partials<3>),
                          reinterpret_cast<const void*>(k_skinny_partials<4>)};
  const int ki = static_cast<int>(p.mb) - 1;
  if (!attr_set[ki]) {
    // up to (64 + 64) rows x (512 + 8) bf16 = 133 KB
    hipError_t e = hipFuncSetAttribute(kerns[ki], hipFuncAttributeMaxDynamicSharedMemorySize,
                                       160 * 1024);
    if (e != hipSuccess) return e;
    attr_set[ki] = true;
  }
  switch (p.mb) {
    case 1:
      hipLaunchKernelGGL(k_skinny_partials<1>, dim3(blocks), dim3(256), lds, stream, a);
      break;
    case 2:
      hipLaunchKernelGGL(k_skinny_partials<2>, dim3(blocks), dim3(256), lds, stream, a);
      break;
    case 3:
      hipLaunchKernelGGL(k_skinny_partials<3>, dim3(blocks), dim3(256), lds, stream, a);
      break;
    default:
      hipLaunchKernelGGL(k_skinny_partials<4>, dim3(blocks), dim3(256), lds, stream, a);
      break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid(static_cast<unsigned>(ceil_div(n, 256)), static_cast<unsigned>(m));
  hipLaunchKernelGGL(k_skinny_finish, grid, dim3(256), 0, stream, a.part_w, a.part_h, p.splits, m,
                     n, rank, lora_b, scale, bias, y, h);
  return hipGetLastError();
}

}  // namespace rpx
