// bf16 MFMA "NT" GEMM for gfx950: C[M, N] = A[M, K] . B[N, K]^T with both
// operands K-contiguous. B is either bf16 rows or packed INT4 rows that are
// dequantized (exactly: bf16(q * s)) while being staged into LDS.
//
// Tiling: BM x BN x 64 block tile, WM x WN waves, each wave a
// (BM/WM) x (BN/WN) sub-tile of v_mfma_f32_32x32x16_bf16 blocks. LDS is
// double buffered; the next K-slice's global loads are in flight while the
// current slice is multiplied, and the INT4 nibble unpack runs on the VALU
// between MFMA issues.
//
// Accumulator orientation: the MFMA's first operand is the B (weight) row
// fragment, so lane l of a 32x32 block owns output row m = l % 32 and the
// registers v = 0..15 hold output columns n = 8*(v/4) + 4*(l/32) + v%4,
// which lets each lane store 4 consecutive bf16 outputs at once.
#include <cstdlib>
#include <cstring>

#include "common.h"
#include "kernels.h"

namespace rpx {

namespace {

constexpr int kBK = 64;
constexpr int kPad = 8;              // bf16 elements of padding per LDS row
constexpr int kLdsLd = kBK + kPad;   // 144-byte rows: conflict-free b128 reads

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

// Exact nibble dequant of one packed dword (8 values) into 4 bf16 pairs.
// q*s = fma(float(u ^ 8), s, -8 s) is exact in f32 (q has 4 bits, s 8).
__device__ __forceinline__ void dequant8(uint32_t word, float s, float m8s, uint32_t* o) {
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

template <int BM, int BN, int WM, int WN, bool INT4, int JB>
__global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(JB == 4 ? 1 : 2)))
    k_gemm_nt(const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ B,
              int64_t ldb, Int4Operand w, int group_shift, int64_t M, int64_t N, int64_t K,
              uint16_t* __restrict__ out, int64_t ldc, LowRankEpilogue epi, int tiles_m) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / WM;
  constexpr int TN = BN / WN;
  constexpr int FM = TM / 32;
  constexpr int FN = TN / 32;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
  extern __shared__ __align__(16) uint16_t smem[];
  uint16_t* sA = smem;
  uint16_t* sB = smem + 2 * BM * kLdsLd;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
  // Tiles in row-major (n fastest) order, dealt to the 8 XCDs (which take
  // workgroups round-robin) in contiguous ranges, so that each XCD's L2
  // holds a few A row-blocks and streams the weight tiles.
  const int tiles = gridDim.x;
  int tile = blockIdx.x;
  if (tiles % 8 == 0) tile = (blockIdx.x % 8) * (tiles / 8) + blockIdx.x / 8;
  const int tiles_n = tiles / tiles_m;
  const int tm = tile / tiles_n;
  const int tn = tile % tiles_n;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int64_t n0 = static_cast<int64_t>(tn) * BN;

  constexpr int A_VECS = BM * kBK / 8;
  static_assert(A_VECS % NT == 0, "A tile must split evenly");
  constexpr int A_PER_T = A_VECS / NT;
  constexpr int B_VECS = INT4 ? BN * kBK / 32 : BN * kBK / 8;
  constexpr int B_PER_T = (B_VECS + NT - 1) / NT;
  constexpr int B_VPR = INT4 ? kBK / 32 : kBK / 8;  // vectors per row

  u32x4_t a_reg[A_PER_T];
  u32x4_t b_reg[B_PER_T];
  float b_scale[B_PER_T];

  auto load_a = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int v = tid + i * NT;
      const int row = v / (kBK / 8);
      const int c = (v % (kBK / 8)) * 8;
      const int64_t gm = m0 + row;
      a_reg[i] = (gm < M) ? *reinterpret_cast<const u32x4_t*>(A + gm * lda + k0 + c)
                          : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto load_b = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int v = tid + i * NT;
      const int row = v / B_VPR;
      const int c = v % B_VPR;
      const int64_t gn = n0 + row;
      const bool ok = (v < B_VECS) && (gn < N);
      if constexpr (INT4) {
        const int64_t kc = k0 + c * 32;
        b_reg[i] = ok ? *reinterpret_cast<const u32x4_t*>(w.packed + gn * w.packed_cols + kc / 2)
                      : u32x4_t{0u, 0u, 0u, 0u};
        const int64_t gi = (w.n_groups == 1) ? 0 : (kc >> group_shift);
        b_scale[i] = ok ? bf16_to_f32(w.scales[gn * w.n_groups + gi]) : 0.0f;
      } else {
        b_reg[i] = ok ? *reinterpret_cast<const u32x4_t*>(B + gn * ldb + k0 + c * 8)
                      : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
  };
  auto store_a = [&](int buf) {
    uint16_t* base = sA + buf * BM * kLdsLd;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int v = tid + i * NT;
      const int row = v / (kBK / 8);
      const int c = (v % (kBK / 8)) * 8;
      *reinterpret_cast<u32x4_t*>(base + row * kLdsLd + c) = a_reg[i];
    }
  };
  auto store_b = [&](int buf) {
    uint16_t* base = sB + buf * BN * kLdsLd;
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int v = tid + i * NT;
      if (v >= B_VECS) continue;
      const int row = v / B_VPR;
      const int c = v % B_VPR;
      if constexpr (INT4) {
        const float s = b_scale[i];
        const float m8s = -8.0f * s;
        uint32_t o[16];
#pragma unroll
        for (int d = 0; d < 4; ++d) dequant8(b_reg[i][d], s, m8s, o + 4 * d);
        u32x4_t* dst = reinterpret_cast<u32x4_t*>(base + row * kLdsLd + c * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          dst[q] = u32x4_t{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
      } else {
        *reinterpret_cast<u32x4_t*>(base + row * kLdsLd + c * 8) = b_reg[i];
      }
    }
  };

  f32x16_t acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[fn][fm][v] = 0.0f;

  auto compute = [&](int buf) {
    const uint16_t* a_base =
        sA + buf * BM * kLdsLd + (wm * TM + (lane & 31)) * kLdsLd + (lane >> 5) * 8;
    const uint16_t* b_base =
        sB + buf * BN * kLdsLd + (wn * TN + (lane & 31)) * kLdsLd + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8_t af[FM];
      bf16x8_t bfr[FN];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        af[fm] = *reinterpret_cast<const bf16x8_t*>(a_base + fm * 32 * kLdsLd + kk * 16);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        bfr[fn] = *reinterpret_cast<const bf16x8_t*>(b_base + fn * 32 * kLdsLd + kk * 16);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
          acc[fn][fm] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[fn], af[fm], acc[fn][fm], 0, 0, 0);
    }
  };

  const int64_t nk = K / kBK;
  load_a(0);
  load_b(0);
  store_a(0);
  store_b(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = static_cast<int>(kt & 1);
    const bool more = kt + 1 < nk;
    if (more) {
      load_a((kt + 1) * kBK);
      load_b((kt + 1) * kBK);
    }
    compute(cur);
    if (more) {
      store_a(cur ^ 1);
      store_b(cur ^ 1);
    }
    __syncthreads();
  }

  // Epilogue --------------------------------------------------------------
  // The low-rank term t = C R^T for this lane's rows m and columns n is one
  // more 32x32x16 MFMA per 16 ranks; its fragments are loaded up front.
  constexpr int kMaxJB = JB > 0 ? JB : 1;  // ceil(rank / 16), rank <= 16 * JB
  const int jblocks = JB > 0 ? static_cast<int>((epi.rank + 15) / 16) : 0;
  const bool vec_store = (ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(out) & 7) == 0);
  bf16x8_t cf[kMaxJB][FM];
  if (jblocks > 0) {
#pragma unroll
    for (int jb = 0; jb < kMaxJB; ++jb) {
      if (jb >= jblocks) break;
      const int64_t jl = jb * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int64_t m = m0 + wm * TM + fm * 32 + (lane & 31);
        cf[jb][fm] = load8_j(epi.cols + m * epi.cols_sm + jl * epi.cols_sj, epi.cols_sj,
                             m < M ? valid8(epi.rank, jl) : 0);
      }
    }
  }
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    const int64_t n_blk = n0 + wn * TN + fn * 32;
    bf16x8_t rf[kMaxJB];
    if (jblocks > 0) {
      const int64_t n_row = n_blk + (lane & 31);
#pragma unroll
      for (int jb = 0; jb < kMaxJB; ++jb) {
        if (jb >= jblocks) break;
        const int64_t jl = jb * 16 + (lane >> 5) * 8;
        rf[jb] = load8_j(epi.rows + n_row * epi.rows_sn + jl * epi.rows_sj, epi.rows_sj,
                         n_row < N ? valid8(epi.rank, jl) : 0);
      }
    }
    float bias4[4][4];
#pragma unroll
    for (int vg = 0; vg < 4; ++vg)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t nn = n_blk + 8 * vg + 4 * (lane >> 5) + e;
        bias4[vg][e] = (epi.bias != nullptr && nn < N) ? bf16_to_f32(epi.bias[nn]) : 0.0f;
      }
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int64_t m = m0 + wm * TM + fm * 32 + (lane & 31);
      f32x16_t t;
#pragma unroll
      for (int v = 0; v < 16; ++v) t[v] = 0.0f;
#pragma unroll
      for (int jb = 0; jb < kMaxJB; ++jb) {
        if (jb >= jblocks) break;
        t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rf[jb], cf[jb][fm], t, 0, 0, 0);
      }
      if (m >= M) continue;
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        const int64_t nb = n_blk + 8 * vg + 4 * (lane >> 5);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = 4 * vg + e;
          float r = round_bf16(acc[fn][fm][v]);
          if (jblocks > 0) r = round_bf16(r + round_bf16(round_bf16(t[v]) * epi.scale));
          if (epi.bias != nullptr) r = round_bf16(r + bias4[vg][e]);
          y[e] = r;
        }
        uint16_t* dst = out + m * ldc + nb;
        if (vec_store && nb + 3 < N) {
          *reinterpret_cast<u32x2_t*>(dst) =
              u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (nb + e < N) dst[e] = f32_to_bf16(y[e]);
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, bool INT4, int JB>
hipError_t run_gemm_jb(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                       const Int4Operand& w, int64_t m, int64_t n, int64_t k, uint16_t* out,
                       int64_t ldc, const LowRankEpilogue& epi, hipStream_t stream) {
  const int tiles_m = static_cast<int>(ceil_div(m, BM));
  const int tiles_n = static_cast<int>(ceil_div(n, BN));
  const size_t lds = static_cast<size_t>(2) * (BM + BN) * kLdsLd * sizeof(uint16_t);
  auto kern = k_gemm_nt<BM, BN, WM, WN, INT4, JB>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  int group_shift = 0;
  if (INT4 && w.n_groups > 1) {
    while ((int64_t{1} << group_shift) < w.group) ++group_shift;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(tiles_m) * tiles_n), dim3(64 * WM * WN),
                     lds, stream, a, lda, b, ldb, w, group_shift, m, n, k, out, ldc, epi,
                     tiles_m);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, bool INT4>
hipError_t run_gemm(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                    const Int4Operand& w, int64_t m, int64_t n, int64_t k, uint16_t* out,
                    int64_t ldc, const LowRankEpilogue& epi, hipStream_t stream) {
  if (epi.rank <= 0)
    return run_gemm_jb<BM, BN, WM, WN, INT4, 0>(a, lda, b, ldb, w, m, n, k, out, ldc, epi, stream);
  if (epi.rank <= 16)
    return run_gemm_jb<BM, BN, WM, WN, INT4, 1>(a, lda, b, ldb, w, m, n, k, out, ldc, epi, stream);
  if (epi.rank <= 32)
    return run_gemm_jb<BM, BN, WM, WN, INT4, 2>(a, lda, b, ldb, w, m, n, k, out, ldc, epi, stream);
  return run_gemm_jb<BM, BN, WM, WN, INT4, 4>(a, lda, b, ldb, w, m, n, k, out, ldc, epi, stream);
}

// Tile configuration: RPX_GEMM_TILE=256x128|128x128|128x64 overrides the
// size-based choice (for tuning sweeps).
int tile_override() {
  static int cached = -1;
  if (cached < 0) {
    const char* env = std::getenv("RPX_GEMM_TILE");
    cached = 0;
    if (env != nullptr) {
      if (std::strcmp(env, "256x128") == 0) cached = 1;
      if (std::strcmp(env, "128x128") == 0) cached = 2;
      if (std::strcmp(env, "128x64") == 0) cached = 3;
    }
  }
  return cached;
}

template <bool INT4>
hipError_t dispatch(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                    const Int4Operand& w, int64_t m, int64_t n, int64_t k, uint16_t* out,
                    int64_t ldc, const LowRankEpilogue& epi, hipStream_t stream) {
  int cfg = tile_override();
  if (cfg == 0) {
    // 128x128 tiles (two workgroups per CU by LDS) unless that leaves CUs
    // idle; measured faster than 256x128 at one workgroup per CU
    const int64_t cus = 256;
    cfg = (ceil_div(m, 128) * ceil_div(n, 128) >= cus) ? 2 : 3;
  }
  if (cfg == 1)
    return run_gemm<256, 128, 2, 2, INT4>(a, lda, b, ldb, w, m, n, k, out, ldc, epi, stream);
  if (cfg == 2)
    return run_gemm<128, 128, 2, 2, INT4>(a, lda, b, ldb, w, m, n, k, out, ldc, epi, stream);
  return run_gemm<128, 64, 2, 2, INT4>(a, lda, b, ldb, w, m, n, k, out, ldc, epi, stream);
}

}  // namespace

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
  return dispatch<true>(a, lda, nullptr, 0, w, m, n, k, out, ldc, epi, stream);
}

hipError_t launch_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                            int64_t m, int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                            const LowRankEpilogue& epi, hipStream_t stream) {
  if (m == 0 || n == 0) return hipSuccess;
  Int4Operand none;
  return dispatch<false>(a, lda, b, ldb, none, m, n, k, out, ldc, epi, stream);
}

}  // namespace rpx
