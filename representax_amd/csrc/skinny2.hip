// Skinny-M INT4 + LoRA forward for M <= 16 tokens (selected for M <= 4), the
// memory-bound embedding-inference regime, where a call is a few dependent
// device round trips. Two forms: two launches with no cross-block exchange
// inside either (below), and one launch in which the adapter's h is
// published to the weight blocks (k_skinny_one, further down), chosen by K.
//
//   k_skinny_main, one grid with two block roles:
//     adapter blocks (first in the grid, so they dispatch first): block
//       (s, q) writes the fp32 partial P[s][m][16 q + i] = sum over its
//       128 NW columns of x[m, k] A[16 q + i, k]; its waves take one 128-column
//       chunk each and reduce through LDS in wave order;
//     weight blocks: block b owns output rows [16 b, 16 b + 16) over the
//       whole K. Every wave issues all of its 16-byte packed-weight, scale
//       and x loads first, dequantizes exactly (bf16(q * s)) and runs
//       v_mfma_f32_16x16x32_bf16 with the weight rows as the row operand and
//       x as the column operand; the waves reduce through LDS in wave order
//       and wave 0 stores base = bf16(acc) into y. Wave 0 also touches the
//       block's rows of B and bias so that they are cache-resident for the
//       second launch.
//   k_skinny_finish: every block sums the partials in slice order into
//     h = bf16(sum_s P[s]) (block 0 also stores h), then for its rows
//     t = bf16(sum_j h[m, j] B[n, j]) (sequential fma over j) and
//     y = bf16(base + bf16(t * c)) (+ bias, rounded again).
// The adapter's cold loads overlap the weight stream instead of preceding
// it, and the second launch reads only cache-resident data.
//
// Within a 128-column chunk lane l takes k = 32 (l >> 4) + [0, 32): one
// 16-byte load of 32 nibbles, and MFMA step s uses k = 32 (l >> 4) + 8 s +
// [0, 8), the same permutation on both operands. The lane then holds
// D[row 4 (l >> 4) + v][column m = l & 15].
#include <atomic>
#include <cstdlib>

#include "coherent.h"
#include "common.h"
#include "kernels.h"
#include "tuning.h"

namespace rpx {

namespace {

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));

constexpr int kFinRows = 64;       // output rows per finishing block
constexpr int kFinThreads = 256;

struct Skinny2Params {
  const uint16_t* x;  // [M, K] bf16
  int m;
  int64_t k;
  int64_t n;
  const uint8_t* packed;
  int64_t pcols;
  const uint16_t* scales;
  int64_t n_groups;
  int group_shift;
  const uint16_t* lora_a;  // [rank, K]
  const uint16_t* lora_b;  // [N, rank]
  int rank;
  float scale;
  const uint16_t* bias;  // [N] or null
  uint16_t* y;           // [M, N]
  uint16_t* h;           // [M, rank]
  float* part;           // [slices][M][rank]
  int slices;            // adapter K slices of 128 * NW columns
  int a_blocks;          // slices * ceil(rank / 16)
  int b_vec;             // B rows may be touched with 16-byte loads
  // one-launch form: the call's slot of arrival words ([0] adapter blocks,
  // [1] h published, [2] done: weight blocks and the publishing adapter
  // block; zero between calls), the published h as f32 [M, rank], the polls
  // of the bounded wait and the device error word
  int slot;
  float* hf;
  int w_blocks;
  int spin;
  unsigned int* err;
};

__device__ __forceinline__ u32x4_t ld16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

__device__ __forceinline__ bf16x8_v as_frag(u32x4_t v) { return __builtin_bit_cast(bf16x8_v, v); }

__device__ __forceinline__ f32x4_v mfma16(u32x4_t a, u32x4_t b, f32x4_v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_frag(a), as_frag(b), c, 0, 0, 0);
}

// 8 bf16 of x row m from column k (zeros for rows past M or chunks past K)
__device__ __forceinline__ u32x4_t x_frag(const Skinny2Params& p, int m, int64_t k, bool ok) {
  const u32x4_t z{0u, 0u, 0u, 0u};
  if (!ok || m >= p.m) return z;
  return ld16(p.x + static_cast<int64_t>(m) * p.k + k);
}

// 8 nibbles (k ascending, low nibble first) -> 8 bf16: bf16(q * s), exact
// in f32 as fma(u, s, -8 s) with u = nibble ^ 8.
__device__ __forceinline__ u32x4_t dequant8(uint32_t word, float s) {
  const float m8s = -8.0f * s;
  const uint32_t xw = word ^ 0x88888888u;
  const uint32_t lo = xw & 0x0F0F0F0Fu;
  const uint32_t hi = (xw >> 4) & 0x0F0F0F0Fu;
  uint32_t o[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float fl = static_cast<float>((lo >> (8 * b)) & 0xFFu);
    const float fh = static_cast<float>((hi >> (8 * b)) & 0xFFu);
    o[b] = pack_bf16x2(__builtin_fmaf(fl, s, m8s), __builtin_fmaf(fh, s, m8s));
  }
  return u32x4_t{o[0], o[1], o[2], o[3]};
}

// Sum of the NW waves' accumulators in wave order; the total is valid in
// wave 0.
template <int NW>
__device__ __forceinline__ f32x4_v reduce_waves(f32x4_v acc, f32x4_v* red) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (wave > 0) red[(wave - 1) * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 1; w < NW; ++w) acc += red[(w - 1) * 64 + lane];
  }
  return acc;
}

// Adapter block a = (K slice s, 16-rank group q): the fp32 partial of
// x A^T over the slice's 128 NW columns, one 128-column chunk per wave,
// summed over the waves in wave order; valid in wave 0, where lane l holds
// P[s][m = l & 15][j = 16 q + 4 (l >> 4) + v].
template <int NW>
__device__ __forceinline__ f32x4_v adapter_partial(const Skinny2Params& p, int a, f32x4_v* red,
                                                   int* s_out, int* q_out) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rl = lane & 15;
  const int g = lane >> 4;
  const int groups = (p.rank + 15) / 16;
  const int q = a % groups;
  const int s = a / groups;
  const int j = 16 * q + rl;
  const bool jok = j < p.rank;
  const uint16_t* arow = p.lora_a + static_cast<int64_t>(jok ? j : p.rank - 1) * p.k;
  const int64_t c = static_cast<int64_t>(s) * NW + wave;
  const bool ok = c < p.k / 128;
  const int64_t k0 = ok ? c * 128 + 32 * g : 0;
  u32x4_t av[4], xv[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    av[st] = ok && jok ? ld16(arow + k0 + 8 * st) : u32x4_t{0u, 0u, 0u, 0u};
    xv[st] = x_frag(p, rl, k0 + 8 * st, ok);
  }
  f32x4_v acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < 4; ++st) acc = mfma16(av[st], xv[st], acc);
  *s_out = s;
  *q_out = q;
  return reduce_waves<NW>(acc, red);
}

template <int NW>
__device__ __forceinline__ void adapter_block(const Skinny2Params& p, int a, f32x4_v* red) {
  int s, q;
  const f32x4_v acc = adapter_partial<NW>(p, a, red, &s, &q);
  const int lane = threadIdx.x & 63;
  const int rl = lane & 15;
  if ((threadIdx.x >> 6) != 0 || rl >= p.m) return;
  float* dst = p.part + (static_cast<int64_t>(s) * p.m + rl) * p.rank;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int jj = 16 * q + 4 * (lane >> 4) + v;
    if (jj < p.rank) dst[jj] = acc[v];
  }
}

// A weight block's loads: rows n0 + (l & 15) over the wave's chunks
// c = wave + i NW of 128 columns (16-byte packed word, scale, 4 x fragments).
template <int CPW>
struct WeightFrags {
  u32x4_t wv[CPW];
  u32x4_t xv[CPW][4];
  uint16_t sv[CPW];
};

template <int NW, int CPW>
__device__ __forceinline__ void weight_loads(const Skinny2Params& p, int64_t n0,
                                             WeightFrags<CPW>& f) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rl = lane & 15;
  const int g = lane >> 4;
  const int64_t row = n0 + rl;
  const int64_t rc = row < p.n ? row : p.n - 1;
  const uint8_t* wrow = p.packed + rc * p.pcols;
  const uint16_t* srow = p.scales + rc * p.n_groups;
  const int64_t nchunks = p.k / 128;
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int64_t c = wave + static_cast<int64_t>(i) * NW;
    const bool ok = c < nchunks;
    const int64_t k0 = ok ? c * 128 + 32 * g : 0;
    f.wv[i] = ok ? ld16(wrow + k0 / 2) : u32x4_t{0u, 0u, 0u, 0u};
    f.sv[i] = srow[p.n_groups == 1 ? 0 : (k0 >> p.group_shift)];
#pragma unroll
    for (int st = 0; st < 4; ++st) f.xv[i][st] = x_frag(p, rl, k0 + 8 * st, ok);
  }
}

// Dequantized MFMAs over the loaded chunks, summed over the waves in wave
// order: valid in wave 0, lane l holding D[n0 + 4 (l >> 4) + v][m = l & 15].
template <int NW, int CPW>
__device__ __forceinline__ f32x4_v weight_mfma(const WeightFrags<CPW>& f, f32x4_v* red) {
  f32x4_v acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const float s = bf16_to_f32(f.sv[i]);
#pragma unroll
    for (int st = 0; st < 4; ++st) acc = mfma16(dequant8(f.wv[i][st], s), f.xv[i][st], acc);
  }
  return reduce_waves<NW>(acc, red);
}

// y[m][nb .. nb + 3] = o (bf16 bits), one 8-byte store when whole and aligned
__device__ __forceinline__ void store_row4(const Skinny2Params& p, int m, int64_t nb,
                                           const uint16_t (&o)[4]) {
  uint16_t* dst = p.y + static_cast<int64_t>(m) * p.n + nb;
  if (nb + 3 < p.n && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
    *reinterpret_cast<u32x2_t*>(dst) =
        u32x2_t{static_cast<uint32_t>(o[0]) | (static_cast<uint32_t>(o[1]) << 16),
                static_cast<uint32_t>(o[2]) | (static_cast<uint32_t>(o[3]) << 16)};
  } else {
    for (int v = 0; v < 4 && nb + v < p.n; ++v) dst[v] = o[v];
  }
}

template <int NW, int CPW>
__device__ __forceinline__ void weight_block(const Skinny2Params& p, int64_t b, f32x4_v* red) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rl = lane & 15;
  const int64_t n0 = 16 * b;
  WeightFrags<CPW> f;
  weight_loads<NW, CPW>(p, n0, f);
  // the block's B rows (16 rank contiguous bf16) and bias, touched for the
  // finishing launch
  uint32_t touch = 0;
  if (wave == 0) {
    const int64_t rows = (p.n - n0 < 16 ? p.n - n0 : 16);
    if (p.b_vec && 8 * lane < rows * p.rank) touch = ld16(p.lora_b + n0 * p.rank + 8 * lane).x;
    if (p.bias != nullptr && lane < rows) touch ^= p.bias[n0 + lane];
  }
  const f32x4_v acc = weight_mfma<NW, CPW>(f, red);
  if (wave != 0) return;
  asm volatile("" ::"v"(touch));
  if (rl >= p.m) return;
  // lane: base[m = rl][n = n0 + 4 g + v]
  const uint16_t o[4] = {f32_to_bf16(acc[0]), f32_to_bf16(acc[1]), f32_to_bf16(acc[2]),
                         f32_to_bf16(acc[3])};
  store_row4(p, rl, n0 + 4 * (lane >> 4), o);
}

template <int NW, int CPW>
__global__ void __launch_bounds__(64 * NW) k_skinny_main(Skinny2Params p) {
  __shared__ f32x4_v red[(NW > 1 ? NW - 1 : 1) * 64];
  const int b = static_cast<int>(blockIdx.x);
  if (b < p.a_blocks) {
    adapter_block<NW>(p, b, red);
  } else {
    weight_block<NW, CPW>(p, b - p.a_blocks, red);
  }
}

// Thread (row n = n0 + (tid & 63), token group tid >> 6) keeps B[n, :] in
// registers (RV 16-byte vectors) and produces y[m, n] for m = tid >> 6,
// (tid >> 6) + 4, ...; h comes from the partials through LDS.
template <int RV>
__device__ __forceinline__ void finish_block(const Skinny2Params& p, int64_t block, float* hs) {
  const int tid = threadIdx.x;
  const int mr = p.m * p.rank;
  const int64_t n = block * kFinRows + (tid & 63);
  const bool nok = n < p.n;
  const int64_t nc = nok ? n : p.n - 1;
  uint32_t bw[4 * RV];
  const uint16_t* brow = p.lora_b + nc * p.rank;
  if (p.b_vec) {
#pragma unroll
    for (int v = 0; v < RV; ++v) {
      const u32x4_t q = ld16(brow + 8 * v);
      bw[4 * v] = q.x;
      bw[4 * v + 1] = q.y;
      bw[4 * v + 2] = q.z;
      bw[4 * v + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4 * RV; ++e) {
      const uint32_t lo = 2 * e < p.rank ? brow[2 * e] : 0u;
      const uint32_t hi = 2 * e + 1 < p.rank ? brow[2 * e + 1] : 0u;
      bw[e] = lo | (hi << 16);
    }
  }
  const float bias = p.bias != nullptr && nok ? bf16_to_f32(p.bias[n]) : 0.0f;
  // the thread's base values, loaded with B before the partials are summed
  constexpr int kPerThread = 16 / (kFinThreads / 64);
  uint16_t base[kPerThread];
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int m = (tid >> 6) + (kFinThreads / 64) * i;
    base[i] = m < p.m ? p.y[static_cast<int64_t>(m) * p.n + nc] : uint16_t{0};
  }
  for (int e = tid; e < mr; e += kFinThreads) {
    float sum = 0.0f;
#pragma unroll 8
    for (int s = 0; s < p.slices; ++s) sum += p.part[static_cast<int64_t>(s) * mr + e];
    const float hv = round_bf16(sum);
    hs[e] = hv;
    if (block == 0) p.h[e] = f32_to_bf16(hv);
  }
  __syncthreads();
  if (!nok) return;
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int m = (tid >> 6) + (kFinThreads / 64) * i;
    if (m >= p.m) break;
    const float* hrow = hs + m * p.rank;
    float t = 0.0f;
#pragma unroll
    for (int e = 0; e < 4 * RV; ++e) {
      if (2 * e < p.rank) t = __builtin_fmaf(hrow[2 * e], bf16lo_to_f32(bw[e]), t);
      if (2 * e + 1 < p.rank) t = __builtin_fmaf(hrow[2 * e + 1], bf16hi_to_f32(bw[e]), t);
    }
    float r = round_bf16(bf16_to_f32(base[i]) + round_bf16(round_bf16(t) * p.scale));
    if (p.bias != nullptr) r = round_bf16(r + bias);
    p.y[static_cast<int64_t>(m) * p.n + n] = f32_to_bf16(r);
  }
}

template <int RV>
__global__ void __launch_bounds__(kFinThreads) k_skinny_finish(Skinny2Params p) {
  __shared__ float hs[16 * 64];
  finish_block<RV>(p, blockIdx.x, hs);
}

// ---------------------------------------------------------------------------
// Several projections of one input in one pair of launches (the q / k / v
// or gate / up projections of a layer at small M): the first grid holds
// every projection's adapter blocks, then every projection's weight blocks;
// the finishing grid every projection's row blocks. Each block does what it
// does in the single-projection launches, on its projection's operands.
constexpr int kMaxProjections = 4;
struct Skinny2Multi {
  Skinny2Params p[kMaxProjections];
  int count;
};

template <int NW, int CPW>
__global__ void __launch_bounds__(64 * NW) k_skinny_main_multi(Skinny2Multi mp) {
  __shared__ f32x4_v red[(NW > 1 ? NW - 1 : 1) * 64];
  int64_t b = blockIdx.x;
#pragma unroll
  for (int i = 0; i < kMaxProjections; ++i) {
    if (i < mp.count) {
      if (b < mp.p[i].a_blocks) {
        adapter_block<NW>(mp.p[i], static_cast<int>(b), red);
        return;
      }
      b -= mp.p[i].a_blocks;
    }
  }
#pragma unroll
  for (int i = 0; i < kMaxProjections; ++i) {
    if (i < mp.count) {
      if (b < mp.p[i].w_blocks) {
        weight_block<NW, CPW>(mp.p[i], b, red);
        return;
      }
      b -= mp.p[i].w_blocks;
    }
  }
}

template <int RV>
__global__ void __launch_bounds__(kFinThreads) k_skinny_finish_multi(Skinny2Multi mp) {
  __shared__ float hs[16 * 64];
  int64_t b = blockIdx.x;
#pragma unroll
  for (int i = 0; i < kMaxProjections; ++i) {
    if (i < mp.count) {
      const int64_t blocks = (mp.p[i].n + kFinRows - 1) / kFinRows;
      if (b < blocks) {
        finish_block<RV>(mp.p[i], b, hs);
        return;
      }
      b -= blocks;
    }
  }
}

// ---------------------------------------------------------------------------
// One-launch form (k_skinny_one): the same two block roles, but the last
// adapter block to arrive sums the partials into h and publishes it
// (device-coherent stores, then a flag), and every weight block applies the
// LoRA term to its own rows after a bounded wait for the flag, so the
// finishing launch and its dispatch disappear. Adapter blocks come first in
// the grid and wait on nothing, so the wait ends once they have run; the
// spin limit only guarantees that every wave exits (h then reads as NaN and
// the device error word gets kDevErrSkinnyOneWait). Slots are taken in turn:
// at most kSlots calls may run at once on a device. Every call leaves its
// slot at zero, also when waits expired: the weight blocks (after their
// wait) and the publishing adapter block (after raising the flag) count into
// a done word, and the last of them clears the slot.

constexpr int kSlots2 = 8;
constexpr int kSpin2 = 1 << 22;  // default polls of the bounded wait
__device__ unsigned int g_skinny2_state[kSlots2][4];

template <int NW>
__device__ __forceinline__ void adapter_block_one(const Skinny2Params& p, int a, f32x4_v* red,
                                                  int* last_sh) {
  int s, q;
  const f32x4_v acc = adapter_partial<NW>(p, a, red, &s, &q);
  const int lane = threadIdx.x & 63;
  const int rl = lane & 15;
  if ((threadIdx.x >> 6) == 0 && rl < p.m) {
    float* dst = p.part + (static_cast<int64_t>(s) * p.m + rl) * p.rank;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int jj = 16 * q + 4 * (lane >> 4) + v;
      if (jj < p.rank) store_coherent_f32(dst + jj, acc[v]);
    }
  }
  drain_stores();
  __syncthreads();
  unsigned int* state = g_skinny2_state[p.slot];
  if (threadIdx.x == 0) *last_sh = arrive(state, static_cast<unsigned int>(p.a_blocks)) ? 1 : 0;
  __syncthreads();
  if (*last_sh == 0) return;
  // the last adapter block: h = bf16(sum over slices in slice order)
  const int mr = p.m * p.rank;
  for (int e = threadIdx.x; e < mr; e += 64 * NW) {
    float sum = 0.0f;
    for (int sl = 0; sl < p.slices; ++sl) sum += load_coherent_f32(p.part + static_cast<int64_t>(sl) * mr + e);
    const float hv = round_bf16(sum);
    store_coherent_f32(p.hf + e, hv);
    p.h[e] = f32_to_bf16(hv);
  }
  drain_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_store(state + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    drain_stores();  // the flag is visible before this block counts as done
    done_count(state, 2, 3, static_cast<unsigned int>(p.w_blocks) + 1u);
  }
}

template <int NW, int CPW>
__device__ __forceinline__ void weight_block_one(const Skinny2Params& p, int64_t b, f32x4_v* red) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rl = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = 16 * b;
  const int64_t rc = n0 + rl < p.n ? n0 + rl : p.n - 1;
  WeightFrags<CPW> f;
  weight_loads<NW, CPW>(p, n0, f);
  // wave 0 also loads its rows of B as MFMA row fragments (rank <= 64: two
  // 32-rank steps, j = 32 q + 8 g + [0, 8)) and its 4 bias values
  u32x4_t bfr[2] = {u32x4_t{0u, 0u, 0u, 0u}, u32x4_t{0u, 0u, 0u, 0u}};
  float bias4[4] = {0.f, 0.f, 0.f, 0.f};
  if (wave == 0) {
    const uint16_t* brow = p.lora_b + rc * p.rank;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int j0 = 32 * q + 8 * g;
      if (j0 >= p.rank) continue;
      if (p.b_vec && j0 + 8 <= p.rank) {
        bfr[q] = ld16(brow + j0);
      } else {
        uint32_t w4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = j0 + 2 * e < p.rank ? brow[j0 + 2 * e] : 0u;
          const uint32_t hi = j0 + 2 * e + 1 < p.rank ? brow[j0 + 2 * e + 1] : 0u;
          w4[e] = lo | (hi << 16);
        }
        bfr[q] = u32x4_t{w4[0], w4[1], w4[2], w4[3]};
      }
    }
    if (p.bias != nullptr) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t nn = n0 + 4 * g + v;
        bias4[v] = nn < p.n ? bf16_to_f32(p.bias[nn]) : 0.0f;
      }
    }
  }
  const f32x4_v acc = weight_mfma<NW, CPW>(f, red);
  if (wave != 0) return;

  // wait (lane 0, bounded) for the published h, then read it as MFMA
  // column fragments: lane (m = rl, g) takes h[m][32 q + 8 g + e]
  unsigned int* state = g_skinny2_state[p.slot];
  int ready = 1;
  if (lane == 0) {
    ready = 0;
    for (int it = 0; it < p.spin; ++it) {
      if (__hip_atomic_load(state + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
        ready = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!ready)
      __hip_atomic_fetch_or(p.err, kDevErrSkinnyOneWait, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    // past its last access to the slot
    done_count(state, 2, 3, static_cast<unsigned int>(p.w_blocks) + 1u);
  }
  ready = __shfl(ready, 0, 64);
  // the h loads below must not be issued before the flag was seen
  asm volatile("" ::: "memory");
  f32x4_v t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (32 * q >= p.rank) break;
    float hv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int jj = 32 * q + 8 * g + e;
      hv[e] = (rl < p.m && jj < p.rank) ? load_coherent_f32(p.hf + rl * p.rank + jj) : 0.0f;
      if (!ready) hv[e] = __builtin_nanf("");
    }
    const u32x4_t hfr{pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3]), pack_bf16x2(hv[4], hv[5]),
                      pack_bf16x2(hv[6], hv[7])};
    t = mfma16(bfr[q], hfr, t);
  }
  if (rl >= p.m) return;
  // lane: y[m = rl][n = n0 + 4 g + v]
  uint16_t o[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    float r = round_bf16(acc[v]);
    r = round_bf16(r + round_bf16(round_bf16(t[v]) * p.scale));
    if (p.bias != nullptr) r = round_bf16(r + bias4[v]);
    o[v] = f32_to_bf16(r);
  }
  store_row4(p, rl, n0 + 4 * g, o);
}

template <int NW, int CPW>
__global__ void __launch_bounds__(64 * NW) k_skinny_one(Skinny2Params p) {
  __shared__ f32x4_v red[(NW > 1 ? NW - 1 : 1) * 64];
  __shared__ int last_sh;
  const int b = static_cast<int>(blockIdx.x);
  if (b < p.a_blocks) {
    adapter_block_one<NW>(p, b, red, &last_sh);
  } else {
    weight_block_one<NW, CPW>(p, b - p.a_blocks, red);
  }
}

template <int NW, int CPW>
void launch_one(const Skinny2Params& p, hipStream_t stream) {
  hipLaunchKernelGGL((k_skinny_one<NW, CPW>), dim3(static_cast<unsigned>(p.a_blocks + p.w_blocks)),
                     dim3(64 * NW), 0, stream, p);
}

std::atomic<unsigned int> g_calls2{0};

// The one-launch form pays for its published h with a chain of dependent
// round trips (the adapter blocks' partials, the last one's sums, the
// flag, the weight blocks' reads) that the weight stream hides only when it
// is long: measured on the Qwen3-2B shapes at M = 1, 6144 -> 2048 takes
// 11.3 us against 13.5 us for two launches, but 2048 -> 6144 12.8 against
// 10.5 and 2048 -> 2048 9.7 against 8.2. Chosen for K >= 4096; the
// kTuneSkinny2One knob forces either form.
bool one_launch_selected(int64_t k) {
  const int force = tune(kTuneSkinny2One);
  if (force == 0) return false;
  if (force > 0) return true;
  return k >= 4096;
}

template <int NW, int CPW>
void launch_main(const Skinny2Params& p, hipStream_t stream) {
  const int64_t blocks = p.a_blocks + ceil_div(p.n, 16);
  hipLaunchKernelGGL((k_skinny_main<NW, CPW>), dim3(static_cast<unsigned>(blocks)), dim3(64 * NW),
                     0, stream, p);
}

struct Skinny2Plan {
  int nw;      // waves per block
  int cpw;     // 128-column chunks per weight wave (1, 2 or 4)
  int slices;  // adapter K slices
};

// Waves per block: enough weight blocks x waves to put ~8 waves on each of
// 256 CUs, 4 to 16 per block.
Skinny2Plan plan2(int64_t n, int64_t k) {
  Skinny2Plan p;
  const int64_t blocks = ceil_div(n, 16);
  p.nw = 4;
  while (p.nw < 16 && blocks * p.nw < 2048) p.nw *= 2;
  const int64_t c = ceil_div(k / 128, p.nw);
  p.cpw = c <= 1 ? 1 : (c <= 2 ? 2 : 4);
  p.slices = static_cast<int>(c);
  return p;
}

}  // namespace

bool skinny2_ok(int64_t m, int64_t n, int64_t k, int64_t rank, int64_t n_groups, int64_t group) {
  if (m < 1 || m > 16 || n < 1 || k % 128 != 0 || rank < 1 || rank > 64) return false;
  if (n_groups > 1 && (group < 32 || (group & (group - 1)) != 0)) return false;
  // every weight wave covers its K range in at most 4 chunks of 128 columns
  return k / 128 <= 4 * plan2(n, k).nw;
}

// Measured on the three Qwen3-2B projection shapes (group 64, rank 32,
// weights cycled beyond the 256 MB MALL): 30-40% faster than the one-launch
// kernel for M <= 4, slower at M = 16, where every weight block re-reads all
// of x and the finish handles 16 rows of y. The kTuneSkinny2 knob selects it
// for every M <= 16 (1) or never (0); a forced one-launch tile shape
// (kTuneSkinnyTile) also turns it off.
bool skinny2_selected(int64_t m, int64_t n, int64_t k, int64_t rank, int64_t n_groups,
                      int64_t group) {
  if (tune(kTuneSkinnyTile) > 0) return false;
  const int force = tune(kTuneSkinny2);
  if (force == 0) return false;
  if (force != 1 && m > 4) return false;
  return skinny2_ok(m, n, k, rank, n_groups, group);
}

int64_t skinny2_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t rank) {
  // K-slice partials of h, then the published h
  return static_cast<int64_t>(plan2(n, k).slices) * m * rank + m * rank;
}

hipError_t launch_skinny2_forward(const uint16_t* x, int64_t m, int64_t k, const Int4Operand& w,
                                  int64_t n, const uint16_t* lora_a, const uint16_t* lora_b,
                                  int64_t rank, float scale, const uint16_t* bias, uint16_t* y,
                                  uint16_t* h, float* ws, hipStream_t stream) {
  Skinny2Params p;
  p.x = x;
  p.m = static_cast<int>(m);
  p.k = k;
  p.n = n;
  p.packed = w.packed;
  p.pcols = w.packed_cols;
  p.scales = w.scales;
  p.n_groups = w.n_groups;
  p.group_shift = 0;
  if (w.n_groups > 1)
    while ((int64_t{1} << p.group_shift) < w.group) ++p.group_shift;
  p.lora_a = lora_a;
  p.lora_b = lora_b;
  p.rank = static_cast<int>(rank);
  p.scale = scale;
  p.bias = bias;
  p.y = y;
  p.h = h;
  p.part = ws;
  const Skinny2Plan pl = plan2(n, k);
  p.slices = pl.slices;
  p.a_blocks = p.slices * static_cast<int>(ceil_div(rank, 16));
  p.b_vec = (reinterpret_cast<uintptr_t>(lora_b) & 15) == 0 && rank % 8 == 0 && rank * 16 <= 512;
  p.hf = ws + static_cast<int64_t>(p.slices) * m * rank;
  p.w_blocks = static_cast<int>(ceil_div(n, 16));
  p.slot = 0;
  p.spin = tune(kTuneSpinLimit) > 0 ? tune(kTuneSpinLimit) : kSpin2;
  p.err = nullptr;
  if (one_launch_selected(k)) {
    p.err = device_error_word();
    if (p.err == nullptr) return hipErrorInvalidSymbol;
    p.slot = static_cast<int>(g_calls2.fetch_add(1, std::memory_order_relaxed) % kSlots2);
    bool one = false;
#define RPX_ONE(NW, CPW)                              \
  if (!one && pl.nw == NW && pl.cpw == CPW) {         \
    launch_one<NW, CPW>(p, stream);                   \
    one = true;                                       \
  }
    RPX_ONE(4, 1) RPX_ONE(4, 2) RPX_ONE(4, 4)
    RPX_ONE(8, 1) RPX_ONE(8, 2) RPX_ONE(8, 4)
    RPX_ONE(16, 1) RPX_ONE(16, 2) RPX_ONE(16, 4)
#undef RPX_ONE
    return one ? hipGetLastError() : hipErrorInvalidValue;
  }
  bool launched = false;
#define RPX_MAIN(NW, CPW)                             \
  if (!launched && pl.nw == NW && pl.cpw == CPW) {    \
    launch_main<NW, CPW>(p, stream);                  \
    launched = true;                                  \
  }
  RPX_MAIN(4, 1) RPX_MAIN(4, 2) RPX_MAIN(4, 4)
  RPX_MAIN(8, 1) RPX_MAIN(8, 2) RPX_MAIN(8, 4)
  RPX_MAIN(16, 1) RPX_MAIN(16, 2) RPX_MAIN(16, 4)
#undef RPX_MAIN
  if (!launched) return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 fin_grid(static_cast<unsigned>(ceil_div(n, kFinRows)));
  switch ((rank + 7) / 8) {
    case 1: hipLaunchKernelGGL(k_skinny_finish<1>, fin_grid, dim3(kFinThreads), 0, stream, p); break;
    case 2: hipLaunchKernelGGL(k_skinny_finish<2>, fin_grid, dim3(kFinThreads), 0, stream, p); break;
    case 3: hipLaunchKernelGGL(k_skinny_finish<3>, fin_grid, dim3(kFinThreads), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(k_skinny_finish<4>, fin_grid, dim3(kFinThreads), 0, stream, p); break;
    case 5: hipLaunchKernelGGL(k_skinny_finish<5>, fin_grid, dim3(kFinThreads), 0, stream, p); break;
    case 6: hipLaunchKernelGGL(k_skinny_finish<6>, fin_grid, dim3(kFinThreads), 0, stream, p); break;
    case 7: hipLaunchKernelGGL(k_skinny_finish<7>, fin_grid, dim3(kFinThreads), 0, stream, p); break;
    default: hipLaunchKernelGGL(k_skinny_finish<8>, fin_grid, dim3(kFinThreads), 0, stream, p); break;
  }
  return hipGetLastError();
}

bool skinny2_multi_ok(int64_t m, int64_t k, int count, const Skinny2Projection* proj) {
  if (count < 1 || count > kMaxProjections) return false;
  int64_t n_total = 0;
  for (int i = 0; i < count; ++i) {
    if (proj[i].rank != proj[0].rank) return false;
    if (!skinny2_ok(m, proj[i].n, k, proj[i].rank, proj[i].w.n_groups, proj[i].w.group))
      return false;
    n_total += proj[i].n;
  }
  // every weight wave covers its K range in at most 4 chunks of 128 columns
  return k / 128 <= 4 * plan2(n_total, k).nw;
}

int64_t skinny2_multi_workspace_floats(int64_t m, int64_t k, int count,
                                       const Skinny2Projection* proj) {
  int64_t n_total = 0;
  for (int i = 0; i < count; ++i) n_total += proj[i].n;
  const int64_t slices = plan2(n_total, k).slices;
  int64_t floats = 0;
  for (int i = 0; i < count; ++i) floats += slices * m * proj[i].rank;
  return floats;
}

hipError_t launch_skinny2_forward_multi(const uint16_t* x, int64_t m, int64_t k, int count,
                                        const Skinny2Projection* proj, float* ws,
                                        hipStream_t stream) {
  int64_t n_total = 0;
  for (int i = 0; i < count; ++i) n_total += proj[i].n;
  // one block shape for the whole grid, planned for all rows together
  const Skinny2Plan pl = plan2(n_total, k);
  Skinny2Multi mp{};
  mp.count = count;
  int64_t a_total = 0, w_total = 0, fin_total = 0;
  float* part = ws;
  for (int i = 0; i < count; ++i) {
    const Skinny2Projection& q = proj[i];
    Skinny2Params& p = mp.p[i];
    p.x = x;
    p.m = static_cast<int>(m);
    p.k = k;
    p.n = q.n;
    p.packed = q.w.packed;
    p.pcols = q.w.packed_cols;
    p.scales = q.w.scales;
    p.n_groups = q.w.n_groups;
    p.group_shift = 0;
    if (q.w.n_groups > 1)
      while ((int64_t{1} << p.group_shift) < q.w.group) ++p.group_shift;
    p.lora_a = q.lora_a;
    p.lora_b = q.lora_b;
    p.rank = static_cast<int>(q.rank);
    p.scale = q.scale;
    p.bias = q.bias;
    p.y = q.y;
    p.h = q.h;
    p.part = part;
    p.slices = pl.slices;
    p.a_blocks = p.slices * static_cast<int>(ceil_div(q.rank, 16));
    p.b_vec = (reinterpret_cast<uintptr_t>(q.lora_b) & 15) == 0 && q.rank % 8 == 0 &&
              q.rank * 16 <= 512;
    p.hf = nullptr;
    p.w_blocks = static_cast<int>(ceil_div(q.n, 16));
    p.slot = 0;
    p.spin = 0;
    p.err = nullptr;
    part += static_cast<int64_t>(pl.slices) * m * q.rank;
    a_total += p.a_blocks;
    w_total += p.w_blocks;
    fin_total += ceil_div(q.n, kFinRows);
  }
  const dim3 main_grid(static_cast<unsigned>(a_total + w_total));
  bool launched = false;
#define RPX_MULTI(NW, CPW)                                                                  \
  if (!launched && pl.nw == NW && pl.cpw == CPW) {                                          \
    hipLaunchKernelGGL((k_skinny_main_multi<NW, CPW>), main_grid, dim3(64 * NW), 0, stream, mp); \
    launched = true;                                                                        \
  }
  RPX_MULTI(4, 1) RPX_MULTI(4, 2) RPX_MULTI(4, 4)
  RPX_MULTI(8, 1) RPX_MULTI(8, 2) RPX_MULTI(8, 4)
  RPX_MULTI(16, 1) RPX_MULTI(16, 2) RPX_MULTI(16, 4)
#undef RPX_MULTI
  if (!launched) return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 fin_grid(static_cast<unsigned>(fin_total));
  switch ((proj[0].rank + 7) / 8) {
    case 1: hipLaunchKernelGGL(k_skinny_finish_multi<1>, fin_grid, dim3(kFinThreads), 0, stream, mp); break;
    case 2: hipLaunchKernelGGL(k_skinny_finish_multi<2>, fin_grid, dim3(kFinThreads), 0, stream, mp); break;
    case 3: hipLaunchKernelGGL(k_skinny_finish_multi<3>, fin_grid, dim3(kFinThreads), 0, stream, mp); break;
    case 4: hipLaunchKernelGGL(k_skinny_finish_multi<4>, fin_grid, dim3(kFinThreads), 0, stream, mp); break;
    case 5: hipLaunchKernelGGL(k_skinny_finish_multi<5>, fin_grid, dim3(kFinThreads), 0, stream, mp); break;
    case 6: hipLaunchKernelGGL(k_skinny_finish_multi<6>, fin_grid, dim3(kFinThreads), 0, stream, mp); break;
    case 7: hipLaunchKernelGGL(k_skinny_finish_multi<7>, fin_grid, dim3(kFinThreads), 0, stream, mp); break;
    default: hipLaunchKernelGGL(k_skinny_finish_multi<8>, fin_grid, dim3(kFinThreads), 0, stream, mp); break;
  }
  return hipGetLastError();
}

}  // namespace rpx
