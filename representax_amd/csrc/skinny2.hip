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
  // one-launch form: the call's slot, the host's call count (mixed into the
  // tag), the polls of the bounded wait and the device error word
  int slot;
  int proj;  // -1, or the projection's index in a shared-input call
  unsigned int tag;
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

// 8 bf16 of x row m from column k. Every fragment load is unconditional
// (rows past M read row M - 1; for chunks past K callers pass a column of
// the first chunk) and keep() turns the fragments that lie outside x (or
// outside the weight) into zeros where they are used: a load under a
// branch made the compiler wait for it inside the branch, which put a full
// memory round trip between a wave's first loads and the rest.
__device__ __forceinline__ u32x4_t x_load(const Skinny2Params& p, int m, int64_t k) {
  return ld16(p.x + static_cast<int64_t>(m < p.m ? m : p.m - 1) * p.k + k);
}

__device__ __forceinline__ u32x4_t keep(u32x4_t v, bool ok) {
  return ok ? v : u32x4_t{0u, 0u, 0u, 0u};
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

// One-launch form state (k_skinny_one, described further down).
constexpr int kSlots2 = 8;
constexpr int kSpin2 = 1 << 22;  // default polls of the bounded wait
constexpr int kOneMaxM = 4;      // rows of x the one-launch form takes
// partial words of a slot: [slice][m][rank], slices <= 4, rank <= 64
constexpr int kOneWords = 4 * kOneMaxM * 64;
constexpr int kOnePerLane = kOneWords / 64;
constexpr int kMaxProjections = 4;
__device__ unsigned long long g_skinny2_words[kSlots2][kOneWords];
// the shared-input calls' own slots, one set of words per projection
__device__ unsigned long long g_skinny2_multi_words[kSlots2][kMaxProjections][kOneWords];

__device__ __forceinline__ unsigned long long* slot_words(const Skinny2Params& p) {
  return p.proj < 0 ? g_skinny2_words[p.slot] : g_skinny2_multi_words[p.slot][p.proj];
}

__device__ __forceinline__ unsigned int call_tag(const Skinny2Params& p) { return launch_tag(p.tag); }

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
  const int64_t k0 = (ok ? c * 128 : 0) + 32 * g;
  u32x4_t av[4], xv[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    av[st] = ld16(arow + k0 + 8 * st);
    xv[st] = x_load(p, rl, k0 + 8 * st);
  }
  const bool aok = ok && jok;
  const bool xok = ok && rl < p.m;
  f32x4_v acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < 4; ++st) acc = mfma16(keep(av[st], aok), keep(xv[st], xok), acc);
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
    const int64_t k0 = (ok ? c * 128 : 0) + 32 * g;
    f.wv[i] = ld16(wrow + k0 / 2);
    f.sv[i] = srow[p.n_groups == 1 ? 0 : (k0 >> p.group_shift)];
#pragma unroll
    for (int st = 0; st < 4; ++st) f.xv[i][st] = x_load(p, rl, k0 + 8 * st);
  }
}

// Dequantized MFMAs over the wave's loaded chunks (chunks past K and rows
// past M as zeros).
template <int NW, int CPW>
__device__ __forceinline__ f32x4_v weight_partial(const Skinny2Params& p, const WeightFrags<CPW>& f) {
  const int wave = threadIdx.x >> 6;
  const bool mok = (threadIdx.x & 15) < p.m;
  f32x4_v acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const bool ok = wave + static_cast<int64_t>(i) * NW < p.k / 128;
    const float s = bf16_to_f32(f.sv[i]);
    const u32x4_t w = keep(f.wv[i], ok);
#pragma unroll
    for (int st = 0; st < 4; ++st)
      acc = mfma16(dequant8(w[st], s), keep(f.xv[i][st], ok && mok), acc);
  }
  return acc;
}

// The same, summed over the waves in wave order: valid in wave 0, lane l
// holding D[n0 + 4 (l >> 4) + v][m = l & 15].
template <int NW, int CPW>
__device__ __forceinline__ f32x4_v weight_mfma(const Skinny2Params& p, const WeightFrags<CPW>& f,
                                               f32x4_v* red) {
  return reduce_waves<NW>(weight_partial<NW, CPW>(p, f), red);
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
  const f32x4_v acc = weight_mfma<NW, CPW>(p, f, red);
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
// The one-launch form of the same grid (k_skinny_one_multi) is further down.
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
// One-launch form (k_skinny_one): the same two block roles, but the adapter
// blocks hand their partials straight to the weight blocks, so the
// finishing launch and its dispatch disappear. Each partial travels as one
// 64-bit word (the f32 bits, and the call's 32-bit tag above them) written
// with a single device-coherent store into the call's slot; a weight block
// polls the words it needs until every one carries the call's tag, sums
// them in slice order into h and applies the LoRA term to its own rows.
//
// The tag is a hash of the dispatch (its dispatch id, which the command
// processor counts up per queue, and the address of its packet, which
// tells queues apart) and of the host's call count, so every launch,
// graph replays included, carries its own tag without any block having to
// count in, and a word left in the slot by an earlier launch is taken for
// this one's only if their 32-bit tags collide. Tags are never zero, the
// value of a fresh slot's words. Adapter blocks come first in the grid and
// wait on nothing, so the wait ends once they have run; the spin limit
// only guarantees that every wave exits (h then reads as NaN and the device
// error word gets kDevErrSkinnyOneWait). Slots are taken in turn: at most
// kSlots2 calls may run at once on a device.

template <int NW>
__device__ __forceinline__ void adapter_block_one(const Skinny2Params& p, int a, f32x4_v* red) {
  int s, q;
  const f32x4_v acc = adapter_partial<NW>(p, a, red, &s, &q);
  if ((threadIdx.x >> 6) != 0) return;
  const unsigned long long tag = static_cast<unsigned long long>(call_tag(p)) << 32;
  const int lane = threadIdx.x & 63;
  const int rl = lane & 15;
  if (rl >= p.m) return;
  unsigned long long* dst = slot_words(p) + (s * p.m + rl) * p.rank;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int jj = 16 * q + 4 * (lane >> 4) + v;
    // (the element goes through a scalar first: a bit cast of a vector
    // element operand compiled to element 0 for every v)
    const float val = acc[v];
    if (jj < p.rank)
      __hip_atomic_store(dst + jj, tag | __builtin_bit_cast(unsigned int, val), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Wave 0 of a weight block: every partial word of the call, polled until
// all carry the call's tag (bounded), into pv[slice][m][rank]. Returns
// whether the wait succeeded; on expiry the values are NaN.
__device__ __forceinline__ bool poll_partials(const Skinny2Params& p, unsigned int tag, float* pv) {
  const int lane = threadIdx.x & 63;
  const int words = p.slices * p.m * p.rank;
  const unsigned long long* src = slot_words(p);
  // every lane's loads go out at once (indices past the call's words read
  // word 0 and are ignored)
  unsigned long long w[kOnePerLane];
#pragma unroll
  for (int u = 0; u < kOnePerLane; ++u) {
    const int e = lane + 64 * u;
    w[u] = __hip_atomic_load(const_cast<unsigned long long*>(src) + (e < words ? e : 0),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  auto missing = [&]() {
    bool miss = false;
#pragma unroll
    for (int u = 0; u < kOnePerLane; ++u)
      miss |= lane + 64 * u < words && static_cast<unsigned int>(w[u] >> 32) != tag;
    return miss;
  };
  bool ready = __ballot(missing()) == 0;
  for (int it = 0; !ready && it < p.spin; ++it) {
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int u = 0; u < kOnePerLane; ++u) {
      const int e = lane + 64 * u;
      if (e < words && static_cast<unsigned int>(w[u] >> 32) != tag)
        w[u] = __hip_atomic_load(const_cast<unsigned long long*>(src) + e, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    }
    ready = __ballot(missing()) == 0;
  }
  if (!ready && lane == 0)
    __hip_atomic_fetch_or(p.err, kDevErrSkinnyOneWait, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int u = 0; u < kOnePerLane; ++u) {
    const int e = lane + 64 * u;
    if (e < words)
      pv[e] = ready ? __builtin_bit_cast(float, static_cast<unsigned int>(w[u])) : __builtin_nanf("");
  }
  return ready;
}

template <int NW, int CPW>
__device__ __forceinline__ void weight_block_one(const Skinny2Params& p, int64_t b, f32x4_v* red,
                                                 float* pv) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rl = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = 16 * b;
  const int64_t rc = n0 + rl < p.n ? n0 + rl : p.n - 1;
  WeightFrags<CPW> f;
  weight_loads<NW, CPW>(p, n0, f);
  // every wave also loads its rows of B as MFMA row fragments (rank <= 64,
  // a multiple of 8: two 32-rank steps, j = 32 q + 8 g + [0, 8); steps past
  // the rank read j = 0 and become zeros) and its 4 bias values; wave 0
  // uses them. All loads are unconditional.
  const uint16_t* brow = p.lora_b + rc * p.rank;
  u32x4_t bfr[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int j0 = 32 * q + 8 * g;
    bfr[q] = ld16(brow + (j0 < p.rank ? j0 : 0));
  }
  // (without a bias the loads read B and are ignored)
  const uint16_t* bias_src = p.bias != nullptr ? p.bias : p.lora_b;
  uint16_t bias_raw[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t nn = n0 + 4 * g + v;
    bias_raw[v] = bias_src[nn < p.n ? nn : p.n - 1];
  }
  const f32x4_v acc = weight_mfma<NW, CPW>(p, f, red);
  if (wave != 0) return;

  poll_partials(p, call_tag(p), pv);
  // h = bf16(sum over slices in slice order) as MFMA column fragments: lane
  // (m = rl, g) takes h[m][32 q + 8 g + e]; block 0 also stores h
  f32x4_v t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (32 * q >= p.rank) break;
    float hv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int jj = 32 * q + 8 * g + e;
      float sum = 0.0f;
      if (rl < p.m && jj < p.rank) {
        for (int sl = 0; sl < p.slices; ++sl) sum += pv[(sl * p.m + rl) * p.rank + jj];
        if (b == 0) p.h[rl * p.rank + jj] = f32_to_bf16(round_bf16(sum));
      }
      hv[e] = round_bf16(sum);
    }
    const u32x4_t hfr{pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3]), pack_bf16x2(hv[4], hv[5]),
                      pack_bf16x2(hv[6], hv[7])};
    t = mfma16(keep(bfr[q], 32 * q + 8 * g < p.rank), hfr, t);
  }
  if (rl >= p.m) return;
  // lane: y[m = rl][n = n0 + 4 g + v]
  uint16_t o[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    float r = round_bf16(acc[v]);
    r = round_bf16(r + round_bf16(round_bf16(t[v]) * p.scale));
    if (p.bias != nullptr) r = round_bf16(r + bf16_to_f32(bias_raw[v]));
    o[v] = f32_to_bf16(r);
  }
  store_row4(p, rl, n0 + 4 * g, o);
}

template <int NW, int CPW>
__global__ void __launch_bounds__(64 * NW) k_skinny_one(Skinny2Params p) {
  __shared__ f32x4_v red[(NW > 1 ? NW - 1 : 1) * 64];
  __shared__ float pv[kOneWords];
  const int b = static_cast<int>(blockIdx.x);
  if (b < p.a_blocks) {
    adapter_block_one<NW>(p, b, red);
  } else {
    weight_block_one<NW, CPW>(p, b - p.a_blocks, red, pv);
  }
}

// Several projections of one input in one launch: every projection's
// adapter blocks, then every projection's weight blocks, each doing what it
// does in k_skinny_one with its projection's operands and words.
template <int NW, int CPW>
__global__ void __launch_bounds__(64 * NW) k_skinny_one_multi(Skinny2Multi mp) {
  __shared__ f32x4_v red[(NW > 1 ? NW - 1 : 1) * 64];
  __shared__ float pv[kOneWords];
  int64_t b = blockIdx.x;
#pragma unroll
  for (int i = 0; i < kMaxProjections; ++i) {
    if (i < mp.count) {
      if (b < mp.p[i].a_blocks) {
        adapter_block_one<NW>(mp.p[i], static_cast<int>(b), red);
        return;
      }
      b -= mp.p[i].a_blocks;
    }
  }
#pragma unroll
  for (int i = 0; i < kMaxProjections; ++i) {
    if (i < mp.count) {
      if (b < mp.p[i].w_blocks) {
        weight_block_one<NW, CPW>(mp.p[i], b, red, pv);
        return;
      }
      b -= mp.p[i].w_blocks;
    }
  }
}

template <int NW, int CPW>
void launch_one(const Skinny2Params& p, hipStream_t stream) {
  hipLaunchKernelGGL((k_skinny_one<NW, CPW>), dim3(static_cast<unsigned>(p.a_blocks + p.w_blocks)),
                     dim3(64 * NW), 0, stream, p);
}

std::atomic<unsigned int> g_calls2{0};
std::atomic<unsigned int> g_calls2_multi{0};

// The one-launch form is the default for M <= 4 (rank a multiple of 8, B
// 16-byte aligned): the weight blocks' one poll of the tagged partials
// replaces the finishing launch. Measured on the Qwen3-2B shapes at M = 1
// (rank 32, group 64, weights cycled beyond the MALL, graph of 96 calls):
// 2048 -> 6144 8.5 us against 9.9 us for two launches, 6144 -> 2048 11.2
// against 13.0, 2048 -> 2048 7.5 against 8.0. The kTuneSkinny2One knob
// forces two launches (0).
bool one_launch_selected(int64_t m, bool b_frag) {
  if (m > kOneMaxM || !b_frag) return false;
  return tune(kTuneSkinny2One) != 0;
}

template <int NW, int CPW>
void launch_main(const Skinny2Params& p, hipStream_t stream) {
  const int64_t blocks = p.a_blocks + ceil_div(p.n, 16);
  hipLaunchKernelGGL((k_skinny_main<NW, CPW>), dim3(static_cast<unsigned>(blocks)), dim3(64 * NW),
                     0, stream, p);
}

struct Skinny2Plan {
  int nw;      // waves per block
  int cpw;     // 128-column chunks per weight wave (1 to 4)
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
  p.cpw = static_cast<int>(c);
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
  // K-slice partials of h (the two-launch form)
  return static_cast<int64_t>(plan2(n, k).slices) * m * rank;
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
  p.w_blocks = static_cast<int>(ceil_div(n, 16));
  p.slot = 0;
  p.proj = -1;
  p.tag = 0;
  p.spin = tune(kTuneSpinLimit) > 0 ? tune(kTuneSpinLimit) : kSpin2;
  p.err = nullptr;
  // the one-launch weight blocks load B rows as 16-byte MFMA fragments
  const bool b_frag = (reinterpret_cast<uintptr_t>(lora_b) & 15) == 0 && rank % 8 == 0;
  if (one_launch_selected(m, b_frag)) {
    p.err = device_error_word();
    if (p.err == nullptr) return hipErrorInvalidSymbol;
    p.tag = g_calls2.fetch_add(1, std::memory_order_relaxed);
    p.slot = static_cast<int>(p.tag % kSlots2);
    bool one = false;
#define RPX_ONE(NW, CPW)                              \
  if (!one && pl.nw == NW && pl.cpw == CPW) {         \
    launch_one<NW, CPW>(p, stream);                   \
    one = true;                                       \
  }
    RPX_ONE(4, 1) RPX_ONE(4, 2) RPX_ONE(4, 3) RPX_ONE(4, 4)
    RPX_ONE(8, 1) RPX_ONE(8, 2) RPX_ONE(8, 3) RPX_ONE(8, 4)
    RPX_ONE(16, 1) RPX_ONE(16, 2) RPX_ONE(16, 3) RPX_ONE(16, 4)
#undef RPX_ONE
    return one ? hipGetLastError() : hipErrorInvalidValue;
  }
  bool launched = false;
#define RPX_MAIN(NW, CPW)                             \
  if (!launched && pl.nw == NW && pl.cpw == CPW) {    \
    launch_main<NW, CPW>(p, stream);                  \
    launched = true;                                  \
  }
  RPX_MAIN(4, 1) RPX_MAIN(4, 2) RPX_MAIN(4, 3) RPX_MAIN(4, 4)
  RPX_MAIN(8, 1) RPX_MAIN(8, 2) RPX_MAIN(8, 3) RPX_MAIN(8, 4)
  RPX_MAIN(16, 1) RPX_MAIN(16, 2) RPX_MAIN(16, 3) RPX_MAIN(16, 4)
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
    p.w_blocks = static_cast<int>(ceil_div(q.n, 16));
    p.slot = 0;
    p.proj = i;
    p.tag = 0;
    p.spin = tune(kTuneSpinLimit) > 0 ? tune(kTuneSpinLimit) : kSpin2;
    p.err = nullptr;
    part += static_cast<int64_t>(pl.slices) * m * q.rank;
    a_total += p.a_blocks;
    w_total += p.w_blocks;
    fin_total += ceil_div(q.n, kFinRows);
  }
  const dim3 main_grid(static_cast<unsigned>(a_total + w_total));
  bool one = true;
  for (int i = 0; i < count; ++i) {
    const bool b_frag =
        (reinterpret_cast<uintptr_t>(proj[i].lora_b) & 15) == 0 && proj[i].rank % 8 == 0;
    one = one && one_launch_selected(m, b_frag);
  }
  if (one) {
    unsigned int* err = device_error_word();
    if (err == nullptr) return hipErrorInvalidSymbol;
    const unsigned int tag = g_calls2_multi.fetch_add(1, std::memory_order_relaxed);
    for (int i = 0; i < count; ++i) {
      mp.p[i].err = err;
      mp.p[i].tag = tag;
      mp.p[i].slot = static_cast<int>(tag % kSlots2);
    }
    bool launched_one = false;
#define RPX_ONE_MULTI(NW, CPW)                                                                  \
  if (!launched_one && pl.nw == NW && pl.cpw == CPW) {                                          \
    hipLaunchKernelGGL((k_skinny_one_multi<NW, CPW>), main_grid, dim3(64 * NW), 0, stream, mp); \
    launched_one = true;                                                                        \
  }
    RPX_ONE_MULTI(4, 1) RPX_ONE_MULTI(4, 2) RPX_ONE_MULTI(4, 3) RPX_ONE_MULTI(4, 4)
    RPX_ONE_MULTI(8, 1) RPX_ONE_MULTI(8, 2) RPX_ONE_MULTI(8, 3) RPX_ONE_MULTI(8, 4)
    RPX_ONE_MULTI(16, 1) RPX_ONE_MULTI(16, 2) RPX_ONE_MULTI(16, 3) RPX_ONE_MULTI(16, 4)
#undef RPX_ONE_MULTI
    return launched_one ? hipGetLastError() : hipErrorInvalidValue;
  }
  bool launched = false;
#define RPX_MULTI(NW, CPW)                                                                  \
  if (!launched && pl.nw == NW && pl.cpw == CPW) {                                          \
    hipLaunchKernelGGL((k_skinny_main_multi<NW, CPW>), main_grid, dim3(64 * NW), 0, stream, mp); \
    launched = true;                                                                        \
  }
  RPX_MULTI(4, 1) RPX_MULTI(4, 2) RPX_MULTI(4, 3) RPX_MULTI(4, 4)
  RPX_MULTI(8, 1) RPX_MULTI(8, 2) RPX_MULTI(8, 3) RPX_MULTI(8, 4)
  RPX_MULTI(16, 1) RPX_MULTI(16, 2) RPX_MULTI(16, 3) RPX_MULTI(16, 4)
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
