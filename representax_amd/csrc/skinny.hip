// Skinny-M INT4 + LoRA forward (M <= 64 tokens): the memory-bound inference
// regime where every call streams the whole packed weight for a few rows.
//
// One launch. Blocks of 4 waves:
//   adapter blocks (one per K split, first in the grid): fp32 partials of
//     h = x A^T over the split's columns;
//   weight blocks (row tile x K split): every wave issues all of its 16-byte
//     packed-weight loads (and their scales) before any arithmetic, so the
//     whole weight is in flight at once; then dequantizes exactly
//     (bf16(q * s)) and runs v_mfma_f32_16x16x32_bf16 with the weight rows as
//     the row operand and x as the column operand. Waves that split the
//     block's K range are reduced through LDS in a fixed order.
// Partials go to the workspace through device-coherent stores. Arrival
// counters (a small per-device array, one slot per call in flight) pick the
// last adapter block to arrive, which sums the adapter partials in split
// order into one fp32 h, and the finisher of each row tile: the last of the
// tile's K-split blocks, which waits (bounded) until that sum has arrived,
// sums the weight partials in split order and applies the reference's
// rounding points: h = bf16(.),
// base = bf16(.), t = bf16(h B^T), y = bf16(base + bf16(t * c)) (+ bias,
// rounded again). Results do not depend on arrival order. Calls take the
// counter slots in turn, so at most kSlots calls may run at once on a device
// (kernels of one stream never overlap).
//
// Slot words return to zero at the end of every call, also when a wait
// timed out: the adapter blocks and the tile finishers each count once more
// into a "done" word after their last access to the slot, and whichever of
// them counts last clears the slot. A finisher whose wait expired poisons h
// (NaN) and raises a bit in the device error word.
#include <atomic>
#include <cstdlib>

#include "coherent.h"
#include "common.h"
#include "kernels.h"
#include "tuning.h"

namespace rpx {

namespace {

constexpr int kMaxTiles = 1024;
constexpr int kSlots = 8;
constexpr int kAdapterSpan = 256;  // columns of x A^T per adapter block
constexpr int kSpinLimit = 1 << 22;  // default polls of the bounded wait

struct SkinnyParams {
  const uint16_t* x;  // [M, K] bf16
  int m;
  int rank;
  int64_t k, n;
  const uint8_t* packed;   // [N, K/2]
  int64_t pcols;
  const uint16_t* scales;  // [N, n_groups] bf16
  int64_t n_groups;
  int group_shift;         // log2(group) when n_groups > 1
  int b_vec;               // lora_b rows load as 16-byte vectors
  const uint16_t* lora_a;  // [r, K] bf16
  const uint16_t* lora_b;  // [N, r] bf16
  float scale;
  const uint16_t* bias;    // [N] bf16 bits or null
  uint16_t* y;             // [M, N]
  uint16_t* h;             // [M, r]
  int64_t tiles;           // row tiles
  int64_t splits;          // K splits of the weight
  int64_t kspan;           // columns per weight split
  int64_t a_splits;        // adapter blocks (kAdapterSpan columns each)
  float* part_w;           // [splits][tiles][frags][64][4]
  float* part_h;           // [a_splits][4][MB][64][4]
  float* h_sum;            // [4][MB][64][4]: the partials summed in split order
  int slot;               // counter slot of this call
  int spin;               // polls of the bounded wait
  unsigned int* err;      // device error word (kDevErrSkinnyWait on timeout)
};

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// Exact dequant of one packed dword (8 nibbles, k ascending) into 4 bf16
// pairs: bf16((nibble ^ 8) * s - 8 s), the product being exact in fp32.
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

// Arrival counters, one slot per call in flight (calls take the slots in
// turn): [0] adapter blocks (one count each, and one more from the last of
// them once the summed h is stored), [1] done (adapter blocks and tile finishers past
// their last access to the slot), [2 + t] K splits of tile t. They are zero
// when the module loads and every call leaves its slot at zero.
__device__ unsigned int g_skinny_counters[kSlots][kMaxTiles + 2];

__device__ __forceinline__ u32x4_t load16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// x fragment for MFMA column m, columns [k, k + 8); zero past the last row.
__device__ __forceinline__ u32x4_t x_frag(const SkinnyParams& p, int m, int64_t k) {
  const int mc = m < p.m ? m : p.m - 1;
  const u32x4_t v = load16(p.x + static_cast<int64_t>(mc) * p.k + k);
  return m < p.m ? v : u32x4_t{0u, 0u, 0u, 0u};
}

// Weight block: rows [tile * 16 T WR, +16 T WR) x columns of `split`.
// Wave (wr, wk) takes rows wr * 16 T + [0, 16 T) and columns
// split * kspan + wk * 128 U + [0, 128 U). Within a 128-column unit, lane
// (rl, g) loads row rl's bytes for columns 32 g + [0, 32), and MFMA step st
// consumes its columns 32 g + 8 st + [0, 8), matched by the x fragment.
// Branch-free: units past K read a clamped address and are zeroed, so every
// load of the wave is issued before the first wait.
template <int MB, int T, int U, int WK>
__device__ __forceinline__ void weight_part(const SkinnyParams& p, int64_t tile, int64_t split,
                                            f32x4_t* red, uint16_t* b_lds) {
  constexpr int WR = 4 / WK;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = wave / WK;
  const int wk = wave % WK;
  const int rl = lane & 15;
  const int g = lane >> 4;
  const int64_t row0 = tile * (16 * T * WR) + wr * (16 * T);
  const int64_t kw = split * p.kspan + wk * (128 * U);

  u32x4_t wv[T][U];
  float sv[T][U];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t row = row0 + 16 * t + rl;
    const bool row_ok = row < p.n;
    const int64_t rc = row_ok ? row : p.n - 1;
    const uint8_t* wrow = p.packed + rc * p.pcols;
    const uint16_t* srow = p.scales + rc * p.n_groups;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = row_ok && kw + 128 * u < p.k;
      const int64_t kk = ok ? kw + 128 * u + 32 * g : 0;
      const u32x4_t v = load16(wrow + kk / 2);
      wv[t][u] = ok ? v : u32x4_t{0u, 0u, 0u, 0u};
      const float s = bf16_to_f32(srow[p.n_groups == 1 ? 0 : (kk >> p.group_shift)]);
      sv[t][u] = ok ? s : 0.0f;
    }
  }
  u32x4_t xf[U][4][MB];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool uok = kw + 128 * u < p.k;
    const int64_t kb = uok ? kw + 128 * u : 0;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const u32x4_t v = x_frag(p, 16 * mb + rl, kb + 32 * g + 8 * st);
        xf[u][st][mb] = uok ? v : u32x4_t{0u, 0u, 0u, 0u};
      }
  }

  // the tile's rows of B, for the block that ends up finishing the tile
  constexpr int ROWS = 16 * T * WR;
  constexpr int BV = (ROWS * 8 + 255) / 256;
  const int r = p.rank;
  const int per_row = r / 8;
  u32x4_t bv[BV];
#pragma unroll
  for (int i = 0; i < BV; ++i) {
    const int v = tid + 256 * i;
    const int brow = per_row > 0 ? v / per_row : 0;
    const int64_t n = tile * ROWS + brow;
    const bool ok = p.b_vec && v < ROWS * per_row && n < p.n;
    const u32x4_t w = load16(p.lora_b + (ok ? n * r + 8 * (v - brow * per_row) : 0));
    bv[i] = ok ? w : u32x4_t{0u, 0u, 0u, 0u};
  }

  f32x4_t acc[T][MB];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[t][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float s = sv[t][u];
      uint32_t dq[16];
#pragma unroll
      for (int d = 0; d < 4; ++d) dequant8_exact(wv[t][u][d], s, -8.0f * s, dq + 4 * d);
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const bf16x8_t af =
            as_bf16x8(u32x4_t{dq[4 * st], dq[4 * st + 1], dq[4 * st + 2], dq[4 * st + 3]});
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[t][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, as_bf16x8(xf[u][st][mb]),
                                                              acc[t][mb], 0, 0, 0);
      }
    }
  }

  if (p.b_vec) {
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int v = tid + 256 * i;
      if (v < ROWS * per_row) {
        const int brow = v / per_row;
        *reinterpret_cast<u32x4_t*>(b_lds + brow * (r + 8) + 8 * (v - brow * per_row)) = bv[i];
      }
    }
  }

  if constexpr (WK > 1) {
    if (wk > 0) {
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          red[((((wk - 1) * WR + wr) * T + t) * MB + mb) * 64 + lane] = acc[t][mb];
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int j = 1; j < WK; ++j)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[t][mb] += red[((((j - 1) * WR + wr) * T + t) * MB + mb) * 64 + lane];
    }
  }
  if (wk == 0) {
    constexpr int F = WR * T * MB;
    f32x4_t* dst = reinterpret_cast<f32x4_t*>(p.part_w) + (split * p.tiles + tile) * F * 64;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        if (16 * mb + rl < p.m) store_coherent(dst + ((wr * T + t) * MB + mb) * 64, lane, acc[t][mb]);
  }
}

// Adapter block: fp32 partial of h[m, j] = sum_k x[m, k] A[j, k] over
// columns [a_split * 256, +256); wave w takes j in [16 w, 16 w + 16). The
// lane holds D[j = 16 w + 4 g + v][m = 16 mb + rl].
template <int MB>
__device__ __forceinline__ void adapter_part(const SkinnyParams& p, int64_t a_split) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int rl = lane & 15;
  const int g = lane >> 4;
  if (16 * wave >= p.rank) return;
  const int j = 16 * wave + rl;
  const bool jok = j < p.rank;
  const uint16_t* arow = p.lora_a + static_cast<int64_t>(jok ? j : p.rank - 1) * p.k;
  const int64_t k0 = a_split * kAdapterSpan;
  u32x4_t av[kAdapterSpan / 32];
  u32x4_t xv[kAdapterSpan / 32][MB];
#pragma unroll
  for (int s = 0; s < kAdapterSpan / 32; ++s) {
    const bool ok = k0 + 32 * s < p.k;
    const int64_t kk = ok ? k0 + 32 * s + 8 * g : 0;
    const u32x4_t v = load16(arow + kk);
    av[s] = ok && jok ? v : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const u32x4_t w = x_frag(p, 16 * mb + rl, kk);
      xv[s][mb] = ok ? w : u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  f32x4_t acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kAdapterSpan / 32; ++s)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[s]), as_bf16x8(xv[s][mb]),
                                                       acc[mb], 0, 0, 0);
  f32x4_t* dst = reinterpret_cast<f32x4_t*>(p.part_h) + a_split * (4 * MB * 64);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    if (16 * mb + rl < p.m) store_coherent(dst + (wave * MB + mb) * 64, lane, acc[mb]);
}

// The last adapter block of a call: h = the adapter partials summed in split
// order (fp32, from zero), one fragment set that every tile finisher loads
// instead of summing all a_splits partials itself.
template <int MB>
__device__ __forceinline__ void adapter_sum(const SkinnyParams& p) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (16 * wave >= p.rank) return;
  const f32x4_t* part_h = reinterpret_cast<const f32x4_t*>(p.part_h);
  f32x4_t acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
  for (int64_t sp = 0; sp < p.a_splits; ++sp) {
    f32x4_t v[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) v[mb] = load_coherent(part_h + (sp * 4 * MB + wave * MB + mb) * 64, lane);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] += v[mb];
  }
  f32x4_t* dst = reinterpret_cast<f32x4_t*>(p.h_sum);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) store_coherent(dst + (wave * MB + mb) * 64, lane, acc[mb]);
}

// Outputs of one row tile. Each lane sums (in split order) the weight
// fragments it would have written and, in waves below rank / 16, loads the
// summed h fragments (issued first). h = bf16(.) goes to LDS
// as fp32 (row stride rank + 1) and as bf16 (row stride rank + 8); the
// tile's rows of B are in LDS (row stride rank + 8) when they load as
// vectors, and then t = h B^T of each fragment is one 16x16x32 MFMA per 32
// ranks (B rows as the row operand, h rows as the column operand), which
// leaves t in the fragment's own layout, D[n = 4 g + v][m = rl].
template <int MB, int T, int WK>
__device__ __forceinline__ void finish_tile(const SkinnyParams& p, int64_t tile, float* h_lds,
                                            uint16_t* hb_lds, const uint16_t* b_lds, bool poison) {
  constexpr int WR = 4 / WK;
  constexpr int F = WR * T * MB;
  constexpr int FI = (F + 3) / 4;
  constexpr int ROWS = 16 * T * WR;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int rl = lane & 15;
  const int g = lane >> 4;
  const int r = p.rank;
  const bool h_wave = 16 * wave < r;
  const f32x4_t* part = reinterpret_cast<const f32x4_t*>(p.part_w);
  const f32x4_t* h_sum = reinterpret_cast<const f32x4_t*>(p.h_sum);
  const int hw = h_wave ? wave : 0;
  f32x4_t hacc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) hacc[mb] = load_coherent(h_sum + (hw * MB + mb) * 64, lane);
  f32x4_t wacc[FI];
#pragma unroll
  for (int i = 0; i < FI; ++i) wacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
  for (int64_t sp = 0; sp < p.splits; ++sp) {
    f32x4_t vw[FI];
#pragma unroll
    for (int i = 0; i < FI; ++i) {
      const int f = wave + 4 * i < F ? wave + 4 * i : 0;
      vw[i] = load_coherent(part + ((sp * p.tiles + tile) * F + f) * 64, lane);
    }
#pragma unroll
    for (int i = 0; i < FI; ++i) wacc[i] += vw[i];
  }
  if (h_wave) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = 16 * mb + rl;
      if (m >= p.m) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int j = 16 * wave + 4 * g + v;
        if (j < r) {
          const float hv = poison ? __builtin_nanf("") : round_bf16(hacc[mb][v]);
          h_lds[m * (r + 1) + j] = hv;
          hb_lds[m * (r + 8) + j] = f32_to_bf16(hv);
        }
      }
    }
  }
  __syncthreads();
  if (tile == 0) {
    for (int idx = tid; idx < p.m * r; idx += 256) {
      const int m = idx / r;
      p.h[idx] = f32_to_bf16(h_lds[m * (r + 1) + (idx - m * r)]);
    }
  }
#pragma unroll
  for (int i = 0; i < FI; ++i) {
    const int f = wave + 4 * i;
    if (f >= F) break;
    const int mb = f % MB;
    const int t = (f / MB) % T;
    const int wr = f / (MB * T);
    const int m = 16 * mb + rl;
    // rank chunks past r are zero in both operands (the LDS rows' padding is
    // never written); h rows past M only reach outputs that are not stored
    f32x4_t tv = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (p.b_vec) {
      const uint16_t* bfr = b_lds + (wr * (16 * T) + 16 * t + rl) * (r + 8);
      const uint16_t* hfr = hb_lds + m * (r + 8);
      for (int c = 0; c < r; c += 32) {
        const bool ok = c + 8 * g < r;
        const int jc = ok ? c + 8 * g : 0;
        const u32x4_t bw = *reinterpret_cast<const u32x4_t*>(bfr + jc);
        const u32x4_t hw = *reinterpret_cast<const u32x4_t*>(hfr + jc);
        const u32x4_t zero{0u, 0u, 0u, 0u};
        tv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ok ? bw : zero),
                                                     as_bf16x8(ok ? hw : zero), tv, 0, 0, 0);
      }
    }
    if (m >= p.m) continue;
    const int lrow0 = wr * (16 * T) + 16 * t + 4 * g;
    const int64_t n0 = tile * ROWS + lrow0;
    const float* hrow = h_lds + m * (r + 1);
    uint16_t o[4] = {0, 0, 0, 0};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t n = n0 + v;
      if (n >= p.n) break;
      float tt = 0.0f;
      if (p.b_vec) {
        tt = tv[v];
      } else {
        const uint16_t* brow = p.lora_b + n * r;
        for (int j = 0; j < r; ++j) tt = __builtin_fmaf(hrow[j], bf16_to_f32(brow[j]), tt);
      }
      float out = round_bf16(round_bf16(wacc[i][v]) + round_bf16(round_bf16(tt) * p.scale));
      if (p.bias != nullptr) out = round_bf16(out + bf16_to_f32(p.bias[n]));
      o[v] = f32_to_bf16(out);
    }
    uint16_t* dst = p.y + static_cast<int64_t>(m) * p.n + n0;
    if (n0 + 3 < p.n && (p.n & 3) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 7) == 0) {
      *reinterpret_cast<u32x2_t*>(dst) =
          u32x2_t{static_cast<uint32_t>(o[0]) | (static_cast<uint32_t>(o[1]) << 16),
                  static_cast<uint32_t>(o[2]) | (static_cast<uint32_t>(o[3]) << 16)};
    } else {
      for (int v = 0; v < 4 && n0 + v < p.n; ++v) dst[v] = o[v];
    }
  }
}

// Bounded wait (lane 0 of the block) until all adapter blocks of this call
// have arrived and the last of them has stored the summed h. Adapter blocks
// come first in the grid and are dispatched before any weight block, and
// none of them waits on anything, so the wait ends as soon as they finish;
// the spin limit only guarantees that every wave exits. Returns false if the
// limit was hit.
__device__ __forceinline__ bool wait_adapters(const unsigned int* word, unsigned int target,
                                              int spin) {
  for (int it = 0; it < spin; ++it) {
    if (__hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == target) return true;
    __builtin_amdgcn_s_sleep(2);
  }
  return false;
}

template <int MB, int T, int U, int WK>
__global__ void __launch_bounds__(256) k_skinny(SkinnyParams p) {
  constexpr int WR = 4 / WK;
  constexpr int kRed = WK > 1 ? (WK - 1) * WR * T * MB * 64 : 1;
  __shared__ f32x4_t red[kRed];
  __shared__ float h_lds[64 * 65];
  __shared__ __align__(16) uint16_t hb_lds[64 * 72];
  __shared__ __align__(16) uint16_t b_lds[16 * T * WR * 72];
  __shared__ int flag;
  const int tid = threadIdx.x;
  unsigned int* ctr = g_skinny_counters[p.slot];
  // the adapter word counts the a_splits arrivals, then once more when the
  // last adapter block has stored the summed h
  const unsigned int a_target = static_cast<unsigned int>(p.a_splits + 1);
  const unsigned int done_target = static_cast<unsigned int>(p.a_splits + p.tiles);
  if (static_cast<int64_t>(blockIdx.x) < p.a_splits) {
    adapter_part<MB>(p, blockIdx.x);
    drain_stores();
    __syncthreads();
    if (tid == 0) {
      const unsigned int old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = old + 1u == static_cast<unsigned int>(p.a_splits) ? 1 : 0;
      if (!last) {
        drain_stores();  // the arrival is performed before it is counted as done
        done_count(ctr, 1, 2, done_target);
      }
      flag = last;
    }
    __syncthreads();
    if (flag == 0) return;
    // every other adapter block's partials were performed before its arrival
    adapter_sum<MB>(p);
    drain_stores();
    __syncthreads();
    if (tid == 0) {
      __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      drain_stores();
      done_count(ctr, 1, 2, done_target);
    }
    return;
  }
  const int64_t b = static_cast<int64_t>(blockIdx.x) - p.a_splits;
  const int64_t split = b / p.tiles;
  const int64_t tile = b - split * p.tiles;
  weight_part<MB, T, U, WK>(p, tile, split, red, b_lds);
  drain_stores();
  __syncthreads();
  if (tid == 0) {
    // the adapter word is read together with the arrival (one round trip);
    // it only grows until every finisher is past its wait
    const unsigned int adapters = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int last = arrive(ctr + 2 + tile, static_cast<unsigned int>(p.splits)) ? 1 : 0;
    if (last && adapters != a_target && !wait_adapters(ctr, a_target, p.spin)) {
      last = 2;
      __hip_atomic_fetch_or(p.err, kDevErrSkinnyWait, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // a finisher is past its last access to the slot once its wait ended
    if (last) done_count(ctr, 1, 2, done_target);
    flag = last;
  }
  __syncthreads();
  const int state = flag;
  if (state == 0) return;
  // state 2: the adapters never arrived within the spin limit; h is poisoned
  finish_tile<MB, T, WK>(p, tile, h_lds, hb_lds, b_lds, state == 2);
}

// (id, T, U, WK): wave = 16 T rows x 128 U columns; block = 4 / WK waves of
// rows x WK waves of columns.
#define RPX_SKINNY_CONFIGS(X) \
  X(1, 1, 1, 4)               \
  X(2, 1, 2, 4)               \
  X(3, 1, 4, 4)               \
  X(4, 1, 2, 1)               \
  X(5, 1, 4, 1)               \
  X(6, 2, 2, 1)               \
  X(7, 2, 2, 2)               \
  X(8, 4, 2, 1)               \
  X(9, 2, 4, 1)               \
  X(10, 1, 8, 1)              \
  X(11, 1, 2, 2)              \
  X(12, 1, 4, 2)              \
  X(13, 1, 1, 2)              \
  X(14, 2, 1, 4)              \
  X(15, 2, 2, 4)

struct SkinnyCfg {
  int id, t, u, wk;
};

constexpr SkinnyCfg kSkinnyCfgs[] = {
#define RPX_SKINNY_ENTRY(id, T, U, WK) {id, T, U, WK},
    RPX_SKINNY_CONFIGS(RPX_SKINNY_ENTRY)
#undef RPX_SKINNY_ENTRY
};

struct SkinnyPlan {
  SkinnyCfg cfg;
  int64_t mb, tiles, splits, kspan, a_splits;
};

SkinnyPlan make_plan(const SkinnyCfg& c, int64_t m, int64_t n, int64_t k) {
  SkinnyPlan p;
  p.cfg = c;
  p.mb = (m + 15) / 16;
  const int64_t rows = 16 * c.t * (4 / c.wk);
  p.kspan = 128 * c.u * c.wk;
  p.tiles = ceil_div(n, rows);
  p.splits = ceil_div(k, p.kspan);
  p.a_splits = ceil_div(k, kAdapterSpan);
  return p;
}

// Tile shape. A call is latency-bound: block dispatch, the weight stream's
// round trip, the partials' coherent stores, one arrival and the finisher's
// loads each cost a device round trip, so the shapes differ mainly in how
// many blocks they dispatch and how long the finisher's reductions are.
// Measured on the three Qwen3-2B projection shapes for M in {8, 16, 32, 64}
// (graph-replayed, weights cycled through HBM): from three 16-row M blocks
// up, and from two when K >= N, 32-row tiles with 1024-column splits over
// four column waves are fastest (M = 64: 26.7 / 33.5 / 19.3 -> 23.1 / 25.6 /
// 14.6 us on 2048->6144 / 6144->2048 / 2048->2048): half the K splits of the
// 64-row tile, so half the fp32 partials of y, at the same x fragments per
// wave. Below that, 64-row tiles with 512-column splits (two row waves x two
// column waves), or for one M block with K >= N 32-row tiles with
// 1024-column splits over two column waves, are best or within 5%. The
// kTuneSkinnyTile knob forces a shape.
SkinnyPlan plan_skinny(int64_t m, int64_t n, int64_t k) {
  int want = tune(kTuneSkinnyTile);
  if (want <= 0) {
    const int64_t mb = (m + 15) / 16;
    if (mb >= 3 || (mb == 2 && k >= n))
      want = 15;
    else
      want = (mb == 1 && k >= n) ? 12 : 7;
  }
  for (const SkinnyCfg& c : kSkinnyCfgs) {
    const SkinnyPlan p = make_plan(c, m, n, k);
    if (c.id == want && p.tiles <= kMaxTiles) return p;
  }
  // unknown id or too many tiles: the first shape that fits
  for (const SkinnyCfg& c : kSkinnyCfgs) {
    const SkinnyPlan p = make_plan(c, m, n, k);
    if (p.tiles <= kMaxTiles) return p;
  }
  return make_plan(kSkinnyCfgs[0], m, n, k);
}

int64_t frags_per_tile(const SkinnyPlan& p) { return (4 / p.cfg.wk) * p.cfg.t * p.mb; }


std::atomic<unsigned int> g_calls{0};

template <int MB, int T, int U, int WK>
void launch_cfg(const SkinnyParams& a, hipStream_t stream) {
  const unsigned blocks = static_cast<unsigned>(a.tiles * a.splits + a.a_splits);
  hipLaunchKernelGGL((k_skinny<MB, T, U, WK>), dim3(blocks), dim3(256), 0, stream, a);
}

template <int MB>
bool launch_mb(int id, const SkinnyParams& a, hipStream_t stream) {
  switch (id) {
#define RPX_SKINNY_CASE(cid, T, U, WK) \
  case cid:                            \
    launch_cfg<MB, T, U, WK>(a, stream); \
    return true;
    RPX_SKINNY_CONFIGS(RPX_SKINNY_CASE)
#undef RPX_SKINNY_CASE
    default:
      return false;
  }
}

}  // namespace

int skinny_tile_count() { return static_cast<int>(sizeof(kSkinnyCfgs) / sizeof(kSkinnyCfgs[0])); }

bool skinny_ok(int64_t m, int64_t n, int64_t k, int64_t rank, int64_t n_groups, int64_t group) {
  if (m < 1 || m > 64 || k % 128 != 0 || rank < 1 || rank > 64) return false;
  if (n_groups > 1 && (group < 32 || (group & (group - 1)) != 0)) return false;
  return plan_skinny(m, n, k).tiles <= kMaxTiles;
}

int64_t skinny_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t rank) {
  const SkinnyPlan p = plan_skinny(m, n, k);
  const int64_t one =
      p.splits * p.tiles * frags_per_tile(p) * 256 + (p.a_splits + 1) * 4 * p.mb * 256;
  const int64_t two = skinny2_ok(m, n, k, rank, 1, 0) ? skinny2_workspace_floats(m, n, k, rank) : 0;
  return one > two ? one : two;
}

hipError_t launch_skinny_forward(const uint16_t* x, int64_t m, int64_t k, const Int4Operand& w,
                                 int64_t n, const uint16_t* lora_a, const uint16_t* lora_b,
                                 int64_t rank, float scale, const uint16_t* bias, uint16_t* y,
                                 uint16_t* h, float* ws, hipStream_t stream) {
  const SkinnyPlan p = plan_skinny(m, n, k);
  if (p.tiles > kMaxTiles) return hipErrorInvalidValue;
  SkinnyParams a;
  a.x = x;
  a.m = static_cast<int>(m);
  a.rank = static_cast<int>(rank);
  a.k = k;
  a.n = n;
  a.packed = w.packed;
  a.pcols = w.packed_cols;
  a.scales = w.scales;
  a.n_groups = w.n_groups;
  a.group_shift = 0;
  if (w.n_groups > 1)
    while ((int64_t{1} << a.group_shift) < w.group) ++a.group_shift;
  a.b_vec = (rank % 8 == 0 && (reinterpret_cast<uintptr_t>(lora_b) & 15) == 0) ? 1 : 0;
  a.lora_a = lora_a;
  a.lora_b = lora_b;
  a.scale = scale;
  a.bias = bias;
  a.y = y;
  a.h = h;
  a.tiles = p.tiles;
  a.splits = p.splits;
  a.kspan = p.kspan;
  a.a_splits = p.a_splits;
  a.part_w = ws;
  a.part_h = a.part_w + p.splits * p.tiles * frags_per_tile(p) * 256;
  a.h_sum = a.part_h + p.a_splits * 4 * p.mb * 256;
  a.slot = static_cast<int>(g_calls.fetch_add(1, std::memory_order_relaxed) % kSlots);
  a.spin = tune(kTuneSpinLimit) > 0 ? tune(kTuneSpinLimit) : kSpinLimit;
  a.err = device_error_word();
  if (a.err == nullptr) return hipErrorInvalidSymbol;
  bool ok = false;
  switch (p.mb) {
    case 1: ok = launch_mb<1>(p.cfg.id, a, stream); break;
    case 2: ok = launch_mb<2>(p.cfg.id, a, stream); break;
    case 3: ok = launch_mb<3>(p.cfg.id, a, stream); break;
    default: ok = launch_mb<4>(p.cfg.id, a, stream); break;
  }
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace rpx
