// Building blocks of the pipelined MFMA GEMMs (gfx950): swizzled 128-byte LDS
// rows filled by direct-to-LDS loads, and the explicit wait + barrier that
// hands a landed K-slice to every wave of the workgroup.
#pragma once

#include "common.h"

namespace rpx {

typedef __attribute__((address_space(3))) void lds_void_t;

// LDS rows of 128 bytes (eight 16-byte chunks), unpadded: chunk c of row r
// lives at physical chunk c ^ swz(r). A ds_read_b128 fragment read puts the
// lanes of each 16-lane group on 16 different rows of one logical chunk;
// with this swizzle they hit 16 distinct 16-byte bank groups of a 256-byte
// LDS cycle, and any 8 consecutive rows hit 8 distinct chunks.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// Waits until at most N of this wave's vector-memory operations are pending
// and every LDS operation has returned, then joins the workgroup barrier. The
// memory clobber keeps the LDS reads of the next slice below the barrier.
template <int N>
__device__ __forceinline__ void wait_sync() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// One direct-to-LDS load of 16 bytes per lane: the wave's 64 lanes fill the
// 1 KB segment `seg` of `stage`, lane l writing bytes [16 l, 16 l + 16).
__device__ __forceinline__ void dma_seg(uint8_t* stage, const uint8_t* src, int64_t koff, int seg) {
  __builtin_amdgcn_global_load_lds(
      src + koff, reinterpret_cast<lds_void_t*>(reinterpret_cast<uintptr_t>(stage) + seg * 1024), 16,
      0, 0);
}

// 16 bytes of a 128-byte swizzled LDS row: logical chunk c of `row`.
__device__ __forceinline__ u32x4_t lds_chunk(const uint8_t* base, int row, int c) {
  return *reinterpret_cast<const u32x4_t*>(base + row * 128 + ((c ^ swz(row)) << 4));
}

// Row-major tiles (n fastest) dealt to the 8 XCDs, which take workgroups
// round-robin (block b runs on XCD b % 8), in contiguous ranges so each
// XCD's L2 keeps a few A row-blocks: XCD x, which gets q = total / 8 blocks
// plus one more when x < total % 8, takes the tiles from
// x q + min(x, total % 8) on. A bijection of [0, total).
__device__ __forceinline__ int xcd_block(int block, int total) {
  const int q = total / 8;
  const int r = total % 8;
  const int x = block % 8;
  return x * q + (x < r ? x : r) + block / 8;
}

// Position (tm, tn) of tile t in banded order: bands of `band` row-blocks,
// each walked column by column with the band's rows fastest. The tiles an
// XCD runs at once then share `band` A row-blocks and about
// (tiles in flight) / band B column-blocks, instead of one A row-block and
// every B column-block (band 1 is plain row-major order). A bijection of
// [0, tiles_m * tiles_n) for every band >= 1.
__device__ __forceinline__ void band_tile(int t, int tiles_m, int tiles_n, int band, int& tm,
                                          int& tn) {
  const int first = (t / (band * tiles_n)) * band;
  const int rows = tiles_m - first < band ? tiles_m - first : band;
  const int w = t - first * tiles_n;
  tm = first + w % rows;
  tn = w / rows;
}

}  // namespace rpx
