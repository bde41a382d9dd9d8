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
// round-robin, in contiguous ranges so each XCD's L2 keeps a few A row-blocks.
__device__ __forceinline__ int xcd_block(int block, int total) {
  return total % 8 == 0 ? (block % 8) * (total / 8) + block / 8 : block;
}

}  // namespace rpx
