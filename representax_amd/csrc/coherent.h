// Block-to-block hand-off inside one launch: arrival counters and
// device-coherent stores and loads of partial results.
#pragma once

#include "common.h"

namespace rpx {

// One arrival; true for the last of `target`, which puts the word back to 0.
__device__ __forceinline__ bool arrive(unsigned int* word, unsigned int target) {
  const unsigned int old = __hip_atomic_fetch_add(word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old + 1u != target) return false;
  __hip_atomic_store(word, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Counts one participant of a call as done with its slot of arrival words
// (after its last access to them); the last of `target` participants clears
// slot[0 .. n_words), the done word among them, so every call leaves its slot
// at zero however its waits ended.
__device__ __forceinline__ void done_count(unsigned int* slot, int done_word, int n_words,
                                           unsigned int target) {
  const unsigned int old =
      __hip_atomic_fetch_add(slot + done_word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old + 1u != target) return;
  for (int i = 0; i < n_words; ++i)
    __hip_atomic_store(slot + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Partial sums cross blocks through agent-scope (device-coherent) 64-bit
// stores and loads instead of plain accesses plus a release/acquire fence
// pair: on this target an agent-scope release fence writes back the whole
// L2 of the XCD, which at one fence per block costs more than the weight
// stream itself. A coherent store has reached the coherence point once the
// wave's vmcnt drains (drain_stores), before the block's arrival is counted.
//
// A wave's fragment (64 lanes x 4 floats, 1 KB at `frag`) is stored by
// halves: lane l's floats 0-1 go to 64-bit word l and floats 2-3 to word
// 64 + l, so each of the two store instructions writes 512 contiguous bytes
// (with the halves interleaved per lane, each instruction covered every
// 64-byte segment only half and the segments were written twice).
__device__ __forceinline__ void store_coherent(f32x4_t* frag, int lane, f32x4_t v) {
  unsigned long long* d = reinterpret_cast<unsigned long long*>(frag);
  const u32x4_t u = __builtin_bit_cast(u32x4_t, v);
  __hip_atomic_store(d + lane, static_cast<unsigned long long>(u[0]) | (static_cast<unsigned long long>(u[1]) << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(d + 64 + lane,
                     static_cast<unsigned long long>(u[2]) | (static_cast<unsigned long long>(u[3]) << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4_t load_coherent(const f32x4_t* frag, int lane) {
  unsigned long long* s = reinterpret_cast<unsigned long long*>(const_cast<f32x4_t*>(frag));
  const unsigned long long a = __hip_atomic_load(s + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long b = __hip_atomic_load(s + 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_bit_cast(f32x4_t, u32x4_t{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32),
                                             static_cast<uint32_t>(b), static_cast<uint32_t>(b >> 32)});
}
__device__ __forceinline__ void drain_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// The running launch's dispatch id (an LLVM intrinsic without a clang
// builtin): the command processor counts it up per queue.
extern "C" __device__ unsigned long long rpx_amdgcn_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

// A 32-bit tag of the running launch, never zero: a hash of its dispatch id,
// the address of its dispatch packet (which tells the queues apart) and a
// count the host passes. Every launch, graph replays included, gets its own
// tag without any block counting in; words that blocks of one launch hand
// to each other carry it, so a word left by an earlier launch is taken only
// if the two 32-bit tags collide.
__device__ __forceinline__ unsigned int launch_tag(unsigned int host) {
  const unsigned long long id = rpx_amdgcn_dispatch_id();
  const unsigned long long pkt = reinterpret_cast<uintptr_t>(__builtin_amdgcn_dispatch_ptr());
  unsigned long long h = (id * 0x9E3779B97F4A7C15ull) ^ (pkt * 0xC2B2AE3D27D4EB4Full) ^ host;
  h ^= h >> 31;
  h *= 0xBF58476D1CE4E5B9ull;
  h ^= h >> 32;
  const unsigned int t = static_cast<unsigned int>(h);
  return t != 0u ? t : 1u;
}

// 32-bit coherent store and load (single values, flags).
__device__ __forceinline__ void store_coherent_f32(float* dst, float v) {
  __hip_atomic_store(reinterpret_cast<unsigned int*>(dst), __builtin_bit_cast(unsigned int, v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent_f32(const float* src) {
  return __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<unsigned int*>(const_cast<float*>(src)),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

}  // namespace rpx
