// Cross-workgroup hand-offs inside one launch (gfx950): device-coherent
// loads and stores, and a grid barrier over resident workgroups.
//
// Agent-scope relaxed atomics compile to accesses with the sc1 cache policy:
// a store is visible to workgroups on every XCD once it has completed (wait
// with s_waitcnt), and a load reads the coherent copy, so no device-scope
// fence is needed (on this GPU that fence writes back and invalidates the
// whole L2).
#pragma once

#include "common.h"

namespace ma {

constexpr uint64_t kGridSpin = 20000000ull;  // 0.2 s of the 100 MHz realtime counter
constexpr int kBarGroups = 16;               // sub-counters (and release flags) per barrier
constexpr int kLine = 64;                    // uint32 words in a 256-byte line

__device__ __forceinline__ uint32_t ld_coh32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_coh64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Stores read back only by workgroups of the same XCD: plain stores, which
// land in the XCD's L2 (the vector L1 is write-through); the readers' sc1
// loads (ld_coh*) are served by that L2.
__device__ __forceinline__ void st_l2_32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void st_l2_64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void st_coh16(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Grid barrier, run by all 64 lanes of wave 0 of every workgroup once its
// global stores (and its read of its group's flag, f_old) have completed.
// Workgroup wg arrives on counter wg % kBarGroups of its group; the group's
// last arriver clears the counter and writes f_old + 1 to the group's flag,
// and every workgroup polls all kBarGroups group flags, one lane each, until
// none holds f_old any more.  The flags thus all hold the number of barriers
// passed once a barrier is over, and nothing needs clearing afterwards.  (One
// atomic per workgroup on a single counter would serialise all G of them at
// one address; a second level of counters above the groups put one more
// returning atomic on the last arrival's path, about 0.2 us slower per
// barrier; polling never-cleared counters directly collided with the
// arrivals and took 2 us.)  Needs G >= kBarGroups, every workgroup
// resident.  Returns true (on all lanes) if the wait timed out.
__device__ inline bool grid_barrier_flags(uint32_t* sub, uint32_t* flags, uint32_t f_old, int G, int wg, int lane,
                                          uint64_t t0) {
  const int g = wg % kBarGroups;
  if (lane == 0) {
    const uint32_t n_g = static_cast<uint32_t>((G - g + kBarGroups - 1) / kBarGroups);
    if (atomicAdd(&sub[kLine * g], 1u) == n_g - 1) {
      st_coh32(&sub[kLine * g], 0u);
      st_coh32(&flags[kLine * g], f_old + 1u);
    }
  }
  int timed_out = 0;
  for (;;) {
    const bool seen = lane >= kBarGroups || ld_coh32(&flags[kLine * lane]) != f_old;
    if (__all(seen)) break;
    if ((__builtin_amdgcn_s_memrealtime() - t0) > kGridSpin) {
      timed_out = 1;
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  return timed_out != 0;
}

// At the head of every iteration of a wait loop that reads through a
// CoherentBuf: the buffer-load builtins count as reads of unchanging memory,
// so without this clobber the compiler hoists them out of the loop.
#define MA_POLL_RELOAD() asm volatile("" ::: "memory")

// Waits until this wave's stores have been acknowledged by the L2, and keeps
// the compiler from moving any memory access across the wait.
#define MA_STORES_DONE() asm volatile("s_waitcnt vmcnt(0)" ::: "memory")

// Device-coherent 8- and 16-byte access through a buffer resource: the sc1 cache policy (the bit agent-scope atomic loads and
// stores carry on this GPU) sends each access to the coherent level, so a
// store is visible to workgroups on every XCD once it has completed, without
// a fence, and one 16-byte access replaces two 8-byte atomics (reading
// data just written elsewhere is bound by the number of coherent requests
// one CU issues).  Offsets are bytes; the hardware range check drops
// accesses past num_bytes.
constexpr int kCoherentPolicy = 16;  // sc1
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
struct CoherentBuf {
  __amdgpu_buffer_rsrc_t r;
  __device__ CoherentBuf(const void* p, uint32_t num_bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, num_bytes, 0x00020000)) {}
  __device__ float2 ld2(uint32_t off) const {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCoherentPolicy));
  }
  __device__ uint4 ld4u(uint32_t off) const {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoherentPolicy));
  }
  __device__ float4 ld4(uint32_t off) const {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoherentPolicy));
  }
  __device__ void st2(uint32_t off, float2 v) const {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), r, off, 0, kCoherentPolicy);
  }
  __device__ void st4(uint32_t off, float4 v) const {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, off, 0, kCoherentPolicy);
  }
};

}  // namespace ma
