// MFMA helpers shared by the batched GEMM kernels (gfx950):
// v_mfma_f32_16x16x32_bf16 on 16-byte operands, and the operand discipline
// the K-split kernels follow.
#pragma once

#include "common.h"

namespace ma {

typedef __bf16 bf16x8d_t __attribute__((ext_vector_type(8)));
typedef float f32x4d_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4d_t mfma16(uint4 a, uint4 b, f32x4d_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8d_t, a),
                                                 __builtin_bit_cast(bf16x8d_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4d_t mfma16v(u32x4v_t a, u32x4v_t b, f32x4d_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8d_t, a),
                                                 __builtin_bit_cast(bf16x8d_t, b), c, 0, 0, 0);
}

// Operand discipline of the K-split GEMMs.  The MFMAs are issued as inline
// assembly that accumulates in place (the result register IS the C operand),
// in blocks: a step's A and B operands, and the rest of its VALU work (pin),
// are all done before the block (mfma_block_begin, which also leaves the VALU
// results a few idle cycles to land); the block holds MFMAs only; and
// mfma_block_end keeps every instruction after it 24 cycles clear of the
// block's last MFMA, after which the operands may be reused (keep_b keeps them
// live until then).  Left to itself, the compiler chained dependent MFMAs
// through different registers (a result written to a new register and read as
// the next MFMA's C operand a cycle or two later) and wrote registers an
// in-flight MFMA was still reading; those schedules gave wrong sums on gfx950.
__device__ __forceinline__ void mfma_acc(f32x4d_t& acc, const u32x4v_t& a, const u32x4v_t& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_block_begin() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 4" ::: "memory");
}
// A value of the step's VALU work that is only used after the block: pinning
// it here keeps its arithmetic out of the MFMA block.
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void mfma_block_end() {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <int NA>
__device__ __forceinline__ void keep_b(const u32x4v_t& b, const f32x4d_t (&acc)[NA]) {
  asm volatile("" ::"v"(b), "v"(acc[0]), "v"(acc[NA - 1]));
}
template <typename T, int M, int NA>
__device__ __forceinline__ void keep_b(const T (&b)[M], const f32x4d_t (&acc)[NA]) {
#pragma unroll
  for (int i = 0; i < M; ++i) keep_b(b[i], acc);
}

template <int N, int M, typename T, int NA>
__device__ __forceinline__ void keep_operands(const u32x4v_t (&av)[N][2], const T (&bv)[M],
                                              const f32x4d_t (&acc)[NA]) {
#pragma unroll
  for (int i = 0; i < N; ++i)
    asm volatile("" ::"v"(av[i][0]), "v"(av[i][1]), "v"(acc[0]), "v"(acc[NA - 1]));
  keep_b(bv, acc);
}

}  // namespace ma
