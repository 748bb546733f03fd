// Shared device/host helpers for the maple_amd HIP library (gfx950 only).
//
// Packed formats (reference src/maple_run/pack.py:17-20):
//   ternary: 16 two-bit codes per uint32, LSB first, value = code - 1
//   rtn4:    8 four-bit codes per uint32, LSB first, value = q * scale + bias
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/maple_amd.h"

namespace ma {

// ---------------------------------------------------------------------------
// Error reporting: the last failure message of the calling host thread.
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int status, const char* fmt, ...);
int check_launch(const char* what);
// Workgroups of `kernel` (with `threads` threads, no dynamic LDS) resident at
// once on the current device: compute units x occupancy.  Persistent kernels
// whose workgroups wait on each other check their grid against it.
int resident_capacity(const void* kernel, int threads, int64_t* capacity);

// The GPU's XCDs (gfx950: 8, each with its own L2) and the XCD a workgroup
// runs on.  Workgroups on one XCD can hand data to each other through its L2
// (a plain store read back with a device-coherent load); across XCDs the data
// goes through memory.  xcd_round_robin: whether the current device hands a
// launch's workgroups to its XCDs in turn (workgroup i on XCD (i + o) mod
// kXcds), checked once per device by a probe launch on ``st`` (runtime.hip).
constexpr int kXcds = 8;
__device__ __forceinline__ int xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return static_cast<int>(v & 0xf);
}
int xcd_round_robin(hipStream_t st, bool* ok);

// ---------------------------------------------------------------------------
// Scalar conversions.  bf16 is carried as raw uint16 bits.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even float -> bf16 (NaN stays a NaN): gfx950's
// v_cvt_pk_bf16_f32, one instruction.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// bf16 bits of a float known to be exactly representable in bf16.
__device__ __forceinline__ uint32_t bf16_bits_exact(float f) { return __float_as_uint(f) >> 16; }

// Typed scalar load with the dtype fixed at compile time (no branch, so the
// load can be issued early and waited on only where it is used).
template <int DT>
__device__ __forceinline__ float ld_t(const void* p, int64_t i) {
  if constexpr (DT == MA_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else if constexpr (DT == MA_F16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  else return static_cast<const float*>(p)[i];
}

// Raw bits of element i of a row-scale array, converted by from_raw<DT>
// where the value is used.  Converted next to the load inside a branch, the
// value makes the wave wait for that load there -- and, memory counters
// completing in issue order, for every load issued before it.
template <int DT>
__device__ __forceinline__ uint32_t ld_raw(const void* p, int64_t i) {
  if constexpr (DT == MA_F32) return static_cast<const uint32_t*>(p)[i];
  else return static_cast<const uint16_t*>(p)[i];
}
template <int DT>
__device__ __forceinline__ float from_raw(uint32_t u) {
  if constexpr (DT == MA_BF16) return bf16_to_f32(static_cast<uint16_t>(u));
  else if constexpr (DT == MA_F16) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u)));
  else return __uint_as_float(u);
}

// Element i of a float32, bf16 or f16 array whose dtype is known only at run
// time, read as the aligned 32-bit word that holds it: one unconditional
// load with no dtype branch around it (a 16-bit element's neighbour comes
// along; an aligned word never crosses a page, so it is as safe to read as
// the element).  any_word_f() converts it where the value is used.  With
// ld_f the load sits in a dtype branch and its conversion, with the wait for
// it, right behind it, so a run of such loads costs a round trip each.
struct AnyWord {
  uint32_t w;
  uint32_t sh;  // 16 for an element in the upper half of the word, else 0
};
__device__ __forceinline__ AnyWord ld_any_word(const void* p, int dt, int64_t i) {
  // pointer arithmetic (not an integer round trip) keeps the global address
  // space known, so this is a global load rather than a flat one
  const char* const e = static_cast<const char*>(p) + i * (dt == MA_F32 ? 4 : 2);
  const uint32_t mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(e)) & 3u;
  return {*reinterpret_cast<const uint32_t*>(e - mis), mis * 8u};
}
__device__ __forceinline__ float any_word_f(AnyWord v, int dt) {
  const uint32_t h = (v.w >> v.sh) & 0xffffu;
  const float f16 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
  return dt == MA_F32 ? __uint_as_float(v.w) : (dt == MA_BF16 ? __uint_as_float(h << 16) : f16);
}

__device__ __forceinline__ float ld_f(const void* p, int dt, int64_t i) {
  switch (dt) {
    case MA_BF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case MA_F16: return static_cast<float>(static_cast<const _Float16*>(p)[i]);
    default: return static_cast<const float*>(p)[i];
  }
}

__device__ __forceinline__ void st_f(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case MA_BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16(v); break;
    case MA_F16: static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v); break;
    default: static_cast<float*>(p)[i] = v; break;
  }
}

__device__ __forceinline__ int64_t ld_id(const void* p, int is64, int64_t i) {
  return is64 ? static_cast<const int64_t*>(p)[i] : static_cast<const int32_t*>(p)[i];
}

// ---------------------------------------------------------------------------
// Ternary expansion for v_dot2_f32_bf16.
//
// A 2-bit code c placed in mantissa bits [p, p+1] of bf16 1.0 (0x3F80) reads
// as exactly 1 + c * 2^(p-7).  With p = 3 that is 1 + c/16, with p = 5 it is
// 1 + c/4.  Pair j of a word holds codes j (low half) and j + 8 (high half);
// one shift lines both up, one and/or builds the bf16x2 operand:
//
//   pair 0,1: w << 3     pair 2,3: w >> 1     pair 4,5: w >> 5     pair 6,7: w >> 9
//   even pair: bits 3-4 (f = 16)               odd pair: bits 5-6 (f = 4)
//
// Dotting against x' = f * x (exact: a power-of-two scale) gives
// sum (f + c) x, so sum (c - 1) x = acc - sum (f + 1) x, where the second sum
// depends only on x and is formed once per lane.  Code 3 therefore reads as
// +2, the reference semantics (kernels/ternary_gemv.py:126-128).
// ---------------------------------------------------------------------------
constexpr uint32_t kOneBf16x2 = 0x3F803F80u;
constexpr uint32_t kMaskP3 = 0x00180018u;
constexpr uint32_t kMaskP5 = 0x00600060u;

__device__ __forceinline__ float pair_scale(int j) { return (j & 1) ? 4.0f : 16.0f; }

// (a & m) | o as one v_and_or_b32.  The operands are pinned to VGPRs: with
// both constants as literals the compiler would split it into two VOP2 ops.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(o));
  return r;
}

// Loop-invariant constants of expand_word, held in registers by the caller.
struct ExpandConsts {
  uint32_t m3, m5, one;
  __device__ __forceinline__ ExpandConsts() : m3(kMaskP3), m5(kMaskP5), one(kOneBf16x2) {}
};

// The 8 bf16x2 operands of one packed word.
__device__ __forceinline__ void expand_word(uint32_t w, uint32_t e[8], const ExpandConsts& k) {
  const uint32_t s0 = w << 3, s1 = w >> 1, s2 = w >> 5, s3 = w >> 9;
  e[0] = and_or(s0, k.m3, k.one);
  e[1] = and_or(s0, k.m5, k.one);
  e[2] = and_or(s1, k.m3, k.one);
  e[3] = and_or(s1, k.m5, k.one);
  e[4] = and_or(s2, k.m3, k.one);
  e[5] = and_or(s2, k.m5, k.one);
  e[6] = and_or(s3, k.m3, k.one);
  e[7] = and_or(s3, k.m5, k.one);
}

// Half hh of a packed word's 8 bf16x2 operands (expand_word's e[4 hh .. +3]):
// one MFMA A operand (8 bf16) per lane.
__device__ __forceinline__ uint4 expand_half(uint32_t w, int hh, const ExpandConsts& k) {
  const uint32_t s0 = hh ? w >> 5 : w << 3, s1 = hh ? w >> 9 : w >> 1;
  return make_uint4(and_or(s0, k.m3, k.one), and_or(s0, k.m5, k.one), and_or(s1, k.m3, k.one),
                    and_or(s1, k.m5, k.one));
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Pack two floats that are exactly representable in bf16 into a bf16x2 word.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return bf16_bits_exact(lo) | (bf16_bits_exact(hi) << 16);
}

// Round two floats to bf16 (nearest even) and pack them, lo in the low half.
__device__ __forceinline__ uint32_t pack_bf16x2_rn(float lo, float hi) {
  typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
  const bf16x2v_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// x' pairs for one word from 16 consecutive activations xs[0..15] (already
// float): pair j = (f_j * xs[j], f_j * xs[j+8]).  Returns sum (f_j + 1) xs.
// Only exact when xs are bf16 values (the fast path's input dtype).
__device__ __forceinline__ float prep_word_pairs(const float xs[16], uint32_t xp[8]) {
  float c = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float f = pair_scale(j);
    xp[j] = pack_bf16x2(f * xs[j], f * xs[j + 8]);
    c += (f + 1.0f) * (xs[j] + xs[j + 8]);
  }
  return c;
}

// Convert 16 bf16 activations (two uint4) into 8 x' pair dwords; returns
// sum (f + 1) x over them.
__device__ __forceinline__ float x16_to_pairs(uint4 a, uint4 b, uint32_t pr[8]) {
  const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float v[16];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    v[2 * q] = __uint_as_float(u[q] << 16);
    v[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
  }
  return prep_word_pairs(v, pr);
}

// SwiGLU of the reference's expert MLP (kernels/ternary_expert.py:314-318):
// clamp(up, -7, 7) * g * sigmoid(g) with g = min(gate, 7), in that order;
// sigmoid(g) = 1 / (1 + exp(-g)), exp(-g) as 2^(-g log2 e) on the hardware
// exponential (v_exp_f32) and the division as the hardware reciprocal
// (v_rcp_f32), each about 1 ulp -- the reference's Triton sigmoid also takes
// its exp as an approximate base-2 exponential and divides approximately.
// (-g log2 e > -10.1 here, so no result is denormal; a very negative gate
// gives exp = +inf and an output of 0.)
constexpr float kMlpClamp = 7.0f;
constexpr float kLog2e = 1.4426950408889634f;
__device__ __forceinline__ float swiglu_act(float up, float gate) {
  up = fminf(fmaxf(up, -kMlpClamp), kMlpClamp);
  gate = fminf(gate, kMlpClamp);
  return (up * gate) * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gate * kLog2e));
}

// ---------------------------------------------------------------------------
// Wave-level helpers (wave64).
// ---------------------------------------------------------------------------
// DPP / swizzle lane exchanges.  quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E;
// row_ror:n = 0x120 + n rotates within each 16-lane row.  ds_swizzle in
// bitmask mode reads lane ((j & 0x1F) ^ xor) within each 32-lane half.
#define MA_DPP(v, ctrl) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, false))
#define MA_SWZ_XOR(v, x) \
  __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, (v)), 0x1F | ((x) << 10)))

// Sum over aligned groups of WIDTH lanes (WIDTH in {1,2,4,8,16,32,64}); every
// lane of a group receives the group's total.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (WIDTH >= 2) v += MA_DPP(v, 0xB1);
  if constexpr (WIDTH >= 4) v += MA_DPP(v, 0x4E);
  if constexpr (WIDTH == 8) v += MA_SWZ_XOR(v, 4);
  if constexpr (WIDTH >= 16) {
    v += MA_DPP(v, 0x124);
    v += MA_DPP(v, 0x128);
  }
  if constexpr (WIDTH >= 32) v += MA_SWZ_XOR(v, 16);
  if constexpr (WIDTH >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, MA_DPP(v, 0xB1));
  v = fmaxf(v, MA_DPP(v, 0x4E));
  v = fmaxf(v, MA_DPP(v, 0x124));
  v = fmaxf(v, MA_DPP(v, 0x128));
  v = fmaxf(v, MA_SWZ_XOR(v, 16));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

// Value of lane `src` (a compile-time or wave-uniform index) in every lane.
__device__ __forceinline__ float lane_bcast(float v, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

// Wave-uniform max and sum without an LDS round trip: prefix steps within each
// 16-lane row (row_shr 1, 2, 4, 8), then row_bcast:15 (rows 1 and 3 take the
// row below's lane 15) and row_bcast:31 (rows 2 and 3 take lane 31) carry the
// total into lane 63, which is read back as a scalar.  Lanes whose DPP source
// is outside the row or in a masked row keep `old` (the identity).
#define MA_DPP_OLD(old, v, ctrl, rmask)                                                 \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, (old)), \
                                                        __builtin_bit_cast(int, (v)), (ctrl), (rmask), 0xF, false))

__device__ __forceinline__ float wave_max_u(float v) {
  v = fmaxf(v, MA_DPP_OLD(v, v, 0x111, 0xF));
  v = fmaxf(v, MA_DPP_OLD(v, v, 0x112, 0xF));
  v = fmaxf(v, MA_DPP_OLD(v, v, 0x114, 0xF));
  v = fmaxf(v, MA_DPP_OLD(v, v, 0x118, 0xF));
  v = fmaxf(v, MA_DPP_OLD(v, v, 0x142, 0xA));
  v = fmaxf(v, MA_DPP_OLD(v, v, 0x143, 0xC));
  return lane_bcast(v, 63);
}

// Sum over aligned groups of WIDTH lanes (16, 32 or 64), complete only in the
// last lane of each group (the same prefix steps, no LDS round trip).
template <int WIDTH>
__device__ __forceinline__ float group_sum_last(float v) {
  static_assert(WIDTH == 16 || WIDTH == 32 || WIDTH == 64, "group width");
  v += MA_DPP_OLD(0.f, v, 0x111, 0xF);
  v += MA_DPP_OLD(0.f, v, 0x112, 0xF);
  v += MA_DPP_OLD(0.f, v, 0x114, 0xF);
  v += MA_DPP_OLD(0.f, v, 0x118, 0xF);
  if constexpr (WIDTH >= 32) v += MA_DPP_OLD(0.f, v, 0x142, 0xA);
  if constexpr (WIDTH == 64) v += MA_DPP_OLD(0.f, v, 0x143, 0xC);
  return v;
}

// Integer form of wave_max_u (v_max_i32 needs no NaN canonicalisation).
__device__ __forceinline__ int wave_max_ui(int v) {
#define MA_DPP_I(v, ctrl, rmask) __builtin_amdgcn_update_dpp(INT_MIN, (v), (ctrl), (rmask), 0xF, false)
  v = max(v, MA_DPP_I(v, 0x111, 0xF));
  v = max(v, MA_DPP_I(v, 0x112, 0xF));
  v = max(v, MA_DPP_I(v, 0x114, 0xF));
  v = max(v, MA_DPP_I(v, 0x118, 0xF));
  v = max(v, MA_DPP_I(v, 0x142, 0xA));
  v = max(v, MA_DPP_I(v, 0x143, 0xC));
#undef MA_DPP_I
  return __builtin_amdgcn_readlane(v, 63);
}

// Signed-integer key with the order of the float v (for every non-NaN v).
__device__ __forceinline__ int float_order_key(float v) {
  const int b = __float_as_int(v);
  return b ^ ((b >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float float_from_order_key(int k) { return __int_as_float(k ^ ((k >> 31) & 0x7fffffff)); }

__device__ __forceinline__ float wave_sum_u(float v) {
  v += MA_DPP_OLD(0.f, v, 0x111, 0xF);
  v += MA_DPP_OLD(0.f, v, 0x112, 0xF);
  v += MA_DPP_OLD(0.f, v, 0x114, 0xF);
  v += MA_DPP_OLD(0.f, v, 0x118, 0xF);
  v += MA_DPP_OLD(0.f, v, 0x142, 0xA);
  v += MA_DPP_OLD(0.f, v, 0x143, 0xC);
  return lane_bcast(v, 63);
}

// Block-wide sum over 256 threads; every thread gets the total.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = group_sum<64>(v);
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wv] = v;
  __syncthreads();
  const float t = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return t;
}

// Nothing may be scheduled across this point: keeps every load issued above
// it ahead of the arithmetic below (the scheduler otherwise sinks loads next
// to their first use to save registers, serialising their latencies).
#define MA_ISSUE_FENCE() __builtin_amdgcn_sched_barrier(0)

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// A grouped MoE combine run in front of a kernel that reads its output rows
// (k_xprep): y[t] = sum_j wts[t, j] * slot_out[inverse[t, j]] + res[t].
// The (row, weight) pairs of token t's k <= 8 slots, in every lane: lane j
// (mod 8) loads slot j's pair (slots past k re-read the last one), then each
// pair is read off its lane -- two loads in flight at once, where 2k uniform
// loads, each under a slot condition, were issued one after the other with a
// wait for each.
__device__ __forceinline__ void slot_pairs8(const int32_t* __restrict__ inverse, const float* __restrict__ wts,
                                            int64_t t, int k, int64_t (&row)[8], float (&w)[8]) {
  const int lj = static_cast<int>(threadIdx.x) & 7;
  const int j = lj < k ? lj : k - 1;
  const int32_t r = inverse[t * k + j];
  const float ww = wts[t * k + j];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    row[s] = __builtin_amdgcn_readlane(r, s);
    w[s] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(ww), s));
  }
}

struct CombineIn {
  const uint16_t* slot_out;  // bf16 [pairs, K * 16] (null: read x)
  const int32_t* inverse;    // [batch, topk] row of each (token, slot) in slot_out
  const float* wts;          // [batch, topk]
  int topk;                  // <= 8
  const uint16_t* res;       // bf16 [batch, K * 16] or null
  uint16_t* x_out;           // bf16 [batch, K * 16]: the combined rows
};


}  // namespace ma
