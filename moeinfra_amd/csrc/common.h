// Shared definitions for the gfx950 MoE expert-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/moeinfra_hip.h"

namespace moe {

// Records a printf-style message as the calling thread's last error.
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
// Number of compute units of the current device (cached per device).
int device_cu_count();

constexpr int kWave = 64;

// ---------------------------------------------------------------- vector types
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
// 16 bytes as a native vector (unlike HIP's uint4 struct, copies of it stay in registers).
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

// ---------------------------------------------------------------- bf16 helpers
// Round-to-nearest-even float -> bf16 bits (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// Two round-to-nearest-even conversions in one v_cvt_pk_bf16_f32, lo in the low half.
typedef float f32x2_ev __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_ev __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_ev){lo, hi}, bf16x2_ev));
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
__device__ __forceinline__ float bf16lo_to_f32(uint32_t w) {
  return __builtin_bit_cast(float, w << 16);
}
__device__ __forceinline__ float bf16hi_to_f32(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}

// ---------------------------------------------------------------- streamed loads
// 16 bytes of global memory loaded with the non-temporal hint (global_load_dwordx4 ... nt),
// for weights that a pass reads exactly once.  A single-pass read of 1 GB streams at
// ~7.0 TB/s this way on MI355X against ~6.1 TB/s with plain loads.
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4v;
__device__ __forceinline__ uint4 ld_stream16(const void *p) {
  const u32x4v v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4v *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------------- kernel arguments
// Kernel arguments arrive through scalar loads from the argument buffer, a memory round trip
// each time the kernel waits for them.  When the first arithmetic needs only some arguments
// (an index division, a loop bound), the compiler waits for those first and issues the
// loads of the others after it, so a second round trip sits before the first global load.
// MOE_ARGS_FIRST(scalars, pointers) is an empty asm that takes every pointer argument
// as an SGPR input and every scalar argument as an SGPR in/out operand: all later code
// depends on it, so every argument is loaded in one batch ahead of it.  Pointers are inputs
// only, so the compiler still knows they point to global memory.  Each operand list is
// wrapped in MOE_LIST(...).
#define MOE_LIST(...) __VA_ARGS__
#define MOE_ARGS_FIRST(outs, ins) asm volatile("" : outs : ins)

// ---------------------------------------------------------------- wave reductions

// op(v, v of lane l ^ 32) and op(v, v of lane l ^ 16) in every lane l (op: + or max), by one
// v_permlane32_swap / v_permlane16_swap (VALU, no LDS round trip).  With both operands v, the
// swap returns [v(0..31), v(0..31)] and [v(32..63), v(32..63)] (16: rows 0, 0, 2, 2 and
// 1, 1, 3, 3), so lane l adds its own value and its partner's, in one order or the other:
// bit-identical to v + __shfl_xor(v, 32) as IEEE addition and max are commutative.  The
// second result passes through an empty asm: without it the compiler reads the first result
// twice when both feed one operation.
template <bool MAX>
__device__ __forceinline__ float op_xor32(float v) {
  const unsigned w = __builtin_bit_cast(unsigned, v);
  const auto x = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  unsigned hi = x[1];
  asm volatile("" : "+v"(hi));
  const float a = __builtin_bit_cast(float, (unsigned)x[0]), b = __builtin_bit_cast(float, hi);
  return MAX ? fmaxf(a, b) : a + b;
}
template <bool MAX>
__device__ __forceinline__ float op_xor16(float v) {
  const unsigned w = __builtin_bit_cast(unsigned, v);
  const auto x = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  unsigned hi = x[1];
  asm volatile("" : "+v"(hi));
  const float a = __builtin_bit_cast(float, (unsigned)x[0]), b = __builtin_bit_cast(float, hi);
  return MAX ? fmaxf(a, b) : a + b;
}

// DPP move of v with control CTRL (row_mask and bank_mask all set, no bound control).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf,
                                                            0xf, false));
}

// Sum over the wave by the butterfly l ^ 32, 16, 8, 4, 2, 1 (every lane gets the sum): the
// exchanges with lane l ^ 8 (row_ror:8 within a 16-lane row), l ^ 2 and l ^ 1 (quad_perm)
// are DPP moves, l ^ 32 and l ^ 16 permlane swaps, l ^ 4 an LDS shuffle.
__device__ __forceinline__ float wave_sum(float v) {
  v = op_xor32<false>(v);
  v = op_xor16<false>(v);
  v += dpp_mov<0x128>(v);
  v += __shfl_xor(v, 4, kWave);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0xB1>(v);
  return v;
}

// Sums (MAX: maxima) of N values over aligned groups of n lanes (n a power of two <= 64,
// uniform), every lane of a group getting its group's result.  Within a 16-lane DPP row the
// steps are register moves: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
// then, with every quad holding one value, row_half_mirror (the other quad of the 8) and
// row_mirror (the other 8 of the 16); beyond 16 lanes, permlane swaps.  The N
// reductions advance step by step together, so their latencies overlap.
template <bool MAX, int N>
__device__ __forceinline__ void lane_groups_reduce(float (&v)[N], int n) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  if (n >= 2) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_mov<0xB1>(v[i]));
  }
  if (n >= 4) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_mov<0x4E>(v[i]));
  }
  if (n >= 8) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_mov<0x141>(v[i]));
  }
  if (n >= 16) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_mov<0x140>(v[i]));
  }
  if (n >= 32) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = op_xor16<MAX>(v[i]);
  }
  if (n >= 64) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = op_xor32<MAX>(v[i]);
  }
}

// Two sums over the whole wave, every lane getting both.
__device__ __forceinline__ void wave_sum_pair(float &a, float &b) {
  float v[2] = {a, b};
  lane_groups_reduce<false>(v, kWave);
  a = v[0];
  b = v[1];
}

}  // namespace moe

// Status helpers for the C-ABI entry points.
#define MOE_REQUIRE(cond, ...)                                                                     \
  do {                                                                                             \
    if (!(cond)) {                                                                                 \
      ::moe::set_error(__VA_ARGS__);                                                               \
      return MOE_STATUS_INVALID_ARGUMENT;                                                          \
    }                                                                                              \
  } while (0)

namespace moe {
// Host-side: whether the byte ranges [a, a + na) and [b, b + nb) share a byte (a null
// pointer is an empty range).  Kernels in which one workgroup writes an output that other
// workgroups still read as an input reject such pairs.
inline bool ranges_overlap(const void *a, int64_t na, const void *b, int64_t nb) {
  if (a == nullptr || b == nullptr || na <= 0 || nb <= 0) return false;
  const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
  return pa < pb + (uintptr_t)nb && pb < pa + (uintptr_t)na;
}
}  // namespace moe

#define MOE_HIP_CHECK(expr)                                                                        \
  do {                                                                                             \
    hipError_t _moe_err = (expr);                                                                  \
    if (_moe_err != hipSuccess) {                                                                  \
      ::moe::set_error("%s failed: %s", #expr, hipGetErrorString(_moe_err));                       \
      return MOE_STATUS_HIP_ERROR;                                                                 \
    }                                                                                              \
  } while (0)

#define MOE_LAUNCH_CHECK() MOE_HIP_CHECK(hipGetLastError())
