// Shared device/host helpers for the aspec_amd HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/aspec_amd.h"

namespace aspec {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kMaskValue = -1.0e30f;  // direct_cp.py:20 MASK_VALUE

// Records a message for aspec_last_error() and returns the status code.
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even float -> bf16 bits (NaN stays NaN), hardware conversion.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const __attribute__((ext_vector_type(2))) float x = {f, 0.f};
  const auto r = __builtin_convertvector(x, __attribute__((ext_vector_type(2))) __bf16);
  return static_cast<uint16_t>(__builtin_bit_cast(uint32_t, r) & 0xffffu);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;

// Two floats -> packed bf16 pair, round-to-nearest-even (one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t x = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2_t));
}

// exp2 as the bare v_exp_f32 (inputs here are <= 8 or -inf; no range fix-up needed).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// s_waitcnt immediates: at most `n` vector-memory loads of this wave outstanding / all LDS
// operations of this wave complete (the other counters left at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
constexpr int kLgkmcnt0 = 0xF | (0x3 << 14) | (0x7 << 4);

// Workgroup barrier for LDS traffic this wave has already waited for. Unlike __syncthreads() it
// does not wait for outstanding global -> LDS loads (the caller waits for the ones it needs with
// vmcnt). The wavefront-scope fences emit nothing; they keep the compiler from moving memory
// operations across the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// All-lane reductions of a wave in registers (no LDS): DPP quad permutes and row mirrors combine
// the 16 lanes of each row (after xor 1 and xor 2 every quad is uniform, so the half mirror and
// the mirror each add an equal partner group), then v_permlane16_swap and v_permlane32_swap
// combine the rows pairwise: swapping the odd rows (halves) of one copy with the even rows
// (halves) of another leaves each lane holding its own value in one result and its partner's in
// the other.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
template <typename Op>
__device__ __forceinline__ uint32_t wave_allreduce_bits(uint32_t v, Op op) {
  v = op(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = op(v, dpp_u32<0x140>(v));  // row_mirror
  const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = op(r16[0], r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return op(r32[0], r32[1]);
}
__device__ __forceinline__ float wave_allsum(float v) {
  return __uint_as_float(wave_allreduce_bits(__float_as_uint(v), [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }));
}
__device__ __forceinline__ float wave_allmax(float v) {  // a NaN operand is skipped, as fmaxf does
  return __uint_as_float(wave_allreduce_bits(__float_as_uint(v), [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}
__device__ __forceinline__ uint32_t wave_allmin(uint32_t v) {
  return wave_allreduce_bits(v, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}

__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

}  // namespace aspec
