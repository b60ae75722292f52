// Helpers shared by the row-level kernels (packing, anchor sampling, output blocks, DSpark
// targets): reading loss / attention masks of any dtype, and a workgroup-wide exclusive scan.
#pragma once

#include "common.h"

namespace aspec {

// Truth of `mask[i] > 0.5` for the mask dtypes of the C ABI (ASPEC_MASK_*). Integer masks compare
// as their value (v > 0.5 <=> v >= 1), bool / uint8 as nonzero.
__device__ __forceinline__ bool mask_set(const void* mask, int dtype, int64_t i) {
  switch (dtype) {
    case ASPEC_MASK_F32: return static_cast<const float*>(mask)[i] > 0.5f;
    case ASPEC_MASK_I64: return static_cast<const int64_t*>(mask)[i] > 0;
    case ASPEC_MASK_I32: return static_cast<const int32_t*>(mask)[i] > 0;
    case ASPEC_MASK_U8: return static_cast<const uint8_t*>(mask)[i] != 0;
    case ASPEC_MASK_BF16: return bf16_to_f32(static_cast<const uint16_t*>(mask)[i]) > 0.5f;
    default: return static_cast<float>(static_cast<const _Float16*>(mask)[i]) > 0.5f;
  }
}

// Truth of `mask[i] != 0` (`.bool()`), for attention masks.
__device__ __forceinline__ bool mask_nonzero(const void* mask, int dtype, int64_t i) {
  switch (dtype) {
    case ASPEC_MASK_F32: return static_cast<const float*>(mask)[i] != 0.f;
    case ASPEC_MASK_I64: return static_cast<const int64_t*>(mask)[i] != 0;
    case ASPEC_MASK_I32: return static_cast<const int32_t*>(mask)[i] != 0;
    case ASPEC_MASK_U8: return static_cast<const uint8_t*>(mask)[i] != 0;
    case ASPEC_MASK_BF16: return (static_cast<const uint16_t*>(mask)[i] & 0x7fffu) != 0;
    default: return (static_cast<const uint16_t*>(mask)[i] & 0x7fffu) != 0;
  }
}

inline bool valid_mask_dtype(int dtype) { return dtype >= ASPEC_MASK_F32 && dtype <= ASPEC_MASK_F16; }

// Exclusive scan of one int per thread over the whole workgroup (blockDim.x a multiple of 64,
// at most 1024). `scratch` holds >= 17 ints of LDS. Returns the thread's exclusive prefix and sets
// `total`. Contains barriers: every thread of the workgroup must call it.
__device__ __forceinline__ int block_exclusive_scan(int v, int* scratch, int& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < nwaves; ++w) {
      const int t = scratch[w];
      scratch[w] = run;
      run += t;
    }
    scratch[16] = run;
  }
  __syncthreads();
  const int result = scratch[wave] + incl - v;
  total = scratch[16];
  __syncthreads();
  return result;
}

}  // namespace aspec
