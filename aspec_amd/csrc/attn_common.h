// Building blocks shared by the DSpark attention kernels: tile staging into LDS (row-major and
// transposed) and the MFMA 32x32x16 bf16 operand conventions.
//
// MFMA convention used throughout (v_mfma_f32_32x32x16_bf16, wave64):
//   lane l = 32*g + c (g = lane group 0/1, c = column 0..31);
//   A operand: lane supplies row c, reduction slots (g, e), e = 0..7;
//   B operand: lane supplies column c, the same reduction slots (g, e);
//   C/D: lane holds column c, register r <-> row (r/4)*8 + g*4 + (r%4).
// Only C's layout is interpreted; for A and B only the pairing of equal (g, e) slots matters.
#pragma once

#include "common.h"

namespace aspec {

constexpr int kHeadDim = 128;
constexpr int kRowLd = kHeadDim + 8;  // row-major tile stride (bf16), 272 B: conflict-free b128 reads

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ uint4 load16(const uint16_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ uint16_t half_of(const uint4& v, int e) {
  const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
  return static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
}

// Reads an A/B operand whose 8 reduction slots live as two runs of 4 contiguous bf16:
// slots e<4 at p[g*4 + e], slots e>=4 at p[8 + g*4 + e-4].
__device__ __forceinline__ bf16x8 read_split_operand(const uint16_t* p, int g) {
  const u32x2 lo = *reinterpret_cast<const u32x2*>(p + g * 4);
  const u32x2 hi = *reinterpret_cast<const u32x2*>(p + 8 + g * 4);
  uint4 v;
  v.x = lo.x;
  v.y = lo.y;
  v.z = hi.x;
  v.w = hi.y;
  return as_bf16x8(v);
}

// Packs C registers [base, base+8) into the bf16 operand whose slot e pairs with C row
// (e/4)*8 + g*4 + e%4 of the 16-row half starting at base/8*16 -- the slot order read_split_operand
// expects from the other operand.
__device__ __forceinline__ bf16x8 pack_c_half(const f32x16& c, int base) {
  uint4 v;
  v.x = pack_bf16x2(c[base + 0], c[base + 1]);
  v.y = pack_bf16x2(c[base + 2], c[base + 3]);
  v.z = pack_bf16x2(c[base + 4], c[base + 5]);
  v.w = pack_bf16x2(c[base + 6], c[base + 7]);
  return as_bf16x8(v);
}

// Stages `rows` rows x 128 dims of a strided [row][head][dim] bf16 tensor into LDS.
//   row_major: dst_rm[r * kRowLd + d]          (may be null)
//   transposed: dst_t[d * t_ld + r]            (may be null; rows must be a multiple of 4)
// Rows at or beyond `limit` are zero-filled. Work items are 4 rows x 8 dims, spread over
// `nthreads` threads starting at `tid`.
__device__ __forceinline__ void stage_tile(const uint16_t* __restrict__ src, int64_t row_stride,
                                           int64_t first_row, int64_t limit, int rows,
                                           uint16_t* dst_rm, uint16_t* dst_t, int t_ld, int tid,
                                           int nthreads) {
  const int items = (rows / 4) * (kHeadDim / 8);
  for (int it = tid; it < items; it += nthreads) {
    const int rg = it / (kHeadDim / 8);
    const int dc = it - rg * (kHeadDim / 8);
    uint4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t row = first_row + rg * 4 + j;
      if (row < limit) {
        v[j] = load16(src + row * row_stride + dc * 8);
      } else {
        v[j] = make_uint4(0, 0, 0, 0);
      }
    }
    if (dst_rm) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<uint4*>(dst_rm + (rg * 4 + j) * kRowLd + dc * 8) = v[j];
    }
    if (dst_t) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x2 w;
        w.x = static_cast<uint32_t>(half_of(v[0], e)) | (static_cast<uint32_t>(half_of(v[1], e)) << 16);
        w.y = static_cast<uint32_t>(half_of(v[2], e)) | (static_cast<uint32_t>(half_of(v[3], e)) << 16);
        *reinterpret_cast<u32x2*>(dst_t + (dc * 8 + e) * t_ld + rg * 4) = w;
      }
    }
  }
}

typedef __attribute__((ext_vector_type(4))) short s16x4;

__device__ __forceinline__ s16x4 ds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(__attribute__((address_space(3))) void*)p);
}

// A operand whose rows are the columns of a row-major LDS tile (a transposed fragment), read with
// gfx950's transpose load ds_read_b64_tr_b16. Within each 16-lane group, lane i receives element
// i%4 of the 8-byte chunks that lanes i/4, i/4+4, i/4+8 and i/4+12 of its group address. Lane s
// therefore addresses row rsub(s) = (s/32)*4 + (s%16)/4 and columns csub(s) = 16*((s/16)%2) +
// 4*(s%4) .. +3, and lane L = 32g + i ends up holding column col0 + i of rows
// row0 + {g*4 + e} (e < 4, first read) and row0 + {8 + g*4 + e-4} (second read): exactly the
// (g, e) reduction slots read_split_operand() / pack_c_half() use.
__device__ __forceinline__ bf16x8 read_tr_operand(const uint16_t* tile, int ld, int row0, int col0,
                                                  int lane) {
  const int rsub = (lane >> 5) * 4 + ((lane & 15) >> 2);
  const int csub = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const uint16_t* p = tile + (row0 + rsub) * ld + col0 + csub;
  const s16x4 lo = ds_read_tr16(p);
  const s16x4 hi = ds_read_tr16(p + 8 * ld);
  const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
  const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
  uint4 v;
  v.x = l2.x;
  v.y = l2.y;
  v.z = h2.x;
  v.w = h2.y;
  return as_bf16x8(v);
}

// Row r (0..31) of C register `reg` for lane group g.
__device__ __forceinline__ int c_row(int reg, int g) { return (reg >> 2) * 8 + g * 4 + (reg & 3); }

// Branch-free two-interval test: key in [cb, ce) or [db, de) (unsigned range compares).
__device__ __forceinline__ bool interval_visible(int key, int cb, int ce, int db, int de) {
  const bool in_ctx = static_cast<uint32_t>(key - cb) < static_cast<uint32_t>(ce - cb);
  const bool in_draft = static_cast<uint32_t>(key - db) < static_cast<uint32_t>(de - db);
  return in_ctx | in_draft;
}

// Row-interval form used per tile: offsets relative to the tile's first key, so the per-element
// test is two compares against values held in registers.
struct RowIntervals {
  int c0, cl, d0, dl;  // context start offset and length, draft start offset and length
  __device__ __forceinline__ void at_tile(int key0, int cb, int ce, int db, int de) {
    c0 = cb - key0;
    cl = ce - cb;
    d0 = db - key0;
    dl = de - db;
  }
  __device__ __forceinline__ bool visible(int off) const {
    return (static_cast<uint32_t>(off - c0) < static_cast<uint32_t>(cl)) |
           (static_cast<uint32_t>(off - d0) < static_cast<uint32_t>(dl));
  }
};

}  // namespace aspec
