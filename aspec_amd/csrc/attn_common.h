// Building blocks shared by the DSpark attention kernels: the swizzled LDS tile layout and the
// MFMA 32x32x16 bf16 operand conventions.
//
// MFMA convention used throughout (v_mfma_f32_32x32x16_bf16, wave64):
//   lane l = 32*g + c (g = lane group 0/1, c = column 0..31);
//   A operand: lane supplies row c, reduction slots (g, e), e = 0..7;
//   B operand: lane supplies column c, the same reduction slots (g, e);
//   C/D: lane holds column c, register r <-> row (r/4)*8 + g*4 + (r%4).
// Only C's layout is interpreted; for A and B only the pairing of equal (g, e) slots matters.
// Row-major operands put slot (g, e) of k-step ds at dim 16*ds + 8*g + e; transposed operands and
// packed C halves put it at reduction row (e/4)*8 + g*4 + e%4 of the 16-row k-step.
#pragma once

#include "common.h"

namespace aspec {

constexpr int kHeadDim = 128;
constexpr int kRowLd = kHeadDim;  // LDS tile row: 128 bf16 = 256 B, unpadded

// LDS tiles hold rows of 128 bf16 as 16 chunks of 16 B; logical chunk j of row r is stored at
// chunk j ^ swz(r). swz is built so that every LDS read pattern used here is bank-conflict free,
// for 64 banks (256 B per cycle) and for 32 (128 B per cycle):
//  * row reads (ds_read_b128, lane c reads row c, all lanes the same logical chunk): swz is a
//    bijection on r % 16, and its low three bits a bijection on r % 8;
//  * transpose reads (ds_read_b64_tr_b16, 4 consecutive rows x 4 adjacent chunks per 32 lanes,
//    4 rows x 2 chunks per 16 lanes): bits 2-3 and bits 1-2 of swz are bijections on r % 4.
// With r = b3 b2 b1 b0: swz = (b1 ^ b3, b0, b1, b2).
__device__ __forceinline__ int swz(int row) {
  return ((row >> 2) & 1) | (row & 2) | ((row & 1) << 2) | ((((row >> 1) ^ (row >> 3)) & 1) << 3);
}

// Element offset of (row, dims col .. col+7) in a swizzled tile (col % 8 == 0).
__device__ __forceinline__ int tile_chunk_off(int row, int col) {
  return row * kRowLd + (((col >> 3) ^ swz(row)) << 3);
}

// Hides a value's origin from the optimizer (emits no instruction). Applied to the lane offsets
// inside a tile loop, it keeps the per-step swizzled addresses (one XOR each) from being hoisted
// out of the loop into a register apiece.
__device__ __forceinline__ void opaque(int& x) { asm volatile("" : "+v"(x)); }

// Element offset of this lane's row-major operand read at k-step 0 (dims 8*g .. 8*g+7 of `row`).
// The read of k-step ds (dims 16*ds + 8*g ..) is at row_operand_off(row, g) ^ (ds << 4).
__device__ __forceinline__ int row_operand_off(int row, int g) {
  return row * kRowLd + ((g ^ swz(row)) << 3);
}

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;

// Operands are carried as 16-byte bf16x8 values whatever the element type; F16 selects the fp16
// instruction (v_mfma_f32_32x32x16_f16) over the same bits.
template <bool F16 = false>
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Two floats -> a packed pair of the element type, round-to-nearest-even.
template <bool F16 = false>
__device__ __forceinline__ uint32_t pack_elem2(float lo, float hi) {
  if constexpr (F16) {
    const f32x2_t x = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2_t));
  } else {
    return pack_bf16x2(lo, hi);
  }
}

// One element of the element type (bits) -> float.
template <bool F16 = false>
__device__ __forceinline__ float elem_to_f32(uint16_t v) {
  if constexpr (F16)
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
  else
    return bf16_to_f32(v);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ uint4 load16(const uint16_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// bf16 element e (0..7) of a 16-byte chunk.
__device__ __forceinline__ uint16_t half_of(const uint4& v, int e) {
  const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
  return static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
}

// Packs C registers [base, base+8) into the bf16 operand whose slot e pairs with C row
// (e/4)*8 + g*4 + e%4 of the 16-row half starting at base/8*16.
template <bool F16 = false>
__device__ __forceinline__ bf16x8 pack_c_half(const f32x16& c, int base) {
  uint4 v;
  v.x = pack_elem2<F16>(c[base + 0], c[base + 1]);
  v.y = pack_elem2<F16>(c[base + 2], c[base + 3]);
  v.z = pack_elem2<F16>(c[base + 4], c[base + 5]);
  v.w = pack_elem2<F16>(c[base + 6], c[base + 7]);
  return as_bf16x8(v);
}

typedef __attribute__((ext_vector_type(4))) short s16x4;

__device__ __forceinline__ s16x4 ds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(__attribute__((address_space(3))) void*)p);
}

// Transposed A operands read from a row-major swizzled tile with gfx950's transpose load
// ds_read_b64_tr_b16. Within each 16-lane group, lane i receives element i%4 of the 8-byte pieces
// that lanes i/4, i/4+4, i/4+8 and i/4+12 of its group address. Lane s therefore addresses row
// rsub(s) = (s/32)*4 + (s%16)/4 and columns csub(s) = 16*((s/16)%2) + 4*(s%4) .. +3, and lane
// L = 32g + i ends up holding column col0 + i of rows row0 + {g*4 + e} (e < 4, first read) and
// row0 + {8 + g*4 + e-4} (second read): the (g, e) slots pack_c_half() produces.
// `lo` / `hi` are this lane's element offsets for row0 = 0, col0 = 0; they hold for any row0 that
// is a multiple of 16 (swz depends on row % 16 only) and any col0 that is a multiple of 32
// (col0 / 8 only flips chunk bits 2-3, which the lane's own chunk bits 0-1 do not touch).
struct TrOffsets {
  int lo, hi;
  __device__ __forceinline__ explicit TrOffsets(int lane) {
    const int rsub = (lane >> 5) * 4 + ((lane & 15) >> 2);
    const int csub = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    lo = rsub * kRowLd + (((csub >> 3) ^ swz(rsub)) << 3) + (csub & 7);
    hi = (rsub + 8) * kRowLd + (((csub >> 3) ^ swz(rsub + 8)) << 3) + (csub & 7);
  }
};

// Transposed fragment: rows row0 .. row0+15 (the reduction; row0 % 16 == 0), columns
// col0 .. col0+31 (the MFMA rows; col0 % 32 == 0).
__device__ __forceinline__ bf16x8 read_tr_operand(const uint16_t* tile, const TrOffsets& o,
                                                  int row0, int col0) {
  const s16x4 lo = ds_read_tr16(tile + row0 * kRowLd + (o.lo ^ col0));
  const s16x4 hi = ds_read_tr16(tile + row0 * kRowLd + (o.hi ^ col0));
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

// Bits [lo, hi) of the 32-key word starting at `base`.
__device__ __forceinline__ uint32_t interval_bits(int lo, int hi, int base) {
  const int a = min(max(lo - base, 0), 32);
  const int e = min(max(hi - base, 0), 32);
  return e > a ? static_cast<uint32_t>((1ull << e) - (1ull << a)) : 0u;
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
  // Visibility of keys 32*kb .. 32*kb+31 of the tile as one word, shifted right by 4*g so that
  // bit (r/4)*8 + r%4 is the key of C register r for lane group g (c_row(r, g) = that + 4*g).
  __device__ __forceinline__ uint32_t word(int kb, int g) const {
    return (interval_bits(c0, c0 + cl, kb * 32) | interval_bits(d0, d0 + dl, kb * 32)) >> (4 * g);
  }
};

// max(x of this lane, x of lane ^ 32) with gfx950's v_permlane32_swap (no LDS round trip):
// swapping lanes 32-63 of one copy with lanes 0-31 of another leaves each lane holding its own
// value in one result and its partner's in the other.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// The score of C register r, or -inf when its key is not visible (`w` from RowIntervals::word).
__device__ __forceinline__ float masked_score(float s, uint32_t w, int r) {
  const int keep = __builtin_amdgcn_sbfe(static_cast<int>(w), (r >> 2) * 8 + (r & 3), 1);  // 0 or -1
  return __int_as_float((__float_as_int(s) & keep) | (~keep & static_cast<int>(0xff800000u)));
}

}  // namespace aspec
