// Attention plan: tile lists at the attention kernels' own geometry, carved out of one opaque
// caller-owned device buffer.
#pragma once

#include "common.h"

namespace aspec {

// Query-major kernels (forward, dQ): tiles of kFwdTileM query rows x kFwdTileN keys.
constexpr int kFwdTileM = 32;
constexpr int kFwdTileN = 64;
// Key-major kernel (dK/dV): tiles of kBwdTileM query rows x kBwdTileN keys.
constexpr int kBwdTileM = 32;
constexpr int kBwdTileN = 128;
// dK/dV work units: a key tile seen by more than kBwdChunk query tiles is split into units of
// max(kBwdChunk, ceil(count / kMaxChunks)) query tiles (the last one shorter), so at most
// kMaxChunks of them, each writing an fp32 partial into its own slot; the finalize sums the slots
// in unit order, so dK/dV are deterministic. A unit's list of query tiles (at most kUnitListCap) is
// staged in LDS.
constexpr int kBwdChunk = 64;
constexpr int kMaxChunks = 4;
constexpr int kUnitListCap = 2048;
// List entries carry the tile index in the low bits and "full tile" in bit 31.
constexpr uint32_t kFullBit = 0x80000000u;
// dK/dV work units are packed as (key tile << kUnitChunkBits) | chunk.
constexpr int kUnitChunkBits = 12;

struct PlanView {
  int64_t nmf, nnf, nmb, nnb, max_units;
  int32_t* f_classes;
  int32_t* f_cnt;     // [nmf] visible key tiles per query tile
  int32_t* f_list;    // [nmf][nnf] ascending key tiles | kFullBit
  int32_t* b_classes;
  int32_t* b_cnt;     // [nnb] visible query tiles per key tile
  int32_t* b_list;    // [nnb][nmb] descending query tiles | kFullBit
  int32_t* b_chunks;  // [nnb] work units of each key tile (1 .. kMaxChunks)
  int32_t* b_units;   // [max_units] (key tile << kUnitChunkBits | chunk), longest first
  int32_t* b_nunits;  // [1]
  size_t bytes;
};

// Unit length (query tiles) and unit count of a key tile seen by `count` query tiles. Full
// kBwdChunk units plus a short remainder while that takes at most kMaxChunks units: the short
// units, sorted last, fill the tail of the launch.
__host__ __device__ inline int bwd_unit_len(int count) {
  const int q = (count + kMaxChunks - 1) / kMaxChunks;
  return q > kBwdChunk ? q : kBwdChunk;
}
__host__ __device__ inline int bwd_chunks(int count) {
  return count <= 0 ? 1 : (count + bwd_unit_len(count) - 1) / bwd_unit_len(count);
}

inline PlanView plan_view(void* base, int64_t nq, int64_t nk) {
  PlanView p;
  p.nmf = (nq + kFwdTileM - 1) / kFwdTileM;
  p.nnf = (nk + kFwdTileN - 1) / kFwdTileN;
  p.nmb = (nq + kBwdTileM - 1) / kBwdTileM;
  p.nnb = (nk + kBwdTileN - 1) / kBwdTileN;
  p.max_units = p.nnb * kMaxChunks;
  int32_t* cur = static_cast<int32_t*>(base);
  size_t used = 0;
  auto take = [&](int64_t count) {
    int32_t* out = cur ? cur + used : nullptr;
    used += static_cast<size_t>((count + 63) / 64 * 64);  // 256-byte aligned pieces
    return out;
  };
  p.f_classes = take(p.nmf * p.nnf);
  p.f_cnt = take(p.nmf);
  p.f_list = take(p.nmf * p.nnf);
  p.b_classes = take(p.nmb * p.nnb);
  p.b_cnt = take(p.nnb);
  p.b_list = take(p.nnb * p.nmb);
  p.b_chunks = take(p.nnb);
  p.b_units = take(p.max_units);
  p.b_nunits = take(1);
  p.bytes = used * sizeof(int32_t);
  return p;
}

int launch_tile_metadata(const int32_t* ends, int64_t nq, int64_t nk, int64_t tm, int64_t tn,
                         int pad_visible, int32_t* classes, int32_t* fpc, int32_t* fpi,
                         int32_t* ffc, int32_t* ffi, int32_t* bpc, int32_t* bpi, int32_t* bfc,
                         int32_t* bfi, hipStream_t stream);

}  // namespace aspec
