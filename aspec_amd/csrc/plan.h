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

struct PlanView {
  int64_t nmf, nnf, nmb, nnb;
  int32_t* f_classes;
  int32_t* f_pcnt;
  int32_t* f_pidx;
  int32_t* f_fcnt;
  int32_t* f_fidx;
  int32_t* b_classes;
  int32_t* b_pcnt;
  int32_t* b_pidx;
  int32_t* b_fcnt;
  int32_t* b_fidx;
  size_t bytes;
};

inline PlanView plan_view(void* base, int64_t nq, int64_t nk) {
  PlanView p;
  p.nmf = (nq + kFwdTileM - 1) / kFwdTileM;
  p.nnf = (nk + kFwdTileN - 1) / kFwdTileN;
  p.nmb = (nq + kBwdTileM - 1) / kBwdTileM;
  p.nnb = (nk + kBwdTileN - 1) / kBwdTileN;
  int32_t* cur = static_cast<int32_t*>(base);
  size_t used = 0;
  auto take = [&](int64_t count) {
    int32_t* out = cur ? cur + used : nullptr;
    used += static_cast<size_t>((count + 63) / 64 * 64);  // 256-byte aligned pieces
    return out;
  };
  p.f_classes = take(p.nmf * p.nnf);
  p.f_pcnt = take(p.nmf);
  p.f_pidx = take(p.nmf * p.nnf);
  p.f_fcnt = take(p.nmf);
  p.f_fidx = take(p.nmf * p.nnf);
  p.b_classes = take(p.nmb * p.nnb);
  p.b_pcnt = take(p.nnb);
  p.b_pidx = take(p.nnb * p.nmb);
  p.b_fcnt = take(p.nnb);
  p.b_fidx = take(p.nnb * p.nmb);
  p.bytes = used * sizeof(int32_t);
  return p;
}

int launch_tile_metadata(const int32_t* ends, int64_t nq, int64_t nk, int64_t tm, int64_t tn,
                         int pad_visible, int32_t* classes, int32_t* fpc, int32_t* fpi,
                         int32_t* ffc, int32_t* ffi, int32_t* bpc, int32_t* bpi, int32_t* bfc,
                         int32_t* bfi, hipStream_t stream);

}  // namespace aspec
