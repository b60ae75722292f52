// Packed-row construction (DFlashPackingCollator, aspec/data/utils.py:199-356): one launch copies
// every document's rows of every field into the row (and zero-fills the padding), one launch
// writes the per-token document ids, positions and attention mask from cu_seqlens.
//
// The copies are HBM-bound byte moves: one workgroup per span (spans are split by the host into
// pieces of at most a few hundred KiB so that a 100 MB hidden-state field spreads over the whole
// chip), 16-byte vectors when source, destination and size allow it.
#include "rowops.h"

namespace aspec {
namespace {

constexpr int kCopyThreads = 256;

__global__ void __launch_bounds__(kCopyThreads) pack_copy_kernel(const AspecCopySpan* spans) {
  const AspecCopySpan sp = spans[blockIdx.x];
  const int64_t bytes = sp.bytes;
  const uintptr_t s = reinterpret_cast<uintptr_t>(sp.src);
  const uintptr_t d = reinterpret_cast<uintptr_t>(sp.dst);
  if (((s | d | static_cast<uintptr_t>(bytes)) & 15u) == 0) {
    const int64_t n = bytes >> 4;
    uint4* dst = reinterpret_cast<uint4*>(sp.dst);
    const uint4* src = reinterpret_cast<const uint4*>(sp.src);
    // Four 16-byte loads in flight per thread.
    int64_t i = threadIdx.x;
    for (; i + 3 * kCopyThreads < n; i += 4 * kCopyThreads) {
      uint4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = src ? src[i + j * kCopyThreads] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) dst[i + j * kCopyThreads] = v[j];
    }
    for (; i < n; i += kCopyThreads) dst[i] = src ? src[i] : make_uint4(0, 0, 0, 0);
  } else if (((s | d | static_cast<uintptr_t>(bytes)) & 3u) == 0) {
    const int64_t n = bytes >> 2;
    uint32_t* dst = reinterpret_cast<uint32_t*>(sp.dst);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(sp.src);
    for (int64_t i = threadIdx.x; i < n; i += kCopyThreads) dst[i] = src ? src[i] : 0u;
  } else {
    uint8_t* dst = static_cast<uint8_t*>(sp.dst);
    const uint8_t* src = static_cast<const uint8_t*>(sp.src);
    for (int64_t i = threadIdx.x; i < bytes; i += kCopyThreads) dst[i] = src ? src[i] : 0;
  }
}

// Thread per token: the document is found by binary search over cu_seqlens.
__global__ void __launch_bounds__(256) pack_metadata_kernel(const int32_t* cu, int64_t num_docs,
                                                            int64_t row_length, int64_t* docs,
                                                            int64_t* positions, int64_t* attention) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= row_length) return;
  const int64_t used = cu[num_docs];
  int64_t doc = -1, pos = 0;
  if (t < used) {
    int64_t lo = 0, hi = num_docs;  // invariant: cu[lo] <= t < cu[hi]
    while (hi - lo > 1) {
      const int64_t mid = (lo + hi) >> 1;
      if (cu[mid] <= t) lo = mid;
      else hi = mid;
    }
    doc = lo;
    pos = t - cu[lo];
  }
  if (docs) docs[t] = doc;
  if (positions) positions[t] = pos;
  if (attention) attention[t] = t < used ? 1 : 0;
}

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_pack_copy(const AspecCopySpan* spans, int64_t count, void* stream) {
  if (count < 0) return set_error(ASPEC_ERR_INVALID, "pack copy needs a non-negative span count");
  if (count == 0) return ASPEC_OK;
  if (!spans) return set_error(ASPEC_ERR_INVALID, "pack copy needs a span table");
  if (count > 0x7fffffff) return set_error(ASPEC_ERR_INVALID, "too many pack copy spans");
  hipLaunchKernelGGL(pack_copy_kernel, dim3(static_cast<uint32_t>(count)), dim3(kCopyThreads), 0,
                     static_cast<hipStream_t>(stream), spans);
  return check_launch("pack_copy_kernel");
}

extern "C" int aspec_pack_row_metadata(const int32_t* cu_seqlens, int64_t num_docs,
                                       int64_t row_length, int64_t* ctx_doc_ids,
                                       int64_t* base_position_ids, int64_t* attention_mask,
                                       void* stream) {
  if (num_docs <= 0 || row_length <= 0 || !cu_seqlens)
    return set_error(ASPEC_ERR_INVALID, "packed row metadata needs documents and a row length");
  const int64_t blocks = (row_length + 255) / 256;
  hipLaunchKernelGGL(pack_metadata_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), cu_seqlens, num_docs, row_length,
                     ctx_doc_ids, base_position_ids, attention_mask);
  return check_launch("pack_metadata_kernel");
}
