// Attention plan build: tile classes at the kernels' geometry, merged ordered lists with a
// "full tile" flag, and the dK/dV work units (key tile, chunk) in longest-first order.
#include "plan.h"

namespace aspec {
namespace {

// One wave per query tile: ascending list of visible key tiles.
__global__ void __launch_bounds__(kWave) plan_rows_kernel(PlanView p) {
  const int64_t m = blockIdx.x;
  const int lane = threadIdx.x;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int32_t* cls = p.f_classes + m * p.nnf;
  int32_t* out = p.f_list + m * p.nnf;
  int count = 0;
  for (int64_t n0 = 0; n0 < p.nnf; n0 += kWave) {
    const int64_t n = n0 + lane;
    const int c = n < p.nnf ? cls[n] : 0;
    const uint64_t mask = __ballot(c != 0);
    if (c != 0) out[count + __popcll(mask & below)] = static_cast<int32_t>(n | (c == 2 ? kFullBit : 0u));
    count += __popcll(mask);
  }
  if (lane == 0) p.f_cnt[m] = count;
}

// One wave per key tile: descending list of the query tiles that see it, and its unit count.
__global__ void __launch_bounds__(kWave) plan_cols_kernel(PlanView p) {
  const int64_t n = blockIdx.x;
  const int lane = threadIdx.x;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int32_t* out = p.b_list + n * p.nmb;
  int count = 0;
  for (int64_t top = p.nmb - 1; top >= 0; top -= kWave) {
    const int64_t m = top - lane;
    const int c = m >= 0 ? p.b_classes[m * p.nnb + n] : 0;
    const uint64_t mask = __ballot(c != 0);
    if (c != 0) out[count + __popcll(mask & below)] = static_cast<int32_t>(m | (c == 2 ? kFullBit : 0u));
    count += __popcll(mask);
  }
  if (lane == 0) {
    p.b_cnt[n] = count;
    p.b_chunks[n] = bwd_chunks(count);
  }
}

// One workgroup: counting sort of the (key tile, chunk) units by unit length, longest first. Lengths
// up to kBwdChunk have a bin each; longer ones share bins 16 lengths wide (their order within a
// bin is arbitrary, which only affects load balance).
constexpr int kUnitThreads = 1024;
constexpr int kLenBins = kBwdChunk + 1 + (kUnitListCap - kBwdChunk + 15) / 16;
static_assert(kLenBins <= kUnitThreads, "one thread per histogram bin");

__device__ __forceinline__ int len_bin(int len) {
  return len <= kBwdChunk ? len : kBwdChunk + 1 + (len - kBwdChunk - 1) / 16;
}

__global__ void __launch_bounds__(kUnitThreads) plan_units_kernel(PlanView p) {
  __shared__ int32_t hist[kLenBins];
  __shared__ int32_t cursor[kLenBins];
  __shared__ int32_t total;
  const int tid = threadIdx.x;
  if (tid < kLenBins) hist[tid] = 0;
  if (tid == 0) total = 0;
  __syncthreads();
  for (int64_t n = tid; n < p.nnb; n += blockDim.x) {
    const int cnt = p.b_cnt[n];
    const int chunks = p.b_chunks[n];
    const int len = bwd_unit_len(cnt);
    for (int c = 0; c < chunks; ++c) atomicAdd(&hist[len_bin(min(len, max(0, cnt - c * len)))], 1);
    atomicAdd(&total, chunks);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int b = kLenBins - 1; b >= 0; --b) {
      cursor[b] = run;
      run += hist[b];
    }
    p.b_nunits[0] = total;
  }
  __syncthreads();
  for (int64_t n = tid; n < p.nnb; n += blockDim.x) {
    const int cnt = p.b_cnt[n];
    const int chunks = p.b_chunks[n];
    const int len = bwd_unit_len(cnt);
    for (int c = 0; c < chunks; ++c) {
      const int pos = atomicAdd(&cursor[len_bin(min(len, max(0, cnt - c * len)))], 1);
      p.b_units[pos] = static_cast<int32_t>((n << kUnitChunkBits) | c);
    }
  }
}

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_dspark_plan_bytes(int64_t num_queries, int64_t num_keys, size_t* bytes) {
  if (num_queries <= 0 || num_keys <= 0 || !bytes)
    return set_error(ASPEC_ERR_INVALID, "plan size needs positive query/key counts");
  *bytes = plan_view(nullptr, num_queries, num_keys).bytes;
  return ASPEC_OK;
}

extern "C" int aspec_dspark_plan_build(const int32_t* endpoints, int64_t num_queries,
                                       int64_t num_keys, void* plan, void* stream) {
  if (num_queries <= 0 || num_keys <= 0 || !endpoints || !plan)
    return set_error(ASPEC_ERR_INVALID, "plan build needs endpoints, a plan buffer and sizes");
  const PlanView p = plan_view(plan, num_queries, num_keys);
  if (p.nnb >= (1LL << (31 - kUnitChunkBits)) || p.nmb > static_cast<int64_t>(kMaxChunks) * kUnitListCap)
    return set_error(ASPEC_ERR_UNSUPPORTED, "attention plan too large (%lld queries, %lld keys)",
                     (long long)num_queries, (long long)num_keys);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = launch_tile_metadata(endpoints, num_queries, num_keys, kFwdTileM, kFwdTileN, 0,
                                p.f_classes, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                nullptr, nullptr, s);
  if (rc) return rc;
  rc = launch_tile_metadata(endpoints, num_queries, num_keys, kBwdTileM, kBwdTileN, 0, p.b_classes,
                            nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, s);
  if (rc) return rc;
  hipLaunchKernelGGL(plan_rows_kernel, dim3(static_cast<uint32_t>(p.nmf)), dim3(kWave), 0, s, p);
  if ((rc = check_launch("plan_rows_kernel"))) return rc;
  hipLaunchKernelGGL(plan_cols_kernel, dim3(static_cast<uint32_t>(p.nnb)), dim3(kWave), 0, s, p);
  if ((rc = check_launch("plan_cols_kernel"))) return rc;
  hipLaunchKernelGGL(plan_units_kernel, dim3(1), dim3(kUnitThreads), 0, s, p);
  return check_launch("plan_units_kernel");
}
