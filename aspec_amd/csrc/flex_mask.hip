// Interval-union masks of the reference's cuDNN FlexAttention path on the GPU.
//
//  * `build_dspark_mla_mask` (aspec/models/ops/cudnn_flex_attention.py:53-170): per query row the
//    endpoints (context_end, draft_begin, draft_end) -- or (0, context_begin, context_end,
//    draft_begin, draft_end) when documents or windows are present -- in each batch row's own key
//    space. `_document_run_starts` (cudnn_flex_attention.py:33-50) is a per-row max-scan of the
//    document boundaries; its "one contiguous run per document" check compares the ids of every
//    pair of runs.
//  * The converter from that format (an odd number E of endpoints e: keys [0, e0) and
//    [e(2i-1), e(2i)) are visible; rows of batch b address keys of b only, BSHD by position and THD
//    through cu_seqlens) to the attention kernels' form: at most two intervals per row in the
//    flattened key space of all batch rows.
#include "common.h"

namespace aspec {
namespace {

constexpr int kScanThreads = 1024;
constexpr int kMaxEndpoints = 9;

// One workgroup per batch row: run_start[t] = the first token of t's run of equal document ids,
// and the run starts in order (runs[0 .. count)).
__global__ void __launch_bounds__(kScanThreads) doc_runs_kernel(const int64_t* docs, int64_t T,
                                                                int32_t* run_start, int32_t* runs,
                                                                int32_t* run_count) {
  __shared__ int32_t wave_max_v[kScanThreads / kWave];
  __shared__ int32_t wave_cnt[kScanThreads / kWave];
  const int64_t b = blockIdx.x;
  docs += b * T;
  run_start += b * T;
  runs += b * T;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int32_t carry = 0, count = 0;
  for (int64_t c0 = 0; c0 < T; c0 += kScanThreads) {
    const int64_t t = c0 + tid;
    const bool boundary = t < T && (t == 0 || docs[t] != docs[t - 1]);
    int32_t v = boundary ? static_cast<int32_t>(t) : 0;
    // inclusive max-scan in the wave
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int32_t u = __shfl_up(v, off);
      if (lane >= off) v = max(v, u);
    }
    const uint64_t bmask = __ballot(boundary);
    if (lane == kWave - 1) {
      wave_max_v[wave] = v;
      wave_cnt[wave] = __popcll(bmask);
    }
    __syncthreads();
    int32_t prev_max = carry, prev_cnt = count;
    for (int w = 0; w < wave; ++w) {
      prev_max = max(prev_max, wave_max_v[w]);
      prev_cnt += wave_cnt[w];
    }
    if (t < T) run_start[t] = max(v, prev_max);
    if (boundary) runs[prev_cnt + __popcll(bmask & below)] = static_cast<int32_t>(t);
    int32_t chunk_max = carry, chunk_cnt = count;
    for (int w = 0; w < kScanThreads / kWave; ++w) {
      chunk_max = max(chunk_max, wave_max_v[w]);
      chunk_cnt += wave_cnt[w];
    }
    carry = chunk_max;
    count = chunk_cnt;
    __syncthreads();
  }
  if (tid == 0) run_count[b] = count;
}

// Bit 2 of *flags when a document id owns two runs of one batch row (grid: runs x batch).
__global__ void __launch_bounds__(256) doc_runs_unique_kernel(const int64_t* docs, int64_t T,
                                                              const int32_t* runs,
                                                              const int32_t* run_count,
                                                              int32_t* flags) {
  const int64_t b = blockIdx.y;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int32_t count = run_count[b];
  if (i >= count) return;
  docs += b * T;
  runs += b * T;
  const int64_t d = docs[runs[i]];
  for (int64_t j = 0; j < i; ++j) {
    if (docs[runs[j]] == d) {
      atomicOr(flags, 2);
      return;
    }
  }
}

struct MlaMaskArgs {
  const int64_t* anchors;  // [B][N]
  const uint8_t* keep;     // [B][N]
  const int64_t* docs;     // [B][T] or null
  const int32_t* run_start;
  int64_t batch, n, block, T;
  int causal;
  int64_t sliding, ctx_window;  // <= 0: none
  int num_ends;                 // 3 or 5
  int32_t* mask;                // [num_ends][B * N * block]
  int32_t* flags;
};

// One thread per query row: the endpoint rows of cudnn_flex_attention.py:99-169.
__global__ void __launch_bounds__(256) mla_mask_kernel(MlaMaskArgs a) {
  const int64_t lq = a.n * a.block;
  const int64_t rows = a.batch * lq;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const int64_t b = row / lq;
  const int64_t qi = row - b * lq;
  const int64_t r = qi / a.block;
  const int64_t o = qi - r * a.block;
  const int64_t anchor = a.anchors[b * a.n + r];
  const bool in_range = anchor >= 0 && anchor < a.T;
  if (!in_range) atomicOr(a.flags, 1);
  const int64_t at = in_range ? anchor : 0;  // reads stay in bounds; the host raises on bit 1
  bool valid = a.keep[b * a.n + r] != 0;
  int64_t cb = 0;
  if (a.docs) {
    cb = a.run_start[b * a.T + at];
    valid = valid && a.docs[b * a.T + at] >= 0;
  }
  const int64_t ce = anchor;
  const int64_t base = a.T + r * a.block;
  int64_t lb = base, le = base + a.block;
  if (a.causal) le = base + o + 1;
  if (a.ctx_window > 0) cb = max(cb, anchor - a.ctx_window);
  if (a.sliding > 0) {
    cb = max(cb, anchor + o - a.sliding + 1);
    cb = min(cb, ce);
    lb = base + max(o - a.sliding + 1, (int64_t)0);
    le = min(le, base + min(o + a.sliding, a.block));
  }
  int64_t e[5];
  if (a.num_ends == 3) {
    e[0] = ce; e[1] = lb; e[2] = le;
  } else {
    e[0] = 0; e[1] = cb; e[2] = ce; e[3] = lb; e[4] = le;
  }
  for (int i = 0; i < a.num_ends; ++i)
    a.mask[static_cast<int64_t>(i) * rows + row] = valid ? static_cast<int32_t>(e[i]) : 0;
}

struct IntervalArgs {
  const int32_t* mask;  // [E][rows]
  int num_ends;
  int64_t rows;
  const int32_t* cu_q;  // [segments + 1] or null (BSHD: fixed lengths)
  const int32_t* cu_k;
  int64_t segments, lq, lk;
  int32_t* ends;        // [5][rows]
  int32_t* flags;
};

// One thread per query row: the union of the row's intervals, merged, as at most two intervals
// shifted into the flattened key space. Bit 1 of *flags: an endpoint outside [0, segment keys];
// bit 2: more than two disjoint intervals; bit 4: a row outside every THD query segment.
__global__ void __launch_bounds__(256) flex_intervals_kernel(IntervalArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= a.rows) return;
  int64_t key_base, seg_keys;
  if (a.cu_q) {
    int64_t lo = 0, hi = a.segments;  // last segment s with cu_q[s] <= row
    while (hi - lo > 1) {
      const int64_t mid = (lo + hi) >> 1;
      if (a.cu_q[mid] <= row) lo = mid; else hi = mid;
    }
    if (row < a.cu_q[lo] || row >= a.cu_q[lo + 1]) {
      atomicOr(a.flags, 4);
      for (int i = 0; i < 5; ++i) a.ends[static_cast<int64_t>(i) * a.rows + row] = 0;
      return;
    }
    key_base = a.cu_k[lo];
    seg_keys = a.cu_k[lo + 1] - a.cu_k[lo];
  } else {
    const int64_t b = row / a.lq;
    key_base = b * a.lk;
    seg_keys = a.lk;
  }
  int64_t lo_v[kMaxEndpoints], hi_v[kMaxEndpoints];
  int n = 0;
  int bad = 0;
  for (int i = 0; i < a.num_ends; i += 2) {
    const int64_t lo = i == 0 ? 0 : a.mask[static_cast<int64_t>(i - 1) * a.rows + row];
    const int64_t hi = a.mask[static_cast<int64_t>(i) * a.rows + row];
    if (lo < 0 || lo > seg_keys || hi < 0 || hi > seg_keys) bad |= 1;
    if (hi > lo) {
      lo_v[n] = lo;
      hi_v[n] = hi;
      ++n;
    }
  }
  // sort by start (at most kMaxEndpoints / 2 + 1 intervals), then merge touching ones
  for (int i = 1; i < n; ++i)
    for (int j = i; j > 0 && lo_v[j] < lo_v[j - 1]; --j) {
      const int64_t tl = lo_v[j], th = hi_v[j];
      lo_v[j] = lo_v[j - 1]; hi_v[j] = hi_v[j - 1];
      lo_v[j - 1] = tl; hi_v[j - 1] = th;
    }
  int m = 0;
  for (int i = 0; i < n; ++i) {
    if (m > 0 && lo_v[i] <= hi_v[m - 1]) {
      hi_v[m - 1] = max(hi_v[m - 1], hi_v[i]);
    } else {
      lo_v[m] = lo_v[i];
      hi_v[m] = hi_v[i];
      ++m;
    }
  }
  if (m > 2) bad |= 2;
  if (bad) atomicOr(a.flags, bad);
  int64_t out[4] = {0, 0, 0, 0};
  if (!bad) {
    for (int i = 0; i < m; ++i) {
      out[2 * i] = key_base + min(lo_v[i], seg_keys);
      out[2 * i + 1] = key_base + min(hi_v[i], seg_keys);
    }
  }
  a.ends[row] = 0;
  for (int i = 0; i < 4; ++i) a.ends[static_cast<int64_t>(i + 1) * a.rows + row] = static_cast<int32_t>(out[i]);
}

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_dspark_mla_mask_workspace_bytes(int64_t batch, int64_t context_length,
                                                     size_t* bytes) {
  if (batch <= 0 || context_length <= 0 || !bytes)
    return set_error(ASPEC_ERR_INVALID, "mask workspace needs a positive batch and context length");
  *bytes = static_cast<size_t>(2 * batch * context_length + batch) * sizeof(int32_t);
  return ASPEC_OK;
}

extern "C" int aspec_dspark_mla_mask(const int64_t* anchors, const uint8_t* keep,
                                     const int64_t* ctx_doc_ids, int64_t batch, int64_t num_anchors,
                                     int64_t block_size, int64_t context_length, int is_causal,
                                     int64_t sliding_window, int64_t context_window,
                                     int32_t* mask_func, void* workspace, int32_t* status_flags,
                                     void* stream) {
  if (batch <= 0 || num_anchors < 0 || block_size <= 0 || context_length <= 0)
    return set_error(ASPEC_ERR_INVALID, "invalid DSpark mask geometry");
  if (batch > 65535)
    return set_error(ASPEC_ERR_UNSUPPORTED, "batch %lld exceeds 65535", (long long)batch);
  if (context_length + num_anchors * block_size >= (1LL << 31) - 1 ||
      batch * num_anchors * block_size >= (1LL << 31) - 1 || batch * context_length >= (1LL << 31) - 1)
    return set_error(ASPEC_ERR_INVALID, "DSpark mask exceeds int32 indexing");
  if (!mask_func || !status_flags || (num_anchors > 0 && (!anchors || !keep)))
    return set_error(ASPEC_ERR_INVALID, "anchors, keep, mask and status buffers are required");
  if (ctx_doc_ids && !workspace)
    return set_error(ASPEC_ERR_INVALID, "document ids need the mask workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t* run_start = static_cast<int32_t*>(workspace);
  int rc;
  if (ctx_doc_ids) {
    int32_t* runs = run_start + batch * context_length;
    int32_t* count = runs + batch * context_length;
    hipLaunchKernelGGL(doc_runs_kernel, dim3(static_cast<uint32_t>(batch)), dim3(kScanThreads), 0, s,
                       ctx_doc_ids, context_length, run_start, runs, count);
    if ((rc = check_launch("doc_runs_kernel"))) return rc;
    hipLaunchKernelGGL(doc_runs_unique_kernel,
                       dim3(static_cast<uint32_t>((context_length + 255) / 256), static_cast<uint32_t>(batch)),
                       dim3(256), 0, s, ctx_doc_ids, context_length, runs, count, status_flags);
    if ((rc = check_launch("doc_runs_unique_kernel"))) return rc;
  }
  MlaMaskArgs a;
  a.anchors = anchors;
  a.keep = keep;
  a.docs = ctx_doc_ids;
  a.run_start = run_start;
  a.batch = batch;
  a.n = num_anchors;
  a.block = block_size;
  a.T = context_length;
  a.causal = is_causal;
  a.sliding = sliding_window;
  a.ctx_window = context_window;
  a.num_ends = (ctx_doc_ids || sliding_window > 0 || context_window > 0) ? 5 : 3;
  a.mask = mask_func;
  a.flags = status_flags;
  const int64_t rows = batch * num_anchors * block_size;
  if (rows == 0) return ASPEC_OK;
  hipLaunchKernelGGL(mla_mask_kernel, dim3(static_cast<uint32_t>((rows + 255) / 256)), dim3(256), 0, s, a);
  return check_launch("mla_mask_kernel");
}

extern "C" int aspec_flex_mask_intervals(const int32_t* mask_func, int64_t num_endpoints,
                                         int64_t rows, const int32_t* cu_seqlens_q,
                                         const int32_t* cu_seqlens_k, int64_t num_segments,
                                         int64_t query_length, int64_t key_length,
                                         int32_t* endpoints, int32_t* status_flags, void* stream) {
  if (num_endpoints <= 0 || num_endpoints > kMaxEndpoints || num_endpoints % 2 == 0)
    return set_error(ASPEC_ERR_UNSUPPORTED, "interval masks need an odd endpoint count up to %d, got %lld",
                     kMaxEndpoints, (long long)num_endpoints);
  if (rows <= 0 || !mask_func || !endpoints || !status_flags)
    return set_error(ASPEC_ERR_INVALID, "interval mask conversion needs rows, a mask and outputs");
  if ((cu_seqlens_q == nullptr) != (cu_seqlens_k == nullptr))
    return set_error(ASPEC_ERR_INVALID, "THD masks require both cumulative lengths");
  if (cu_seqlens_q) {
    if (num_segments <= 0) return set_error(ASPEC_ERR_INVALID, "THD masks need at least one segment");
  } else if (query_length <= 0 || key_length <= 0 || rows % query_length) {
    return set_error(ASPEC_ERR_INVALID, "BSHD masks need rows = batch x query length");
  } else if ((rows / query_length) * key_length >= (1LL << 31) - 1) {
    return set_error(ASPEC_ERR_INVALID, "flattened keys exceed int32 indexing");
  }
  IntervalArgs a;
  a.mask = mask_func;
  a.num_ends = static_cast<int>(num_endpoints);
  a.rows = rows;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.segments = num_segments;
  a.lq = query_length;
  a.lk = key_length;
  a.ends = endpoints;
  a.flags = status_flags;
  hipLaunchKernelGGL(flex_intervals_kernel, dim3(static_cast<uint32_t>((rows + 255) / 256)), dim3(256),
                     0, static_cast<hipStream_t>(stream), a);
  return check_launch("flex_intervals_kernel");
}
