// Anchor layout (aspec/models/ops/anchors.py): the document sampler, the per-sample sampler and
// the validation of injected anchors.
//
// The samplers follow the reference's arithmetic step by step so that, given the same uniform
// draws (torch.rand with the caller's generator), they select the same anchors:
//   candidates (anchors.py:31-53): position i < count = min(max(S - B, 0) + 1, S - 1) is usable
//     if loss_mask[i] and loss_mask[i + 1] are set (plus attention-mask terms when given, and for
//     the document sampler: same document at i and i + 1, document longer than B, i <= end - B);
//   `ordered` (the ascending valid positions) is a stream compaction here instead of a sort;
//   count c, divisor max(c, 1), stride clamp(c / A, 1, gap + 1), phase trunc(u * divisor) in fp32;
//   slot s selects ordered[start + (phase + s * stride) % divisor] and is kept if s < c.
// One workgroup per row: a row is at most a few hundred thousand tokens, well within one
// workgroup's reach at the latency of a handful of scans.
#include "rowops.h"

namespace aspec {
namespace {

constexpr int kSamplerThreads = 1024;
constexpr int kMaxSamplerDocs = 4096;
constexpr int kDocsPerThread = kMaxSamplerDocs / kSamplerThreads;

// Exclusive scan of kMaxSamplerDocs values held kDocsPerThread per thread (thread t owns entries
// [t * kDocsPerThread, ...)); in place in `vals`, returns the total.
__device__ int64_t scan_docs(int64_t* vals, int64_t n, int* scratch) {
  const int base = threadIdx.x * kDocsPerThread;
  int64_t local[kDocsPerThread];
  int64_t sum = 0;
#pragma unroll
  for (int j = 0; j < kDocsPerThread; ++j) {
    local[j] = base + j < n ? vals[base + j] : 0;
    sum += local[j];
  }
  // Sums fit in int32 here (token counts of one row).
  int total;
  int64_t run = block_exclusive_scan(static_cast<int>(sum), scratch, total);
#pragma unroll
  for (int j = 0; j < kDocsPerThread; ++j) {
    if (base + j < n) vals[base + j] = run;
    run += local[j];
  }
  __syncthreads();
  return total;
}

// anchors.py:130-194 for one row. LDS: per-document counts, prefix of counts, document ends and
// slot prefix.
__global__ void __launch_bounds__(kSamplerThreads)
    document_sampler_kernel(const void* loss_mask, int mask_dtype, const int64_t* docs,
                            int64_t seq_len, const int64_t* lengths, int64_t num_docs,
                            int64_t num_anchors, int64_t block, int64_t total_slots,
                            int64_t padded_slots, const float* uniform, int32_t* ordered,
                            int64_t* anchors, uint8_t* keep) {
  __shared__ int64_t s_ends[kMaxSamplerDocs];    // cumsum(lengths)
  __shared__ int64_t s_start[kMaxSamplerDocs];   // exclusive prefix of valid counts
  __shared__ int64_t s_slot[kMaxSamplerDocs + 1];  // exclusive prefix of slot counts
  __shared__ int s_count[kMaxSamplerDocs];
  __shared__ int s_scratch[17];
  const int tid = threadIdx.x;

  for (int64_t d = tid; d < num_docs; d += kSamplerThreads) {
    const int64_t len = lengths[d];
    s_ends[d] = len;
    s_count[d] = 0;
    s_slot[d] = len > block ? min(num_anchors, max(len - block + 1, static_cast<int64_t>(0))) : 0;
  }
  __syncthreads();
  scan_docs(s_ends, num_docs, s_scratch);  // exclusive prefix of lengths
  for (int64_t d = tid; d < num_docs; d += kSamplerThreads) s_ends[d] += lengths[d];  // inclusive
  scan_docs(s_slot, num_docs, s_scratch);
  __syncthreads();

  // Valid candidates, compacted in ascending order, counted per document.
  const int64_t count = min(max(seq_len - block, static_cast<int64_t>(0)) + 1, seq_len - 1);
  int running = 0;
  for (int64_t base = 0; base < count; base += kSamplerThreads) {
    const int64_t i = base + tid;
    bool v = false;
    int64_t d = -1;
    if (i < count) {
      d = docs[i];
      v = mask_set(loss_mask, mask_dtype, i) && mask_set(loss_mask, mask_dtype, i + 1) && d >= 0 &&
          d < num_docs && docs[i + 1] == d;
      if (v) v = lengths[d] > block && i <= s_ends[d] - block;
    }
    int total;
    const int pos = block_exclusive_scan(v ? 1 : 0, s_scratch, total);
    if (v) {
      ordered[running + pos] = static_cast<int32_t>(i);
      atomicAdd(&s_count[d], 1);
    }
    running += total;
  }
  __syncthreads();
  for (int64_t d = tid; d < num_docs; d += kSamplerThreads) s_start[d] = s_count[d];
  __syncthreads();
  scan_docs(s_start, num_docs, s_scratch);
  if (tid == 0) s_slot[num_docs] = total_slots;
  __syncthreads();

  for (int64_t j = tid; j < padded_slots; j += kSamplerThreads) {
    int64_t a = 0;
    bool k = false;
    if (j < total_slots) {
      int64_t lo = 0, hi = num_docs;  // owner: s_slot[lo] <= j < s_slot[hi] with a nonempty range
      while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (s_slot[mid] <= j) lo = mid;
        else hi = mid;
      }
      const int64_t local = j - s_slot[lo];
      const int64_t c = s_count[lo];
      const int64_t divisor = max(c, static_cast<int64_t>(1));
      const int64_t stride = min(max(c / num_anchors, static_cast<int64_t>(1)), block + 1);
      const int64_t phase = static_cast<int64_t>(__fmul_rn(uniform[lo], static_cast<float>(divisor)));
      const int64_t rank = (phase + local * stride) % divisor;
      const int64_t idx = min(s_start[lo] + rank, count - 1);
      k = local < c;
      a = k ? ordered[idx] : 0;
    }
    anchors[j] = a;
    keep[j] = k ? 1 : 0;
  }
}

// anchors.py:197-266, one workgroup per row.
__global__ void __launch_bounds__(kSamplerThreads)
    sample_sampler_kernel(const void* loss_mask, int mask_dtype, const void* attn, int attn_dtype,
                          int64_t seq_len, int64_t num_anchors, int64_t block, int64_t max_gap,
                          const float* uniform, int32_t* workspace, int64_t* anchors,
                          uint8_t* keep) {
  __shared__ int s_scratch[17];
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t row = b * seq_len;
  int32_t* ordered = workspace + row;
  const int64_t count = min(max(seq_len - block, static_cast<int64_t>(0)) + 1, seq_len - 1);
  int running = 0;
  for (int64_t base = 0; base < count; base += kSamplerThreads) {
    const int64_t i = base + tid;
    bool v = false;
    if (i < count) {
      v = mask_set(loss_mask, mask_dtype, row + i) && mask_set(loss_mask, mask_dtype, row + i + 1);
      if (attn)
        v = v && mask_nonzero(attn, attn_dtype, row + i) &&
            mask_nonzero(attn, attn_dtype, row + block - 1 + i) &&
            mask_nonzero(attn, attn_dtype, row + block);
    }
    int total;
    const int pos = block_exclusive_scan(v ? 1 : 0, s_scratch, total);
    if (v) ordered[running + pos] = static_cast<int32_t>(i);
    running += total;
  }
  __syncthreads();
  const int64_t c = running;
  const int64_t divisor = max(c, static_cast<int64_t>(1));
  const int64_t stride = min(max(c / num_anchors, static_cast<int64_t>(1)), max_gap + 1);
  const int64_t offset = static_cast<int64_t>(__fmul_rn(uniform[b], static_cast<float>(divisor)));
  for (int64_t s = tid; s < num_anchors; s += kSamplerThreads) {
    const int64_t rank = (offset + s * stride) % divisor;
    const bool k = s < c;
    anchors[b * num_anchors + s] = k ? ordered[min(rank, count - 1)] : 0;
    keep[b * num_anchors + s] = k ? 1 : 0;
  }
}

// anchors.py:77-116, thread per anchor slot.
__global__ void __launch_bounds__(256)
    validate_anchors_kernel(const int64_t* anchors, const uint8_t* keep, const void* loss_mask,
                            int mask_dtype, const int64_t* docs, int64_t batch, int64_t seq_len,
                            int64_t num_anchors, int64_t block, int allow_partial,
                            int64_t* anchors_out, int32_t* flags) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= batch * num_anchors) return;
  const int64_t b = t / num_anchors;
  const bool k = keep[t] != 0;
  const int64_t a = k ? anchors[t] : 0;
  anchors_out[t] = a;
  if (!k) return;
  int32_t f = 8;
  const int64_t row = b * seq_len;
  if (a < 0 || a >= max(seq_len - 1, static_cast<int64_t>(0))) {
    f |= 1;
  } else {
    const int64_t first = min(a + 1, seq_len - 1);
    if (!(mask_set(loss_mask, mask_dtype, row + a) && mask_set(loss_mask, mask_dtype, row + first)))
      f |= 2;
    if (docs) {
      const int64_t last = min(a + block - allow_partial, seq_len - 1);
      const int64_t ad = docs[row + a];
      if (!(ad >= 0 && ad == docs[row + last])) f |= 4;
    }
  }
  atomicOr(flags, f);
}

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_sample_document_anchors(const void* loss_mask, int mask_dtype,
                                             const int64_t* ctx_doc_ids, int64_t seq_len,
                                             const int64_t* document_lengths, int64_t num_docs,
                                             int64_t num_anchors, int64_t block_size,
                                             int64_t total_slots, int64_t padded_slots,
                                             const float* uniform, int32_t* workspace,
                                             int64_t* anchors, uint8_t* keep, void* stream) {
  if (!valid_mask_dtype(mask_dtype)) return set_error(ASPEC_ERR_INVALID, "unknown loss_mask dtype code");
  if (num_docs <= 0 || seq_len <= 1 || num_anchors <= 0 || block_size <= 0 || total_slots <= 0 ||
      padded_slots < total_slots)
    return set_error(ASPEC_ERR_INVALID, "document anchor sampling needs positive sizes and slots");
  if (num_docs > kMaxSamplerDocs)
    return set_error(ASPEC_ERR_UNSUPPORTED, "document anchor sampling supports at most %d documents",
                     kMaxSamplerDocs);
  if (seq_len > 0x7fffffff) return set_error(ASPEC_ERR_INVALID, "row too long for anchor sampling");
  if (!loss_mask || !ctx_doc_ids || !document_lengths || !uniform || !workspace || !anchors || !keep)
    return set_error(ASPEC_ERR_INVALID, "null pointer passed to document anchor sampling");
  hipLaunchKernelGGL(document_sampler_kernel, dim3(1), dim3(kSamplerThreads), 0,
                     static_cast<hipStream_t>(stream), loss_mask, mask_dtype, ctx_doc_ids, seq_len,
                     document_lengths, num_docs, num_anchors, block_size, total_slots, padded_slots,
                     uniform, workspace, anchors, keep);
  return check_launch("document_sampler_kernel");
}

extern "C" int aspec_sample_anchors(const void* loss_mask, int mask_dtype, const void* attention_mask,
                                    int attn_dtype, int64_t batch, int64_t seq_len,
                                    int64_t num_anchors, int64_t block_size, int64_t max_gap,
                                    const float* uniform, int32_t* workspace, int64_t* anchors,
                                    uint8_t* keep, void* stream) {
  if (!valid_mask_dtype(mask_dtype) || (attention_mask && !valid_mask_dtype(attn_dtype)))
    return set_error(ASPEC_ERR_INVALID, "unknown mask dtype code");
  if (batch <= 0 || num_anchors <= 0 || block_size <= 0 || max_gap < 0 || seq_len <= block_size)
    return set_error(ASPEC_ERR_INVALID, "anchor sampling needs positive sizes and seq_len > block_size");
  if (seq_len > 0x7fffffff || batch > 0x7fffffff)
    return set_error(ASPEC_ERR_INVALID, "rows too long for anchor sampling");
  if (!loss_mask || !uniform || !workspace || !anchors || !keep)
    return set_error(ASPEC_ERR_INVALID, "null pointer passed to anchor sampling");
  hipLaunchKernelGGL(sample_sampler_kernel, dim3(static_cast<uint32_t>(batch)), dim3(kSamplerThreads),
                     0, static_cast<hipStream_t>(stream), loss_mask, mask_dtype, attention_mask,
                     attn_dtype, seq_len, num_anchors, block_size, max_gap, uniform, workspace,
                     anchors, keep);
  return check_launch("sample_sampler_kernel");
}

extern "C" int aspec_validate_injected_anchors(const int64_t* anchors, const uint8_t* keep,
                                               const void* loss_mask, int mask_dtype,
                                               const int64_t* ctx_doc_ids, int64_t batch,
                                               int64_t seq_len, int64_t num_anchors,
                                               int64_t block_size, int allow_partial_last_target,
                                               int64_t* anchors_out, int32_t* status_flags,
                                               void* stream) {
  if (!valid_mask_dtype(mask_dtype)) return set_error(ASPEC_ERR_INVALID, "unknown loss_mask dtype code");
  if (batch <= 0 || num_anchors < 0 || seq_len <= 0 || block_size <= 0)
    return set_error(ASPEC_ERR_INVALID, "injected anchor validation needs positive sizes");
  if (num_anchors == 0) return ASPEC_OK;
  if (!anchors || !keep || !loss_mask || !anchors_out || !status_flags)
    return set_error(ASPEC_ERR_INVALID, "null pointer passed to injected anchor validation");
  const int64_t n = batch * num_anchors;
  hipLaunchKernelGGL(validate_anchors_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256),
                     0, static_cast<hipStream_t>(stream), anchors, keep, loss_mask, mask_dtype,
                     ctx_doc_ids, batch, seq_len, num_anchors, block_size,
                     allow_partial_last_target ? 1 : 0, anchors_out, status_flags);
  return check_launch("validate_anchors_kernel");
}
