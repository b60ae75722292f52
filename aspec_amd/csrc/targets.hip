// Output-block compaction (aspec/models/ops/output_blocks.py:19-98) and the DSpark labels, eval
// mask and decay weights (aspec/models/dspark.py:163-172, 240-272, 311-315, 325).
#include "rowops.h"

namespace aspec {
namespace {

constexpr int kLayoutThreads = 256;

// One workgroup per (row, owner): stable partition of the owner's `width` slots, kept first.
__global__ void __launch_bounds__(kLayoutThreads)
    block_partition_kernel(const uint8_t* keep, int64_t slots, int64_t owners, int64_t* order) {
  __shared__ int s_scratch[17];
  const int64_t b = blockIdx.x / owners;
  const int64_t o = blockIdx.x % owners;
  const int64_t width = slots / owners;
  const uint8_t* k = keep + b * slots + o * width;
  int64_t* out = order + b * slots + o * width;
  // kept count of the group
  int kept_total = 0;
  for (int64_t base = 0; base < width; base += kLayoutThreads) {
    const int64_t i = base + threadIdx.x;
    int t;
    block_exclusive_scan(i < width && k[i] ? 1 : 0, s_scratch, t);
    kept_total += t;
  }
  int kept_run = 0, drop_run = 0;
  for (int64_t base = 0; base < width; base += kLayoutThreads) {
    const int64_t i = base + threadIdx.x;
    const bool in = i < width;
    const bool kp = in && k[i];
    int kt, dt;
    const int kpos = block_exclusive_scan(kp ? 1 : 0, s_scratch, kt);
    const int dpos = block_exclusive_scan(in && !kp ? 1 : 0, s_scratch, dt);
    if (in) out[kp ? kept_run + kpos : kept_total + drop_run + dpos] = o * width + i;
    kept_run += kt;
    drop_run += dt;
  }
}

// Workgroup-wide integer sum (blockDim.x = kLayoutThreads); every thread gets the total.
__device__ __forceinline__ int block_sum(int v, int* scratch) {
  int total;
  block_exclusive_scan(v, scratch, total);
  return total;
}

// One workgroup: summary[0] = max kept count over (row, owner) groups; summary[1 + c] = max over
// rows of the kept count of chunk c of [chunk_begin, chunk_end). Groups and chunks are counted
// one at a time by the whole workgroup.
__global__ void __launch_bounds__(kLayoutThreads)
    block_summary_kernel(const uint8_t* keep, int64_t batch, int64_t slots, int64_t owners,
                         int64_t chunk_begin, int64_t chunk_end, int64_t chunk, int32_t* summary) {
  __shared__ int s_scratch[17];
  const int64_t width = slots / owners;
  int best = 0;
  for (int64_t g = 0; g < batch * owners; ++g) {
    const uint8_t* k = keep + (g / owners) * slots + (g % owners) * width;
    int n = 0;
    for (int64_t i = threadIdx.x; i < width; i += kLayoutThreads) n += k[i] != 0;
    best = max(best, block_sum(n, s_scratch));
  }
  if (threadIdx.x == 0) summary[0] = best;
  const int64_t chunks = (chunk_end - chunk_begin + chunk - 1) / chunk;
  for (int64_t c = 0; c < chunks; ++c) {
    const int64_t lo = chunk_begin + c * chunk;
    const int64_t hi = min(lo + chunk, chunk_end);
    int cbest = 0;
    for (int64_t b = 0; b < batch; ++b) {
      int n = 0;
      for (int64_t i = lo + threadIdx.x; i < hi; i += kLayoutThreads) n += keep[b * slots + i] != 0;
      cbest = max(cbest, block_sum(n, s_scratch));
    }
    if (threadIdx.x == 0) summary[1 + c] = cbest;
  }
}

// One lane per (row, block, slot), the lanes of a block adjacent inside one wave (`seg` lanes
// per block, seg = the block size rounded up to a power of two <= 64). The eval mask is the
// running product of the per-slot conditions: slot k is supervised iff no slot <= k fails,
// found from the wave's ballot of failing slots.
__global__ void __launch_bounds__(256)
    dspark_targets_kernel(const int64_t* anchors, const uint8_t* keep, const int64_t* ids,
                          const void* loss_mask, int mask_dtype, const int64_t* docs,
                          int64_t batch, int64_t seq_len, int64_t num_blocks, int64_t block,
                          int seg_log2, int64_t prediction_start, const float* decay,
                          int64_t* label_index, int64_t* target_ids, int64_t* prev_ids,
                          int64_t* teacher_index, float* eval_mask, float* weights) {
  const int seg = 1 << seg_log2;
  const int64_t lane_id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t t = lane_id >> seg_log2;          // (row, block)
  const int k = static_cast<int>(lane_id & (seg - 1));  // slot
  const bool active = t < batch * num_blocks && k < block;
  bool fail = false;
  int64_t idx = 0, a_rd = 0, row = 0;
  if (active) {
    const int64_t b = t / num_blocks;
    row = b * seq_len;
    const int64_t a = anchors[t];
    const bool kept = keep[t] != 0;
    // Anchors come validated (in [0, seq_len)); reads are clamped anyway so that no input can
    // make the kernel access memory outside the row.
    a_rd = min(max(a, static_cast<int64_t>(0)), seq_len - 1);
    const int64_t label = a + 1 + k;
    const int64_t safe = min(max(label, static_cast<int64_t>(0)), seq_len - 1);
    bool valid = label < seq_len;
    if (docs) valid = valid && docs[row + safe] == docs[row + a_rd];
    idx = kept ? safe : 0;
    fail = !(kept && valid && mask_set(loss_mask, mask_dtype, row + idx));
  }
  // first failing slot of this block (seg lanes starting at a multiple of seg inside the wave)
  const uint64_t ballot = __ballot(fail);
  const int wlane = threadIdx.x & 63;
  const int first = wlane & ~(seg - 1);
  const uint64_t mine = (seg == 64 ? ballot : (ballot >> first) & ((1ull << seg) - 1)) |
                        (block < seg ? (~0ull << block) : 0ull);
  const int first_fail = mine ? __builtin_ctzll(mine) : 64;
  if (!active) return;
  const float em = __fmul_rn(k < first_fail ? 1.f : 0.f, k >= prediction_start ? 1.f : 0.f);
  const int64_t o = t * block + k;
  const int64_t target = ids[row + idx];
  if (label_index) label_index[o] = idx;
  if (target_ids) target_ids[o] = target;
  if (prev_ids) {
    // previous token: the anchor's for slot 0, else the target of slot k - 1
    int64_t prev_idx = a_rd;
    if (k > 0) {
      const int64_t a = anchors[t];
      const int64_t pl = min(max(a + k, static_cast<int64_t>(0)), seq_len - 1);
      prev_idx = keep[t] != 0 ? pl : 0;
    }
    prev_ids[o] = ids[row + prev_idx];
  }
  if (teacher_index) teacher_index[o] = max(idx - 1, static_cast<int64_t>(0));
  if (eval_mask) eval_mask[o] = em;
  if (weights) weights[o] = __fmul_rn(em, decay[k]);
}

}  // namespace
}  // namespace aspec

using namespace aspec;

extern "C" int aspec_output_block_layout(const uint8_t* keep, int64_t batch, int64_t slots,
                                         int64_t owners, int64_t chunk_begin, int64_t chunk_end,
                                         int64_t chunk_size, int64_t* order, int32_t* summary,
                                         void* stream) {
  if (batch <= 0 || slots < 0 || owners <= 0 || slots % owners)
    return set_error(ASPEC_ERR_INVALID, "Query slots must divide evenly across CP owners");
  if (chunk_size <= 0 || chunk_begin < 0 || chunk_end < chunk_begin || chunk_end > slots)
    return set_error(ASPEC_ERR_INVALID, "invalid output-block chunk range");
  if (!keep || !summary) return set_error(ASPEC_ERR_INVALID, "null pointer passed to output-block layout");
  if (batch * owners > 0x7fffffff) return set_error(ASPEC_ERR_INVALID, "too many output-block groups");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc;
  if (order && slots > 0) {
    hipLaunchKernelGGL(block_partition_kernel, dim3(static_cast<uint32_t>(batch * owners)),
                       dim3(kLayoutThreads), 0, s, keep, slots, owners, order);
    if ((rc = check_launch("block_partition_kernel"))) return rc;
  }
  hipLaunchKernelGGL(block_summary_kernel, dim3(1), dim3(kLayoutThreads), 0, s, keep, batch, slots,
                     owners, chunk_begin, chunk_end, chunk_size, summary);
  return check_launch("block_summary_kernel");
}

extern "C" int aspec_dspark_targets(const int64_t* anchors, const uint8_t* keep,
                                    const int64_t* input_ids, const void* loss_mask, int mask_dtype,
                                    const int64_t* ctx_doc_ids, int64_t batch, int64_t seq_len,
                                    int64_t num_blocks, int64_t block_size,
                                    int64_t prediction_start, const float* decay,
                                    int64_t* label_index, int64_t* target_ids, int64_t* prev_ids,
                                    int64_t* teacher_index, float* eval_mask, float* weights,
                                    void* stream) {
  if (!valid_mask_dtype(mask_dtype)) return set_error(ASPEC_ERR_INVALID, "unknown loss_mask dtype code");
  if (batch <= 0 || seq_len <= 0 || num_blocks < 0 || block_size <= 0)
    return set_error(ASPEC_ERR_INVALID, "DSpark targets need positive sizes");
  if (num_blocks == 0) return ASPEC_OK;
  if (!anchors || !keep || !input_ids || !loss_mask || (weights && !decay))
    return set_error(ASPEC_ERR_INVALID, "null pointer passed to DSpark targets");
  if (block_size > 64)
    return set_error(ASPEC_ERR_UNSUPPORTED, "DSpark targets support block sizes up to 64");
  int seg_log2 = 0;
  while ((1 << seg_log2) < block_size) ++seg_log2;
  const int64_t lanes = (batch * num_blocks) << seg_log2;
  hipLaunchKernelGGL(dspark_targets_kernel, dim3(static_cast<uint32_t>((lanes + 255) / 256)), dim3(256),
                     0, static_cast<hipStream_t>(stream), anchors, keep, input_ids, loss_mask,
                     mask_dtype, ctx_doc_ids, batch, seq_len, num_blocks, block_size, seg_log2,
                     prediction_start, decay, label_index, target_ids, prev_ids, teacher_index,
                     eval_mask, weights);
  return check_launch("dspark_targets_kernel");
}
