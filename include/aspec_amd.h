/*
 * aspec_amd C ABI: the drop-in boundary of the DSpark draft hot path on MI355X (gfx950).
 *
 * Every entry point is `extern "C"`, takes plain device pointers, sizes and element strides plus a
 * `hipStream_t` (passed as `void*`), enqueues its kernels on that stream and returns an int status:
 *
 *   ASPEC_OK (0)              success
 *   ASPEC_ERR_INVALID (1)     shape / size / layout / alignment violation  -> Python ValueError
 *   ASPEC_ERR_UNSUPPORTED (2) valid but unsupported combination           -> NotImplementedError
 *   ASPEC_ERR_RUNTIME (3)     HIP launch or runtime failure                -> RuntimeError
 *
 * `aspec_last_error()` returns the message of the last failure on the calling thread.
 * Inputs are caller-owned; outputs and workspaces are caller-allocated device buffers. The library
 * keeps no mutable global state besides the per-thread error string.
 *
 * Index conventions (one packed THD row, context-parallel degree 1):
 *   N  = anchor slots, B = draft block size, Nq = N*B query rows,
 *   T  = context tokens, K = T + Nq keys (context keys first, then draft keys in block order).
 */
#ifndef ASPEC_AMD_H_
#define ASPEC_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ASPEC_OK 0
#define ASPEC_ERR_INVALID 1
#define ASPEC_ERR_UNSUPPORTED 2
#define ASPEC_ERR_RUNTIME 3

/* ABI version; bumped on any signature change. */
int aspec_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* aspec_last_error(void);

/*
 * THD row metadata: the eight int32 mask tensors and the per-query interval endpoints.
 *
 * Replaces `_query_metadata` / `_key_metadata` (aspec/models/ops/thd_attention.py:25-56) and
 * `_build_cudnn_thd_mask` (aspec/models/ops/direct_cp.py:750-900) at CP=1.
 *
 * anchors, anchor_docs: int64 [N]; keep: uint8/bool [N];
 * context_positions, context_docs: int64 [T] (positions non-decreasing; docs ascending with any
 * negative padding ids at the tail; violations set bits 1/2 of *status_flags).
 * sequence_length <= 0 means None; context_window/query_window <= 0 mean None.
 * Outputs (int32, any may be NULL):
 *   query_aux [4][Nq] = (anchors, query_keep, query_blocks, query_docs),
 *   key_aux   [4][K]  = (key_docs, key_positions, key_blocks, key_keep),
 *   endpoints [5][Nq] = (0, context_begin, context_end, draft_begin, draft_end),
 *   status_flags [1]  = OR of violated layout invariants (must be zeroed by the caller; may be NULL).
 */
int aspec_thd_row_metadata(const int64_t* anchors, const uint8_t* keep, const int64_t* anchor_docs,
                           const int64_t* context_positions, const int64_t* context_docs,
                           int64_t num_blocks, int64_t block_size, int64_t context_length,
                           int64_t sequence_length, int64_t context_window, int64_t query_window,
                           int draft_is_causal, int32_t* query_aux, int32_t* key_aux,
                           int32_t* endpoints, int32_t* status_flags, void* stream);

/*
 * Interval endpoints [5][Nq] recovered from the eight THD mask tensors (query_aux [4][Nq],
 * key_aux [4][K], the layout of `_query_metadata` / `_key_metadata` at CP=1, context keys first).
 * This is the input `_classify_tiles` consumes (aspec/models/ops/thd_sparse_metadata.py:20-94);
 * visibility is the mask_mod of thd_attention.py:77-131. Bits 1/2/4 of *status_flags report
 * non-monotone context positions, non-monotone documents, or kept draft offsets that do not form a
 * prefix of their block (layouts the interval form cannot represent).
 */
int aspec_thd_aux_endpoints(const int32_t* query_aux, const int32_t* key_aux, int64_t num_queries,
                            int64_t num_keys, int64_t block_size, int64_t context_window,
                            int64_t query_window, int draft_is_causal, int32_t* endpoints,
                            int32_t* status_flags, void* stream);

/*
 * Block-sparse tile metadata at an arbitrary (tile_m, tile_n) geometry, from the endpoints.
 *
 * Replaces `_classify_tiles` + `_build_sparse_source` (aspec/models/ops/thd_sparse_metadata.py:20-146),
 * `_dense_to_ordered` (aspec/models/ops/fa4_sparse.py:84-91) and `_transpose_fixed_sparse`
 * (fa4_sparse.py:94-113). Class 0 = empty, 1 = partial, 2 = full; with pad_visible=1 padded
 * rows/columns count as visible for "full" exactly like the reference; with pad_visible=0 a tile
 * that reaches past Nq or K is never full (the attention kernels' own convention).
 * classes [nm][nn]; forward lists: cnt [nm], idx [nm][nn] (ascending, zero tail);
 * backward (transposed) lists: cnt [nn], idx [nn][nm]. Any output pointer may be NULL.
 */
int aspec_thd_tile_metadata(const int32_t* endpoints, int64_t num_queries, int64_t num_keys,
                            int64_t tile_m, int64_t tile_n, int pad_visible, int32_t* classes,
                            int32_t* fwd_partial_cnt, int32_t* fwd_partial_idx,
                            int32_t* fwd_full_cnt, int32_t* fwd_full_idx,
                            int32_t* bwd_partial_cnt, int32_t* bwd_partial_idx,
                            int32_t* bwd_full_cnt, int32_t* bwd_full_idx, void* stream);

/*
 * Attention plan: the tile lists the attention kernels traverse, built once per forward and shared
 * by every layer (the role of `DirectCPMetadata._fa4_cache`, aspec/models/ops/direct_cp.py:124-145).
 * `aspec_dspark_plan_bytes` gives the size of the opaque device buffer `plan`.
 */
int aspec_dspark_plan_bytes(int64_t num_queries, int64_t num_keys, size_t* bytes);
int aspec_dspark_plan_build(const int32_t* endpoints, int64_t num_queries, int64_t num_keys,
                            void* plan, void* stream);

/*
 * DSpark block-sparse attention forward (bf16 in, fp32 accumulation, bf16 out, fp32 natural-log LSE).
 *
 * Replaces the forward of `direct_cp_attention_from_kv` (aspec/models/ops/direct_cp.py:1047-1100)
 * at CP=1 via `thd_fa4_attention` (thd_attention.py:136-220) / `_cudnn_partial`
 * (direct_cp.py:903-1024), including `_apply_block_keep` (direct_cp.py:470-477): rows with no
 * visible key get O = 0 and LSE = -1e30.
 * q: [Nq] x [Hq] x [D] with element strides (q_stride_token, q_stride_head), unit stride on D;
 * k, v: [K] x [Hkv] x [D] likewise; out: [Nq] x [Hq] x [D]; lse: [Hq][Nq] contiguous.
 * Requires D == 128, Hq % Hkv == 0, Hq/Hkv <= 8, 16-byte aligned rows.
 */
int aspec_dspark_attn_fwd(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                          const void* k, int64_t k_stride_token, int64_t k_stride_head,
                          const void* v, int64_t v_stride_token, int64_t v_stride_head,
                          const int32_t* endpoints, const void* plan, int64_t num_queries,
                          int64_t num_keys, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                          float scale, void* out, int64_t o_stride_token, int64_t o_stride_head,
                          float* lse, void* stream);

/*
 * Workspace (bytes) needed by aspec_dspark_attn_bwd: per-row delta and log2-scaled LSE
 * ([Hq][Nq] fp32 each) and fp32 dK/dV accumulators ([K][Hkv][128] each) for key tiles whose
 * query list is split over several work units.
 */
int aspec_dspark_attn_bwd_workspace_bytes(int64_t num_queries, int64_t num_keys, int64_t q_heads,
                                          int64_t kv_heads, size_t* bytes);

/*
 * DSpark attention backward: dQ, dK, dV (bf16) from dO (bf16) and an optional dLSE (fp32 [Hq][Nq],
 * NULL = zero). Replaces FA4's block-sparse backward and `_InternalGQA.backward`
 * (aspec/models/ops/cudnn_gqa_backward.py:128-342): the q heads of one KV group are reduced
 * inside the kernel, so dK/dV are written once, without atomics. Same layout rules as the forward.
 */
int aspec_dspark_attn_bwd(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                          const void* k, int64_t k_stride_token, int64_t k_stride_head,
                          const void* v, int64_t v_stride_token, int64_t v_stride_head,
                          const void* out, int64_t o_stride_token, int64_t o_stride_head,
                          const void* dout, int64_t do_stride_token, int64_t do_stride_head,
                          const float* lse, const float* dlse, const int32_t* endpoints,
                          const void* plan, int64_t num_queries, int64_t num_keys, int64_t q_heads,
                          int64_t kv_heads, int64_t head_dim, float scale, void* dq,
                          int64_t dq_stride_token, int64_t dq_stride_head, void* dk,
                          int64_t dk_stride_token, int64_t dk_stride_head, void* dv,
                          int64_t dv_stride_token, int64_t dv_stride_head, void* workspace,
                          void* stream);

/*
 * The same backward, one stage at a time: `stages` is a bit mask of 1 = prepare
 * (delta = rowsum(dO*O) - dLSE and LSE*log2(e) into the workspace, zeroed split-tile
 * accumulators; the role of the reference's preprocess launch,
 * aspec/kernels/cutedsl/cudnn_gqa/preprocess.py:44-333), 2 = dQ, 4 = dK/dV (the main launch,
 * cudnn_gqa_backward.py:276-296), 8 = finalize (split-tile accumulators to bf16, the role of
 * postprocess.py:38-581). Stages run in that order; a later stage needs the workspace an earlier
 * call prepared on the same stream.
 */
int aspec_dspark_attn_bwd_stages(int stages, const void* q, int64_t q_stride_token,
                                 int64_t q_stride_head, const void* k, int64_t k_stride_token,
                                 int64_t k_stride_head, const void* v, int64_t v_stride_token,
                                 int64_t v_stride_head, const void* out, int64_t o_stride_token,
                                 int64_t o_stride_head, const void* dout, int64_t do_stride_token,
                                 int64_t do_stride_head, const float* lse, const float* dlse,
                                 const int32_t* endpoints, const void* plan, int64_t num_queries,
                                 int64_t num_keys, int64_t q_heads, int64_t kv_heads,
                                 int64_t head_dim, float scale, void* dq, int64_t dq_stride_token,
                                 int64_t dq_stride_head, void* dk, int64_t dk_stride_token,
                                 int64_t dk_stride_head, void* dv, int64_t dv_stride_token,
                                 int64_t dv_stride_head, void* workspace, void* stream);

/* Floats of per-row statistics written by aspec_ce_l1_fwd and read by aspec_ce_l1_bwd (8). */
int aspec_loss_stats_floats(void);

/*
 * Fused selective-head loss forward over bf16 logits [rows][vocab] (contiguous):
 *   l1_out[r] = sum_v |softmax(x_r)_v - softmax(y_t(r))_v|   (fp32; teacher row t(r) = r, or
 *               teacher_index[r] into a [teacher_rows][vocab] table)
 *   ce_out[r] = logsumexp(x_r) - x_r[targets[r]]            (0 where targets[r] == ignore_index)
 * Either output may be NULL (then the teacher / targets may be NULL too). stats [rows][8] fp32 is
 * required and feeds the backward. Out-of-range teacher indices / targets set bits 1 / 2 of
 * *status_flags (caller-zeroed) and produce NaN rows.
 * Replaces `tiled_l1_from_logits` forward (aspec/models/ops/tiled_l1.py:130-209) and
 * `F.cross_entropy(reduction="none")` as called at aspec/models/dspark.py:568-570.
 */
int aspec_ce_l1_fwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                    int64_t teacher_rows, const int64_t* targets, int64_t ignore_index, int64_t rows,
                    int64_t vocab, float* l1_out, float* ce_out, float* stats,
                    int32_t* status_flags, void* stream);

/*
 * Fused backward: grad_logits = grad_ce[r] * (softmax(x_r) - onehot(targets[r]))
 *                             + grad_l1[r] * p * (sign(p - q) - E_p[sign(p - q)])
 * (the L1 term in the cancellation-free form of aspec/models/ops/tiled_l1.py:107-127).
 * grad_l1 or grad_ce may be NULL (that term is skipped). Writes bf16 [rows][vocab].
 */
int aspec_ce_l1_bwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                    int64_t teacher_rows, const int64_t* targets, int64_t ignore_index, int64_t rows,
                    int64_t vocab, const float* stats, const float* grad_l1, const float* grad_ce,
                    void* grad_logits, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ASPEC_AMD_H_ */
