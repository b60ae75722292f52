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
 * aspec_thd_row_metadata for `batch` rows at once (unpacked or packed batch > 1, the rows
 * `DirectCPMetadata` carries as [batch, ...] tensors, aspec/models/ops/direct_cp.py:147-262, and
 * `_build_cudnn_thd_mask` builds for one cuDNN THD call, direct_cp.py:750-900). Inputs are
 * [batch][N] / [batch][T] contiguous. Outputs hold every batch row back to back: query_aux
 * [4][batch*Nq], key_aux [4][batch*K], endpoints [5][batch*Nq] in the flattened key space (row b's
 * keys are b*K .. b*K + K - 1, its queries b*Nq .. b*Nq + Nq - 1; dropped rows stay all zero), so one
 * attention launch serves the whole batch. batch = 1 is aspec_thd_row_metadata.
 */
int aspec_thd_batch_row_metadata(const int64_t* anchors, const uint8_t* keep,
                                 const int64_t* anchor_docs, const int64_t* context_positions,
                                 const int64_t* context_docs, int64_t batch, int64_t num_blocks,
                                 int64_t block_size, int64_t context_length,
                                 int64_t sequence_length, int64_t context_window,
                                 int64_t query_window, int draft_is_causal, int32_t* query_aux,
                                 int32_t* key_aux, int32_t* endpoints, int32_t* status_flags,
                                 void* stream);

/*
 * Interval endpoints of one context-parallel rank's partial attention: the cp_size > 1 case of
 * `_build_cudnn_thd_mask` (aspec/models/ops/direct_cp.py:750-878), whose visibility is `_visibility`
 * (direct_cp.py:382-425). The queries are every block in the collective order query_blocks
 * [num_query_blocks] (the ranks' `local_block_ids` concatenated, direct_cp.py:255-262), each expanded
 * to block_size rows; the rank's keys are its context shard (context_positions / context_docs
 * [batch][context_length], ascending positions, from `build_context_positions`) followed by the
 * draft keys of its own blocks local_blocks [num_local_blocks] (ascending), block_size each. Query
 * row q of block r sees the shard's context keys of its document before its anchor (windows as in
 * aspec_thd_row_metadata) and, when this rank owns block r as local slot j, draft keys
 * [T + j*B, T + j*B + valid); a block the rank does not own has both draft endpoints at the key
 * length T + num_local_blocks*B, as the reference writes them. Dropped rows stay all zero.
 * endpoints [5][batch * num_query_blocks * block_size] in the flattened key space (batch row b's keys
 * at b*K). Bits of *status_flags (zeroed by the caller): 1 non-monotone context positions, 2
 * non-monotone documents, 4 a block id out of range or local blocks not strictly ascending.
 * The partial's attention runs through aspec_dspark_attn_fwd / _bwd with these endpoints; the
 * ranks' (O, LSE) partials merge as in `_merge_partials` (direct_cp.py:460-467).
 */
int aspec_thd_cp_shard_endpoints(const int64_t* anchors, const uint8_t* keep,
                                 const int64_t* anchor_docs, const int64_t* context_positions,
                                 const int64_t* context_docs, int64_t batch, int64_t num_blocks,
                                 int64_t block_size, int64_t context_length,
                                 const int64_t* query_blocks, int64_t num_query_blocks,
                                 const int64_t* local_blocks, int64_t num_local_blocks,
                                 int64_t sequence_length, int64_t context_window,
                                 int64_t query_window, int draft_is_causal, int32_t* endpoints,
                                 int32_t* status_flags, void* stream);

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
 * The DSpark interval-union mask of the cuDNN FlexAttention path: `build_dspark_mla_mask`
 * (aspec/models/ops/cudnn_flex_attention.py:53-170) with `_document_run_starts` (33-50).
 * anchors int64 / keep uint8 [batch][num_anchors]; ctx_doc_ids int64 [batch][context_length] or
 * NULL; sliding_window / context_window <= 0 mean None. Writes mask_func int32 [E][batch*Nq]
 * (Nq = num_anchors * block_size) in each batch row's own key space: E = 3, (context_end,
 * draft_begin, draft_end), without documents and windows, else E = 5, (0, context_begin,
 * context_end, draft_begin, draft_end); rows of dropped blocks are all zero. *status_flags
 * (caller-zeroed) gets bit 1 for an anchor outside [0, context_length) and bit 2 for a document
 * id with more than one run in a batch row (the reference's two ValueErrors). workspace:
 * aspec_dspark_mla_mask_workspace_bytes (needed with ctx_doc_ids).
 */
int aspec_dspark_mla_mask_workspace_bytes(int64_t batch, int64_t context_length, size_t* bytes);
int aspec_dspark_mla_mask(const int64_t* anchors, const uint8_t* keep, const int64_t* ctx_doc_ids,
                          int64_t batch, int64_t num_anchors, int64_t block_size,
                          int64_t context_length, int is_causal, int64_t sliding_window,
                          int64_t context_window, int32_t* mask_func, void* workspace,
                          int32_t* status_flags, void* stream);

/*
 * An interval-union mask in the cuDNN FlexAttention format (`CudnnFlexMask.mask_func`,
 * aspec/models/ops/cudnn_flex_attention.py:173-215, consumed by `cudnn_flex_attention` 331-440)
 * turned into the attention kernels' endpoints. mask_func int32 [E][rows], E odd <= 9: row r sees
 * keys [0, e0) and [e(2i-1), e(2i)) of its own sequence. BSHD (cu_seqlens NULL): rows are
 * batch x query_length and sequence b owns keys b*key_length ..; THD: cu_seqlens_q / cu_seqlens_k
 * int32 [num_segments + 1] give each segment's rows and keys. Writes endpoints int32 [5][rows]
 * (0, cb, ce, db, de) in the flattened key space. *status_flags (caller-zeroed): bit 1 an endpoint
 * outside [0, sequence keys]; bit 2 a row whose visible keys form more than two disjoint
 * intervals (beyond the kernels' two-interval form); bit 4 a row outside every THD segment.
 */
int aspec_flex_mask_intervals(const int32_t* mask_func, int64_t num_endpoints, int64_t rows,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                              int64_t num_segments, int64_t query_length, int64_t key_length,
                              int32_t* endpoints, int32_t* status_flags, void* stream);

/*
 * Attention plan: the tile lists the attention kernels traverse, built once per forward and shared
 * by every layer (the role of `DirectCPMetadata._fa4_cache`, aspec/models/ops/direct_cp.py:124-145).
 * `aspec_dspark_plan_bytes` gives the size of the opaque device buffer `plan`.
 */
int aspec_dspark_plan_bytes(int64_t num_queries, int64_t num_keys, size_t* bytes);
int aspec_dspark_plan_build(const int32_t* endpoints, int64_t num_queries, int64_t num_keys,
                            void* plan, void* stream);

/*
 * DSpark block-sparse attention forward (bf16 or fp16 in, fp32 accumulation, out in the input type,
 * fp32 natural-log LSE).
 *
 * Replaces the forward of `direct_cp_attention_from_kv` (aspec/models/ops/direct_cp.py:1047-1100)
 * at CP=1 via `thd_fa4_attention` (thd_attention.py:136-220) / `_cudnn_partial`
 * (direct_cp.py:903-1024), including `_apply_block_keep` (direct_cp.py:470-477): rows with no
 * visible key get O = 0 and LSE = -1e30.
 * q: [Nq] x [Hq] x [D] with element strides (q_stride_token, q_stride_head), unit stride on D;
 * k, v: [K] x [Hkv] x [D] likewise; out: [Nq] x [Hq] x [D]; lse: [Hq][Nq] contiguous.
 * Requires D == 128, Hq % Hkv == 0, Hq/Hkv <= 8, 16-byte aligned rows. dtype is ASPEC_MASK_BF16
 * or ASPEC_MASK_F16 (Q, K, V, out and the P.V operand; `cudnn_flex_attention` accepts both,
 * aspec/models/ops/cudnn_flex_attention.py:353-356); anything else returns ASPEC_ERR_UNSUPPORTED.
 */
int aspec_dspark_attn_fwd(const void* q, int64_t q_stride_token, int64_t q_stride_head,
                          const void* k, int64_t k_stride_token, int64_t k_stride_head,
                          const void* v, int64_t v_stride_token, int64_t v_stride_head,
                          const int32_t* endpoints, const void* plan, int64_t num_queries,
                          int64_t num_keys, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                          float scale, void* out, int64_t o_stride_token, int64_t o_stride_head,
                          float* lse, int dtype, void* stream);

/*
 * Workspace (bytes) needed by aspec_dspark_attn_bwd: per-row delta and log2-scaled LSE
 * ([Hq][Nq] fp32 each) and fp32 dK/dV partials ([4][K][Hkv][128] each: one slot per work unit,
 * at most 4 units per key tile) for key tiles whose query list is split over several units. Only
 * the slots of split key tiles are written.
 */
int aspec_dspark_attn_bwd_workspace_bytes(int64_t num_queries, int64_t num_keys, int64_t q_heads,
                                          int64_t kv_heads, size_t* bytes);

/*
 * DSpark attention backward: dQ, dK, dV from dO (all in the dtype of the forward: ASPEC_MASK_BF16
 * or ASPEC_MASK_F16) and an optional dLSE (fp32 [Hq][Nq], NULL = zero). Replaces FA4's
 * block-sparse backward and `_InternalGQA.backward`
 * (aspec/models/ops/cudnn_gqa_backward.py:128-342): the q heads of one KV group are reduced
 * inside the kernel. Every output is deterministic (bitwise equal across runs): dQ is written once
 * per row; a key tile whose query list fits one work unit writes its dK/dV rows once; a key tile
 * split over several units (long context prefixes, at most 4 units) has each unit write its fp32
 * partial into its own slot, and the finalize sums the slots in unit order (no atomics). Same
 * layout rules as the forward.
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
                          int dtype, void* stream);

/*
 * The same backward, one stage at a time: `stages` is a bit mask of 1 = prepare
 * (delta = rowsum(dO*O) - dLSE and LSE*log2(e) into the workspace; the role of the reference's
 * preprocess launch, aspec/kernels/cutedsl/cudnn_gqa/preprocess.py:44-333), 2 = dQ, 4 = dK/dV (the
 * main launch, cudnn_gqa_backward.py:276-296), 8 = finalize (split-tile partials summed in unit
 * order to the element type, the role of postprocess.py:38-581). Stages run in that order; a later stage needs the workspace an earlier
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
                                 int64_t dv_stride_head, void* workspace, int dtype, void* stream);

/* Floats of per-row statistics written by aspec_ce_l1_fwd and read by aspec_ce_l1_bwd (8). */
int aspec_loss_stats_floats(void);

/*
 * Fused selective-head loss forward over bf16 logits [rows][vocab] (contiguous):
 *   l1_out[r] = sum_v |softmax(x_r)_v - softmax(y_t(r))_v|   (fp32; teacher row t(r) = r, or
 *               teacher_index[r] into a [teacher_rows][vocab] table)
 *   ce_out[r] = logsumexp(x_r) - x_r[targets[r]]            (0 where targets[r] == ignore_index)
 * Either output may be NULL (then the teacher / targets may be NULL too). stats [rows][8] fp32 is
 * required and feeds the backward. Out-of-range teacher indices / targets set bits 1 / 2 of
 * *status_flags (caller-zeroed) and produce NaN rows; the caller must read the flag and fail
 * closed (the Python wrappers raise ValueError, as the reference device-asserts).
 * Replaces `tiled_l1_from_logits` forward (aspec/models/ops/tiled_l1.py:130-209) and
 * `F.cross_entropy(reduction="none")` as called at aspec/models/dspark.py:568-570.
 */
int aspec_ce_l1_fwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                    int64_t teacher_rows, const int64_t* targets, int64_t ignore_index, int64_t rows,
                    int64_t vocab, float* l1_out, float* ce_out, float* stats,
                    int32_t* status_flags, void* stream);

/*
 * aspec_ce_l1_fwd plus the row argmax in the same pass over the logits: argmax_out[r] (int64, may
 * be NULL) is the index torch.argmax returns -- the first NaN if the row has one, else the first
 * index of the row maximum. Vocabularies of 2^31 or more are rejected when argmax_out is set.
 * Replaces, in the same pass, `logits.argmax(-1)` of the DSpark head's accuracy metric
 * (aspec/models/dspark.py:628-629).
 */
int aspec_ce_l1_argmax_fwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                           int64_t teacher_rows, const int64_t* targets, int64_t ignore_index,
                           int64_t rows, int64_t vocab, float* l1_out, float* ce_out,
                           int64_t* argmax_out, float* stats, int32_t* status_flags, void* stream);

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

/*
 * aspec_ce_l1_argmax_fwd and aspec_ce_l1_bwd in one pass, for an objective whose per-row weights
 * are known before the forward: sum_r (grad_ce[r] * ce[r] + grad_l1[r] * l1[r]) (the DSpark loss
 * numerator ce_alpha * ce_num + l1_alpha * l1_num, aspec/models/dspark.py:485-491, with the
 * eval-mask x decay weights folded into grad_ce / grad_l1). Writes l1_out, ce_out, argmax_out (may
 * be NULL), stats, and grad_logits = the aspec_ce_l1_bwd result for these gradients, each row once
 * its statistics are final. grad_logits may be the logits buffer itself (in place). Needs a teacher,
 * vocab % 8 == 0, vocab <= 32768 and 16-byte aligned rows (status 2 otherwise). Removes the
 * backward's second read of the logits and teacher rows: the selective head's vocab GEMM + CE/L1
 * (aspec/models/dspark.py:553-612, aspec/models/ops/tiled_l1.py:31-127) then moves its logits
 * through HBM once.
 */
int aspec_ce_l1_fused_fwd_bwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                              int64_t teacher_rows, const int64_t* targets, int64_t ignore_index,
                              int64_t rows, int64_t vocab, const float* grad_ce, const float* grad_l1,
                              float* l1_out, float* ce_out, int64_t* argmax_out, float* stats,
                              void* grad_logits, int32_t* status_flags, void* stream);

/*
 * x *= *scalar in place over n bf16 values (fp32 product, one round to nearest even), the scalar
 * read on the device. The upstream gradient of the fused objective scales the dgrad GEMM's dh
 * with it (the gradient a loss's backward receives, aspec/models/dspark.py:485-491). A scalar of
 * exactly 1 leaves x untouched (every product would equal its input), without a host read.
 */
int aspec_scale_bf16_by_device_scalar(void* x, int64_t n, const float* scalar, void* stream);

/*
 * Sampled L1 (aspec/models/ops/loss.py:57-89; DSparkModel._prediction_terms with l1 sampling,
 * aspec/models/dspark.py:606-609). Per row and side the logits are filtered as
 * sampling_logits(x, (temperature, top_p, top_k)): scaled = (x - max x) * (1/T) when T != 1
 * (else x), ordered descending with ties by token index; a token is kept iff its rank < top_k
 * (0 < top_k < V) and the softmax(scaled) mass of the tokens before it <= top_p (top_p < 1).
 * Parameters: temperature finite > 0, top_p in (0, 1], top_k -1 or >= 1 (status 1 otherwise).
 * bf16 logits, any V up to 2^24, rows < 2^31. No sort: a binary search over the 16-bit bf16
 * keys per row (the row in registers up to 98304 tokens).
 *
 * aspec_sampling_logits_fwd writes the filtered fp32 logits ([rows][vocab], -inf outside the
 * support) and aspec_sampling_stats_floats() floats of stats per row; aspec_sampling_logits_bwd
 * maps an fp32 gradient of them to the bf16 logits (keep * g / T, with the max subtraction's
 * gradient shared by the tokens equal to the max).
 */
int aspec_sampling_stats_floats(void);
int aspec_sampling_logits_fwd(const void* logits, int64_t rows, int64_t vocab, double temperature,
                              double top_p, int64_t top_k, float* out, float* stats, void* stream);
int aspec_sampling_logits_bwd(const void* logits, const float* grad_out, const float* stats,
                              int64_t rows, int64_t vocab, void* grad_logits, void* stream);

/*
 * l1_out[r] = sum |softmax_kept(draft) - softmax_kept(teacher)| with draft_* and target_* the two
 * sides' filters (compiled_l1_from_logits(logits, target, target_sampling, draft_sampling),
 * aspec/models/ops/loss.py:83-89); the teacher row is teacher_index[r] when given (an
 * out-of-range index sets bit 0 of status_flags and gives a NaN row). Stats:
 * aspec_sampled_l1_stats_floats() floats per row. The backward writes the bf16 draft gradient
 * grad_l1[r] / T * p * (sign(p - q) - sum p sign(p - q)); the teacher is frozen.
 */
int aspec_sampled_l1_stats_floats(void);
int aspec_sampled_l1_fwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                         int64_t teacher_rows, int64_t rows, int64_t vocab, double draft_temperature,
                         double draft_top_p, int64_t draft_top_k, double target_temperature,
                         double target_top_p, int64_t target_top_k, float* l1_out, float* stats,
                         int32_t* status_flags, void* stream);
int aspec_sampled_l1_bwd(const void* logits, const void* teacher, const int64_t* teacher_index,
                         int64_t teacher_rows, int64_t rows, int64_t vocab, const float* stats,
                         const float* grad_l1, void* grad_logits, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Row-level operations around the attention and loss: packing, anchors, output blocks, targets.
 * ------------------------------------------------------------------------------------------- */

/* dtype codes of loss / attention mask inputs. */
#define ASPEC_MASK_F32 0
#define ASPEC_MASK_I64 1
#define ASPEC_MASK_I32 2
#define ASPEC_MASK_U8 3 /* bool */
#define ASPEC_MASK_BF16 4
#define ASPEC_MASK_F16 5

/* One copy of a packed-row build: `bytes` bytes from `src` to `dst`; src == NULL zero-fills. */
typedef struct AspecCopySpan {
  const void* src;
  void* dst;
  int64_t bytes;
} AspecCopySpan;

/*
 * Executes `count` copy spans (a device array; destinations must not overlap) in one launch, one
 * workgroup per span, 16-byte vectors where src, dst and size allow.
 * Replaces the concatenation and padding copies of DFlashPackingCollator.__call__
 * (aspec/data/utils.py:226-323): input_ids, loss_mask, hidden_states, last_hidden_states.
 */
int aspec_pack_copy(const AspecCopySpan* spans, int64_t count, void* stream);

/*
 * Per-token metadata of one packed row from cu_seqlens (int32 [num_docs + 1], device,
 * cu_seqlens[0] = 0, non-decreasing, cu_seqlens[num_docs] = used tokens <= row_length):
 *   ctx_doc_ids[t] = d where cu_seqlens[d] <= t < cu_seqlens[d+1], -1 on padding;
 *   base_position_ids[t] = t - cu_seqlens[d], 0 on padding;
 *   attention_mask[t] = t < used.
 * All int64 [row_length]; any may be NULL.
 * Replaces aspec/data/utils.py:263-285 (doc_ids, positions, attention_mask).
 */
int aspec_pack_row_metadata(const int32_t* cu_seqlens, int64_t num_docs, int64_t row_length,
                            int64_t* ctx_doc_ids, int64_t* base_position_ids,
                            int64_t* attention_mask, void* stream);

/*
 * Document anchor sampler for one packed row: sample_document_anchor_positions with
 * _candidates and document_anchor_slots (aspec/models/ops/anchors.py:31-53,119-194).
 *   loss_mask [seq_len] (ASPEC_MASK_* dtype), ctx_doc_ids int64 [seq_len],
 *   document_lengths int64 [num_docs] (device), uniform float32 [num_docs]: the torch.rand draws
 *   of anchors.py:180 (the phase is trunc(uniform * max(count, 1)) in float32);
 *   total_slots / padded_slots as document_anchor_slots computes them (host), total_slots > 0;
 *   workspace int32 [seq_len].
 * Outputs anchors int64 [padded_slots], keep uint8 [padded_slots]. num_docs <= 4096.
 */
int aspec_sample_document_anchors(const void* loss_mask, int mask_dtype, const int64_t* ctx_doc_ids,
                                  int64_t seq_len, const int64_t* document_lengths,
                                  int64_t num_docs, int64_t num_anchors, int64_t block_size,
                                  int64_t total_slots, int64_t padded_slots, const float* uniform,
                                  int32_t* workspace, int64_t* anchors, uint8_t* keep,
                                  void* stream);

/*
 * Per-sample anchor sampler: sample_anchor_positions (aspec/models/ops/anchors.py:197-266) for
 * `batch` rows of seq_len > block_size tokens. loss_mask [batch][seq_len]; attention_mask may be
 * NULL (else [batch][seq_len], ASPEC_MASK_* dtype attn_dtype); max_gap >= 0; uniform float32
 * [batch] (the draws of anchors.py:260); workspace int32 [batch][seq_len].
 * Outputs anchors int64 [batch][num_anchors], keep uint8 [batch][num_anchors].
 */
int aspec_sample_anchors(const void* loss_mask, int mask_dtype, const void* attention_mask,
                         int attn_dtype, int64_t batch, int64_t seq_len, int64_t num_anchors,
                         int64_t block_size, int64_t max_gap, const float* uniform,
                         int32_t* workspace, int64_t* anchors, uint8_t* keep, void* stream);

/*
 * Injected-anchor validation: validate_injected_anchors (aspec/models/ops/anchors.py:77-116).
 * anchors int64 / keep uint8 [batch][num_anchors]; loss_mask [batch][seq_len]; ctx_doc_ids int64
 * [batch][seq_len] or NULL. Writes anchors_out = keep ? anchors : 0 and ORs into *status_flags
 * (caller-zeroed): 1 a kept anchor without an in-bounds first target, 2 a kept anchor or its first
 * target unsupervised, 4 a kept block crossing a document boundary, 8 some anchor kept.
 */
int aspec_validate_injected_anchors(const int64_t* anchors, const uint8_t* keep,
                                    const void* loss_mask, int mask_dtype,
                                    const int64_t* ctx_doc_ids, int64_t batch, int64_t seq_len,
                                    int64_t num_anchors, int64_t block_size,
                                    int allow_partial_last_target, int64_t* anchors_out,
                                    int32_t* status_flags, void* stream);

/*
 * Output-block layout over keep uint8 [batch][slots], slots = owners * width:
 *   order int64 [batch][slots] (may be NULL): inside each (row, owner) the slots with keep set in
 *     original order, then the others in original order, as global slot indices (the stable
 *     descending argsort of output_blocks.py:48 / 71, offset by owner * width);
 *   summary int32 [1 + num_chunks]: summary[0] = max over rows and owners of the kept count;
 *     summary[1 + c] = max over rows of the kept count in slots
 *     [chunk_begin + c * chunk_size, min(chunk_begin + (c + 1) * chunk_size, chunk_end)),
 *     num_chunks = ceil((chunk_end - chunk_begin) / chunk_size).
 * Replaces output_block_counts / output_block_indices / owner_block_indices /
 * prepare_block_layout (aspec/models/ops/output_blocks.py:19-98).
 */
int aspec_output_block_layout(const uint8_t* keep, int64_t batch, int64_t slots, int64_t owners,
                              int64_t chunk_begin, int64_t chunk_end, int64_t chunk_size,
                              int64_t* order, int32_t* summary, void* stream);

/*
 * DSpark labels, eval mask and decay weights (aspec/models/dspark.py:240-272, 311-315, 325):
 * for block j of row b with anchor a and slot k < block_size,
 *   label = a + 1 + k, valid = label < seq_len (and same document as the anchor if ctx_doc_ids),
 *   label_index = keep ? min(label, seq_len - 1) : 0,
 *   eval_mask = cumprod_k(keep & valid & loss_mask[label_index] > 0.5) * (k >= prediction_start),
 *   weights = eval_mask * decay[k]   (decay float32 [block_size], as _decay_weights computes it),
 *   target_ids = input_ids[label_index], prev_ids = (input_ids[a], target_ids[k-1]),
 *   teacher_index = max(label_index - 1, 0).
 * anchors int64 (in [0, seq_len)) / keep uint8 [batch][num_blocks]; input_ids int64, loss_mask,
 * ctx_doc_ids (int64, may be NULL) [batch][seq_len]. Outputs [batch][num_blocks][block_size]; any
 * may be NULL.
 */
int aspec_dspark_targets(const int64_t* anchors, const uint8_t* keep, const int64_t* input_ids,
                         const void* loss_mask, int mask_dtype, const int64_t* ctx_doc_ids,
                         int64_t batch, int64_t seq_len, int64_t num_blocks, int64_t block_size,
                         int64_t prediction_start, const float* decay, int64_t* label_index,
                         int64_t* target_ids, int64_t* prev_ids, int64_t* teacher_index,
                         float* eval_mask, float* weights, void* stream);

/*
 * DSpark Q/K preparation, forward: per-head RMSNorm of query and keys, the context/draft key join
 * and indexed RoPE. Replaces `dspark_qk_norm_rope` / `_DSparkQkNormRope.forward`
 * (aspec/models/ops/dspark_qk_norm_rope.py:134-280, run_dspark_qk_norm_rope); the math is
 * `_prepare_dflash_qk` (aspec/models/draft/dflash.py:280-327) in fp32 with one rounding to the
 * activation dtype.
 *
 * dtype ASPEC_MASK_BF16 or ASPEC_MASK_F16 (activations, weights and cos/sin alike; the
 * reference serves both, dspark_qk_norm_rope.py:169-170), head_dim 128: query [batch*draft_len][q_heads][128], context_key [batch*context_len]
 * [kv_heads][128], draft_key [batch*draft_len][kv_heads][128]; q_weight, k_weight [128];
 * cos, sin [rope_rows][rope_stride] (first 128 columns used); positions int64, one per token.
 * Outputs: q_out like query; k_out [batch][context_len + draft_len][kv_heads][128] (context first);
 * rstd_q [batch*draft_len][q_heads], rstd_k [batch*(context_len+draft_len)][kv_heads] fp32.
 * A position outside [0, rope_rows) gives a NaN output row and sets bit 0 of *status_flags.
 */
int aspec_qk_norm_rope_fwd(const void* query, const void* context_key, const void* draft_key,
                           const void* q_weight, const void* k_weight, const void* cos,
                           const void* sin, int64_t rope_rows, int64_t rope_stride,
                           const int64_t* query_positions, const int64_t* context_positions,
                           const int64_t* draft_positions, int64_t batch, int64_t context_len,
                           int64_t draft_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                           float eps, int32_t dtype, void* q_out, void* k_out, float* rstd_q,
                           float* rstd_k, int32_t* status_flags, void* stream);

/* Bytes of the backward's workspace (per-workgroup weight-gradient partials). */
int aspec_qk_norm_rope_bwd_workspace_bytes(int64_t batch, int64_t context_len, int64_t draft_len,
                                           int64_t q_heads, int64_t kv_heads, size_t* bytes);

/*
 * DSpark Q/K preparation, backward (`_DSparkQkNormRope.backward`,
 * aspec/models/ops/dspark_qk_norm_rope.py:282-398, run_dspark_qk_norm_rope_bwd): grad_q / grad_k
 * in the forward's output layouts -> d_query, d_context_key, d_draft_key (bf16, input layouts) and
 * dw_q, dw_k (fp32 [128], deterministic). rstd_q / rstd_k are the forward's.
 */
int aspec_qk_norm_rope_bwd(const void* grad_q, const void* grad_k, const void* query,
                           const void* context_key, const void* draft_key, const float* rstd_q,
                           const float* rstd_k, const void* q_weight, const void* k_weight,
                           const void* cos, const void* sin, int64_t rope_rows,
                           int64_t rope_stride, const int64_t* query_positions,
                           const int64_t* context_positions, const int64_t* draft_positions,
                           int64_t batch, int64_t context_len, int64_t draft_len, int64_t q_heads,
                           int64_t kv_heads, int64_t head_dim, float eps, int32_t dtype,
                           void* d_query, void* d_context_key, void* d_draft_key, float* dw_q,
                           float* dw_k,
                           void* workspace, int32_t* status_flags, void* stream);

/*
 * aspec_qk_norm_rope_bwd without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The weight-gradient partials live in a static 2 MiB device array
 * that the library holds on each GPU it runs on until the process ends (every size fits: the
 * kernel's grid is capped); its address is looked up on the first call on each device, with that
 * device current. The entry point allocates nothing and calls no allocating routine. Calls that
 * overlap on one GPU share the array and race: serialize them (one stream, or events).
 */
int aspec_qk_norm_rope_bwd_noalloc(const void* grad_q, const void* grad_k, const void* query,
                                   const void* context_key, const void* draft_key,
                                   const float* rstd_q, const float* rstd_k, const void* q_weight,
                                   const void* k_weight, const void* cos, const void* sin,
                                   int64_t rope_rows, int64_t rope_stride,
                                   const int64_t* query_positions,
                                   const int64_t* context_positions,
                                   const int64_t* draft_positions, int64_t batch,
                                   int64_t context_len, int64_t draft_len, int64_t q_heads,
                                   int64_t kv_heads, int64_t head_dim, float eps, int32_t dtype,
                                   void* d_query, void* d_context_key, void* d_draft_key,
                                   float* dw_q, float* dw_k, int32_t* status_flags, void* stream);

/*
 * RMSNorm forward over rows of `hidden` bf16 values (multiple of 8, at most 8192), with an
 * optional residual add: y = x + residual (bf16, written to y_out), rstd[r] = 1/sqrt(mean(y^2) +
 * eps), out = bf16(y * rstd * weight). Replaces `DFlashRMSNorm.forward` / `_dflash_rms_norm`
 * (aspec/models/draft/dflash.py:175-188, 282-293) and, with a residual, the residual add before
 * `post_attention_layernorm` (dflash.py:1046-1050). residual and y_out may be NULL together.
 */
int aspec_rmsnorm_fwd(const void* x, const void* residual, const void* weight, int64_t rows,
                      int64_t hidden, float eps, void* y_out, void* out, float* rstd, void* stream);

/* Bytes of the RMSNorm backward's workspace (per-workgroup weight-gradient partials). */
int aspec_rmsnorm_bwd_workspace_bytes(int64_t hidden, size_t* bytes);

/*
 * RMSNorm backward: with g = grad_out * weight and n = y * rstd,
 * dy = rstd * (g - n * mean(g * n)) + dy_extra (bf16; dy_extra may be NULL) and
 * dweight = sum over rows of grad_out * n (fp32 [hidden], deterministic). y and rstd are the
 * forward's normalized input and rstd. Backward of `aspec_rmsnorm_fwd` (autograd of
 * dflash.py:282-293).
 */
int aspec_rmsnorm_bwd(const void* grad_out, const void* dy_extra, const void* y, const void* weight,
                      const float* rstd, int64_t rows, int64_t hidden, void* dy, float* dweight,
                      void* workspace, void* stream);

/*
 * SwiGLU over one GEMM output gate_up = [gate | up] (rows x 2*ffn bf16, ffn a multiple of 8):
 * out = bf16(silu(gate) * up). Replaces `act_fn(gate_proj(x)) * up_proj(x)` of `DFlashMLP`
 * (aspec/models/draft/dflash.py:967-980).
 */
int aspec_swiglu_fwd(const void* gate_up, int64_t rows, int64_t ffn, void* out, void* stream);

/* SwiGLU backward: d_gate_up = [dout * up * silu'(gate) | dout * silu(gate)] (bf16). */
int aspec_swiglu_bwd(const void* grad_out, const void* gate_up, int64_t rows, int64_t ffn,
                     void* d_gate_up, void* stream);

/* Bytes of the device-side AdamW state (step count, clip coefficient, skip flag, ...); the caller
 * zero-initializes it once. */
int aspec_adamw_state_bytes(void);

/* Bytes of the AdamW step's workspace (gradient-norm partials). */
int aspec_adamw_workspace_bytes(size_t* bytes);

/*
 * One optimizer step of `BF16Optimizer` (aspec/training/optimizer.py:40-164: fp32 master weights,
 * global-norm clipping to max_grad_norm, a non-finite norm skips the step, torch's fused AdamW,
 * bf16 copy-back) over n flat parameters: params bf16, master / exp_avg / exp_avg_sq fp32, grads
 * bf16 (all 16-byte aligned). The step count, clip coefficient and gradient norm stay in `state` on
 * the device (no host synchronization).
 */
int aspec_adamw_step(void* params, float* master, float* exp_avg, float* exp_avg_sq,
                     const void* grads, int64_t n, float lr, float weight_decay, float beta1,
                     float beta2, float eps, float max_grad_norm, void* state, void* workspace,
                     void* stream);

/*
 * The same step with the gradients where autograd leaves them (one tensor per parameter) instead
 * of one flat buffer: segment i covers the next seg_numel[i] flat parameters and seg_grads[i] is
 * its bf16 gradient (device pointer, 16-byte aligned), or NULL for a parameter without a gradient,
 * which is then left unchanged and adds nothing to the norm (as `optimizer.step()` skips a
 * parameter whose grad is None, optimizer.py:99-109). Each segment keeps its own step count in
 * `state` (torch's AdamW counts steps per parameter), so its bias corrections count only the steps
 * in which it had a gradient. Both arrays are host memory; 1 <= nseg <= 64, and every segment but
 * the last holds a multiple of 8 elements. When every segment has a gradient, the results are
 * bitwise equal to aspec_adamw_step over the same gradients gathered into one buffer.
 */
int aspec_adamw_step_segments(void* params, float* master, float* exp_avg, float* exp_avg_sq,
                              const void* const* seg_grads, const int64_t* seg_numel, int nseg,
                              float lr, float weight_decay, float beta1, float beta2, float eps,
                              float max_grad_norm, void* state, void* workspace, void* stream);

/* ---- Row packing policy (host only: plain host arrays, no GPU, no stream) ---- */

/*
 * Useful anchor starts per pooled sample: count_eligible_anchor_starts
 * (aspec/controller/packing.py:43-67), batched. Sample s has run lengths
 * runs[run_offsets[s] .. run_offsets[s+1]) of its packed loss mask (alternating unsupervised /
 * supervised, unsupervised first) and length sample_lengths[s]; counts_out[s] is the number of
 * supervised positions p with p <= length - block_size (0 when length or block_size is not
 * positive). A negative run length is an error.
 */
int aspec_count_eligible_anchor_starts(const int64_t* runs, const int64_t* run_offsets,
                                       const int64_t* sample_lengths, int64_t num_samples,
                                       int64_t block_size, int64_t* counts_out);

/*
 * Work-aware row packing: pack_work_aware_rows (aspec/controller/packing.py:87-167). Samples
 * 0..dp_size-1 seed one row each; the rest, by useful_work/length (double quotient), useful_work and
 * length (descending) and index, go to the fitting row with the least slack (ties: lower row) until
 * max_selected samples are taken (max_selected < 0: no limit; otherwise >= dp_size). Rows come out
 * ordered by tokens, descending (ties: lower row): row k holds
 * row_samples[row_offsets[k] .. row_offsets[k+1]) in placement order, row_tokens_out[k] tokens.
 * row_offsets [dp_size + 1], row_samples [count], row_tokens_out [dp_size].
 * count < dp_size packs nothing (row_offsets all 0: the reference returns None). Errors: lengths
 * outside [1, max_seq_length] (message names the first), non-positive dp_size / max_seq_length,
 * max_selected below dp_size, lengths or useful_work beyond 2^53.
 */
int aspec_pack_work_aware_rows(const int64_t* lengths, const int64_t* useful_work, int64_t count,
                               int64_t dp_size, int64_t max_seq_length, int64_t max_selected,
                               int64_t* row_offsets, int64_t* row_samples, int64_t* row_tokens_out);

#ifdef __cplusplus
}
#endif

#endif /* ASPEC_AMD_H_ */
