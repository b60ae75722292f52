"""Row-level operations oracle (numpy). TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

Packing, anchor layout, output-block compaction and DSpark targets, restated from the reference.
The anchor samplers take their uniform draws as an argument (the reference draws them with
torch.rand from the caller's generator; the product path draws them the same way and hands them
to the HIP kernel), so they are deterministic functions here.
"""

from __future__ import annotations

import numpy as np


# --------------------------------------------------------------------------------------------
# a1: DFlashPackingCollator (aspec/data/utils.py:199-356)
# --------------------------------------------------------------------------------------------
def context_shard_bounds(sequence_length, rank, world_size, alignment=1):
    """`context_shard_bounds` (aspec/inference/context.py:30-55)."""
    if sequence_length < 0:
        raise ValueError("sequence_length must be non-negative")
    if world_size <= 0 or not 0 <= rank < world_size:
        raise ValueError("invalid context-parallel rank or world size")
    if isinstance(alignment, bool) or not isinstance(alignment, int) or alignment <= 0:
        raise ValueError("context shard alignment must be a positive integer")
    groups = sequence_length // alignment
    start = groups * rank // world_size * alignment
    end = groups * (rank + 1) // world_size * alignment
    if rank == world_size - 1:
        end = sequence_length
    return start, end


def pack_row(features, max_seq_length, pad_to_max_length=True, cp_rank=0, cp_size=1,
             cp_alignment=1):
    """The tensors of `DFlashPackingCollator.__call__` (utils.py:226-356) for numpy features.

    Each feature: dict with input_ids [1, L'], loss_mask [1, L'] and optionally hidden_states /
    last_hidden_states [1, L'', H] (L' >= L = input_ids length; the collator slices to L, or to
    the CP-owned [start, end) for the hidden fields). Returns the batch fields plus cu_seqlens.
    """
    lengths = [int(f["input_ids"].shape[1]) for f in features]
    used = sum(lengths)
    if used <= 0 or used > max_seq_length:
        raise ValueError(f"Packed row has {used} tokens; expected 1..{max_seq_length}")
    pad = max_seq_length - used if pad_to_max_length else 0

    def cat(parts, fill):
        value = np.concatenate(parts, axis=1)
        if pad:
            value = np.concatenate([value, np.full((1, pad) + value.shape[2:], fill, value.dtype)],
                                   axis=1)
        return value

    out = {
        "packed_document_lengths": tuple(lengths),
        "input_ids": cat([f["input_ids"][:, :n] for f, n in zip(features, lengths)], 0),
        "attention_mask": np.concatenate([np.ones((1, used), np.int64), np.zeros((1, pad), np.int64)], 1),
        "loss_mask": cat([f["loss_mask"][:, :n] for f, n in zip(features, lengths)], 0),
        "ctx_doc_ids": cat([np.full((1, n), d, np.int64) for d, n in enumerate(lengths)], -1),
        "base_position_ids": cat([np.arange(n, dtype=np.int64)[None] for n in lengths], 0),
        "cu_seqlens": np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32),
    }
    for name in ("hidden_states", "last_hidden_states"):
        if all(f.get(name) is not None for f in features):
            bounds = [context_shard_bounds(n, cp_rank, cp_size, cp_alignment) for n in lengths]
            out[name] = cat([f[name][:, :e - s] for f, (s, e) in zip(features, bounds)], 0)
    if cp_size > 1:
        offset, owned = 0, []
        for n in lengths:
            s, e = context_shard_bounds(n, cp_rank, cp_size, cp_alignment)
            owned.append(np.arange(offset + s, offset + e, dtype=np.int64))
            offset += n
        out["packed_context_positions"] = np.concatenate(owned)[None]
    return out


# --------------------------------------------------------------------------------------------
# a2: anchor layout (aspec/models/ops/anchors.py)
# --------------------------------------------------------------------------------------------
def _phase(u, divisor):
    """`(torch.rand(...) * divisor).long()`: float32 product, truncated (anchors.py:180, 260)."""
    return np.trunc(np.float32(u) * np.float32(divisor)).astype(np.int64)


def document_anchor_slots(document_lengths, num_anchors, block_size, alignment=1):
    """`document_anchor_slots` (anchors.py:119-127)."""
    if min(num_anchors, block_size, alignment) < 1:
        raise ValueError("Anchor budget, block size and alignment must be positive")
    slots = tuple(min(num_anchors, max(n - block_size + 1, 0)) if n > block_size else 0
                  for n in document_lengths)
    total = sum(slots)
    padded = max(alignment, ((total + alignment - 1) // alignment) * alignment)
    return slots, total, padded


def sample_document_anchors(loss_mask, ctx_doc_ids, lengths, num_anchors, block, uniform,
                            alignment=1):
    """`sample_document_anchor_positions` (anchors.py:130-194) for one row [S]; `uniform` holds
    the per-document draws of anchors.py:180. Returns (anchors [padded], keep [padded])."""
    lm = np.asarray(loss_mask, np.float64).reshape(-1) > 0.5
    docs = np.asarray(ctx_doc_ids, np.int64).reshape(-1)
    S = lm.size
    n_docs = len(lengths)
    slot_counts, total, padded = document_anchor_slots(lengths, num_anchors, block, alignment)
    if total == 0:
        return np.zeros(padded, np.int64), np.zeros(padded, bool)
    count = min(max(S - block, 0) + 1, S - 1)                                  # anchors.py:46-47
    lens = np.asarray(lengths, np.int64)
    ends = np.cumsum(lens)
    d = docs[:count]
    safe = np.clip(d, 0, n_docs - 1)
    idx = np.arange(count)
    valid = (lm[:count] & lm[1:count + 1] & (d >= 0) & (d < n_docs)            # anchors.py:48, 167-171
             & (docs[1:count + 1] == d) & (lens[safe] > block) & (idx <= ends[safe] - block))
    counts = np.bincount(safe[valid], minlength=n_docs).astype(np.int64)
    ordered = idx[valid]                                                       # sort of anchors.py:176
    starts = np.cumsum(counts) - counts
    divisor = np.maximum(counts, 1)
    stride = np.clip(counts // num_anchors, 1, block + 1)
    phase = _phase(np.asarray(uniform, np.float32), divisor)
    anchors = np.zeros(padded, np.int64)
    keep = np.zeros(padded, bool)
    j = 0
    for o, slots in enumerate(slot_counts):                                   # anchors.py:182-190
        for local in range(slots):
            rank = (phase[o] + local * stride[o]) % divisor[o]
            k = local < counts[o]
            if k:
                anchors[j] = ordered[min(starts[o] + rank, count - 1)]
            keep[j] = k
            j += 1
    return anchors, keep


def sample_anchors(loss_mask, num_anchors, block, uniform, max_gap=None, attention_mask=None):
    """`sample_anchor_positions` (anchors.py:197-266) for rows [B, S]; `uniform` [B] holds the
    draws of anchors.py:260. Returns (anchors [B, A], keep [B, A])."""
    lm = np.asarray(loss_mask, np.float64) > 0.5
    B, S = lm.shape
    if max(S - block, 0) == 0:
        return np.zeros((B, num_anchors), np.int64), np.zeros((B, num_anchors), bool)
    if max_gap is None:
        max_gap = block
    count = min(max(S - block, 0) + 1, S - 1)
    valid = lm[:, :count] & lm[:, 1:count + 1]
    if attention_mask is not None:
        am = np.asarray(attention_mask) != 0
        valid = valid & am[:, :count] & am[:, block - 1:block - 1 + count] & am[:, block:block + 1]
    anchors = np.zeros((B, num_anchors), np.int64)
    keep = np.zeros((B, num_anchors), bool)
    for b in range(B):
        ordered = np.nonzero(valid[b])[0]
        c = ordered.size
        counts = max(c, 1)
        stride = min(max(c // num_anchors, 1), max_gap + 1)
        offset = _phase(np.float32(uniform[b]), counts)
        for s in range(num_anchors):
            rank = (offset + s * stride) % counts
            keep[b, s] = s < c
            if s < c:
                anchors[b, s] = ordered[min(rank, count - 1)]
    return anchors, keep


def validate_injected_anchors(anchors, keep, loss_mask, num_anchors, block, ctx_doc_ids=None,
                              allow_partial_last_target=False):
    """`validate_injected_anchors` (anchors.py:77-116) for rows [B, A]: raises the reference's
    ValueError messages in its order; returns (anchors with dropped slots zeroed, keep)."""
    anchors = np.asarray(anchors, np.int64)
    keep = np.asarray(keep, bool)
    lm = np.asarray(loss_mask, np.float64)
    if anchors.shape != (lm.shape[0], num_anchors) or keep.shape != anchors.shape:
        raise ValueError(f"Injected anchors and keep mask must both have shape {(lm.shape[0], num_anchors)}")
    anchors = np.where(keep, anchors, 0)
    S = lm.shape[1]
    if ((anchors < 0) | (anchors >= max(S - 1, 0)))[keep].any():
        raise ValueError("Kept injected anchors must have an in-bounds first prediction target")
    if not keep.any():
        return anchors, keep
    rows = np.arange(lm.shape[0])[:, None]
    first = np.minimum(anchors + 1, S - 1)
    valid = (lm[rows, anchors] > 0.5) & (lm[rows, first] > 0.5)
    if not valid[keep].all():
        raise ValueError("Kept injected anchors and their first targets must be supervised")
    if ctx_doc_ids is not None:
        docs = np.asarray(ctx_doc_ids, np.int64)
        last = np.minimum(anchors + block - int(allow_partial_last_target), S - 1)
        ad = docs[rows, anchors]
        same = (ad >= 0) & (ad == docs[rows, last])
        if not same[keep].all():
            raise ValueError("Kept injected anchor blocks must not cross document boundaries")
    return anchors, keep


# --------------------------------------------------------------------------------------------
# a11: output-block compaction (aspec/models/ops/output_blocks.py:19-98)
# --------------------------------------------------------------------------------------------
def block_order(keep, owners=1):
    """Inside each (row, owner) group: kept slots in order, then the rest in order, as global
    slot indices -- `argsort(descending=True, stable=True)` (output_blocks.py:48, 71-74)."""
    keep = np.asarray(keep, bool)
    B, N = keep.shape
    width = N // owners
    out = np.zeros((B, N), np.int64)
    for b in range(B):
        for o in range(owners):
            g = keep[b, o * width:(o + 1) * width]
            idx = np.arange(width)
            out[b, o * width:(o + 1) * width] = np.concatenate([idx[g], idx[~g]]) + o * width
    return out


def output_block_counts(keep, chunk_size):
    """`_output_block_counts` (output_blocks.py:19-25): per-chunk kept counts, max over rows."""
    keep = np.asarray(keep, bool)
    B, N = keep.shape
    chunks = (N + chunk_size - 1) // chunk_size
    padded = np.zeros((B, chunks * chunk_size), bool)
    padded[:, :N] = keep
    return padded.reshape(B, chunks, chunk_size).sum(-1).max(0).astype(np.int64).tolist()


def output_block_indices(keep, count=None):
    """`output_block_indices` (output_blocks.py:33-48)."""
    keep = np.asarray(keep, bool)
    if count is None:
        count = int(keep.sum(1).max())
    if count == keep.shape[1]:
        return None
    if count == 0:
        return np.zeros((keep.shape[0], 0), np.int64)
    return block_order(keep)[:, :count]


def owner_block_indices(keep, owners, retained=None):
    """`owner_block_indices` (output_blocks.py:57-75)."""
    keep = np.asarray(keep, bool)
    if owners < 1 or keep.shape[1] % owners:
        raise ValueError("Query slots must divide evenly across CP owners")
    width = keep.shape[1] // owners
    grouped = keep.reshape(keep.shape[0], owners, width)
    if retained is None:
        retained = max(1, int(grouped.sum(-1).max()))
    if not 1 <= retained <= width:
        raise ValueError("Retained owner width must be within the original query slots")
    if retained == width:
        return None
    order = block_order(keep, owners).reshape(keep.shape[0], owners, width)[..., :retained]
    return order.reshape(keep.shape[0], -1)


def prepare_block_layout(keep, owners, rank, chunk_size):
    """`prepare_block_layout` (output_blocks.py:78-91)."""
    keep = np.asarray(keep, bool)
    if owners < 1 or not 0 <= rank < owners or keep.shape[1] % owners:
        raise ValueError("Query slots and rank must match contiguous CP owners")
    width = keep.shape[1] // owners
    owner_width = int(keep.reshape(keep.shape[0], owners, width).sum(-1).max())
    counts = output_block_counts(keep[:, rank * width:(rank + 1) * width], chunk_size)
    return owner_block_indices(keep, owners, retained=max(1, owner_width)), counts


# --------------------------------------------------------------------------------------------
# a12: DSpark labels / eval mask / decay weights (aspec/models/dspark.py)
# --------------------------------------------------------------------------------------------
def decay_weights(block_size, gamma, prediction_start=0):
    """`_decay_weights` (dspark.py:163-172) in float32 (exp evaluated in float64, then rounded:
    the product path takes the table torch computes)."""
    k = np.arange(block_size)
    if gamma is not None and gamma > 0:
        return np.exp(-np.maximum(k - prediction_start, 0).astype(np.float32) / np.float32(gamma)).astype(np.float32)
    return np.ones(block_size, np.float32)


def dspark_targets(anchors, keep, input_ids, loss_mask, block, decay, ctx_doc_ids=None,
                   prediction_start=0):
    """dspark.py:240-272 (labels, eval mask, decay mask), 311-315 (target / previous ids) and
    325 (teacher index) for rows [B, S] and blocks [B, nb]. `decay` is the float32 table."""
    anchors = np.asarray(anchors, np.int64)
    keep = np.asarray(keep, bool)
    ids = np.asarray(input_ids, np.int64)
    lm = np.asarray(loss_mask, np.float64)
    B, S = ids.shape
    nb = anchors.shape[1]
    offsets = np.arange(1, block + 1)
    label = anchors[..., None] + offsets                                     # dspark.py:242-243
    valid = label < S
    safe = np.minimum(label, S - 1)
    rows = np.arange(B)[:, None, None]
    if ctx_doc_ids is not None:
        docs = np.asarray(ctx_doc_ids, np.int64)
        anchor_docs = docs[np.arange(B)[:, None], anchors]
        valid = valid & (docs[rows, safe] == anchor_docs[..., None])        # dspark.py:246-251
    safe = np.where(keep[..., None], safe, 0)                                 # dspark.py:252-256
    target_lm = lm[rows, safe]
    ev = keep[..., None] & valid & (target_lm > 0.5)
    ev = np.cumprod(ev.astype(np.int32), axis=-1).astype(bool)               # dspark.py:264-266
    eval_mask = ev.astype(np.float32) * (np.arange(block) >= prediction_start).astype(np.float32)
    weights = (eval_mask * np.asarray(decay, np.float32)).astype(np.float32)  # dspark.py:271
    target_ids = ids[rows, safe]                                              # dspark.py:311-313
    anchor_ids = ids[np.arange(B)[:, None], anchors]
    prev_ids = np.concatenate([anchor_ids[..., None], target_ids[..., :-1]], axis=-1)
    teacher_index = np.maximum(safe - 1, 0)                                   # dspark.py:325
    return {"label_index": safe, "target_ids": target_ids, "prev_ids": prev_ids,
            "teacher_index": teacher_index, "eval_mask": eval_mask, "weights": weights}
