"""Interval-union masks of the cuDNN FlexAttention path (numpy). TEST INFRASTRUCTURE ONLY -- see
oracle/__init__.py.

  dflash_mask_dense     `_create_dflash_mask_mod` (aspec/models/dflash.py:71-131) evaluated at every
                        (batch, query, key): [B, Lq, K] bool, the brute force the reference pins the
                        endpoints against (tests/test_cudnn_flex_attention.py:208-273)
  document_run_starts   `_document_run_starts` (aspec/models/ops/cudnn_flex_attention.py:33-50)
  dspark_mla_mask       `build_dspark_mla_mask` (cudnn_flex_attention.py:53-170): mask_func [1, E, B*Lq]
  endpoint_visible      the interval-union semantics of `_endpoint_visible`
                        (tests/test_cudnn_flex_attention.py:48-55): keys [0, e0) and [e(2i-1), e(2i))
  intervals_to_endpoints  that union as at most two intervals per row in the flattened key space of
                        all sequences (BSHD by position, THD through cu_seqlens): the attention
                        kernels' (0, cb, ce, db, de) rows
Pinned by tests/test_oracle_flex_mask.py: endpoints against the mask_mod brute force on the
reference's own cases (causal, sliding windows, dropped blocks, packed documents), the reference's
error cases, and the two-interval form against the interval-union semantics by enumeration.
"""

from __future__ import annotations

import numpy as np


def dflash_mask_dense(anchors, keep, ctx_len, block, *, is_causal=False, sliding_window=None,
                      ctx_doc_ids=None, context_window=None):
    anchors = np.asarray(anchors, np.int64)
    keep = np.asarray(keep, bool)
    bsz, n = anchors.shape
    lq = n * block
    kv = np.arange(ctx_len + lq)
    q = np.arange(lq)
    qb = q // block
    qo = q % block
    out = np.zeros((bsz, lq, kv.size), bool)
    for b in range(bsz):
        a = anchors[b, qb][:, None]
        is_ctx = kv[None, :] < ctx_len
        m_ctx = is_ctx & (kv[None, :] < a)
        if ctx_doc_ids is not None:
            docs = np.asarray(ctx_doc_ids, np.int64)[b]
            adoc = docs[anchors[b, qb]][:, None]
            cdoc = docs[np.where(kv < ctx_len, kv, 0)][None, :]
            m_ctx &= (adoc >= 0) & (cdoc == adoc)
        is_draft = kv[None, :] >= ctx_len
        kvb = (kv[None, :] - ctx_len) // block
        kvo = (kv[None, :] - ctx_len) % block
        m_draft = is_draft & (qb[:, None] == kvb)
        if is_causal:
            m_draft &= kvo <= qo[:, None]
        if context_window is not None:
            m_ctx &= kv[None, :] >= a - context_window
        if sliding_window is not None:
            qpos = a + qo[:, None]
            m_ctx &= qpos - kv[None, :] < sliding_window
            m_draft &= np.abs(qpos - (a + kvo)) < sliding_window
        out[b] = (m_ctx | m_draft) & keep[b, qb][:, None]
    return out


def document_run_starts(ctx_doc_ids):
    """First token of each token's run of equal ids; ValueError when an id has two runs."""
    docs = np.asarray(ctx_doc_ids, np.int64)
    if docs.ndim != 2:
        raise ValueError("ctx_doc_ids must have shape [batch, context_length]")
    starts = np.zeros_like(docs)
    for b in range(docs.shape[0]):
        row = docs[b]
        boundary = np.ones(row.size, bool)
        boundary[1:] = row[1:] != row[:-1]
        run_ids = row[boundary]
        if np.unique(run_ids).size != run_ids.size:
            raise ValueError("ctx_doc_ids must contain each document in one contiguous run")
        starts[b] = np.maximum.accumulate(np.where(boundary, np.arange(row.size), 0))
    return starts


def dspark_mla_mask(anchors, keep, context_length, block, *, is_causal=False, sliding_window=None,
                    context_window=None, ctx_doc_ids=None):
    anchors = np.asarray(anchors, np.int64)
    keep = np.asarray(keep, bool)
    if anchors.ndim != 2 or keep.shape != anchors.shape:
        raise ValueError("anchor_positions and block_keep_mask must have identical [batch, anchors] shapes")
    if context_length <= 0:
        raise ValueError(f"context_length must be positive, got {context_length}")
    if block <= 0:
        raise ValueError(f"block_size must be positive, got {block}")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError(f"sliding_window must be positive, got {sliding_window}")
    if ((anchors < 0) | (anchors >= context_length)).any():
        raise ValueError("anchor_positions must lie inside the context sequence")
    bsz, n = anchors.shape
    lq = n * block
    qa = np.repeat(anchors, block, axis=1)
    valid = np.repeat(keep, block, axis=1)
    qo = np.tile(np.arange(block), (bsz, n))
    qb = np.broadcast_to(np.repeat(np.arange(n), block), (bsz, lq))
    cb = np.zeros_like(qa)
    if ctx_doc_ids is not None:
        docs = np.asarray(ctx_doc_ids, np.int64)
        starts = document_run_starts(docs)
        cb = np.repeat(np.take_along_axis(starts, anchors, 1), block, axis=1)
        adoc = np.repeat(np.take_along_axis(docs, anchors, 1), block, axis=1)
        valid = valid & (adoc >= 0)
    ce = qa
    base = context_length + qb * block
    lb, le = base.copy(), base + block
    if is_causal:
        le = base + qo + 1
    if context_window is not None:
        if isinstance(context_window, bool) or not isinstance(context_window, int) or context_window <= 0:
            raise ValueError("context_window must be a positive integer or null")
        cb = np.maximum(cb, qa - context_window)
    if sliding_window is not None:
        cb = np.maximum(cb, qa + qo - sliding_window + 1)
        cb = np.minimum(cb, ce)
        lb = base + np.clip(qo - sliding_window + 1, 0, None)
        le = np.minimum(le, base + np.clip(qo + sliding_window, None, block))
    if ctx_doc_ids is None and sliding_window is None and context_window is None:
        ends = np.stack([ce, lb, le], axis=1)
    else:
        ends = np.stack([np.zeros_like(qa), cb, ce, lb, le], axis=1)
    ends = np.where(valid[:, None, :], ends, 0)
    return ends.transpose(1, 0, 2).reshape(1, ends.shape[1], bsz * lq).astype(np.int32)


def endpoint_visible(mask_func, row, key):
    e = np.asarray(mask_func)[0, :, row]
    vis = key < e[0]
    for i in range(1, e.size, 2):
        vis |= (e[i] <= key) & (key < e[i + 1])
    return vis


def intervals_to_endpoints(mask_func, *, query_length=None, key_length=None, cu_seqlens_q=None,
                           cu_seqlens_k=None):
    """[1, E, rows] interval-union rows -> int32 [5, rows] (0, cb, ce, db, de) in the flattened key
    space; ValueError for an endpoint outside its sequence's keys, NotImplementedError for a row
    with more than two disjoint intervals."""
    m = np.asarray(mask_func, np.int64)[0]
    e_count, rows = m.shape
    out = np.zeros((5, rows), np.int64)
    for r in range(rows):
        if cu_seqlens_q is None:
            b = r // query_length
            base, nkeys = b * key_length, key_length
        else:
            cq, ck = np.asarray(cu_seqlens_q), np.asarray(cu_seqlens_k)
            b = int(np.searchsorted(cq, r, side="right")) - 1
            if b < 0 or b >= cq.size - 1 or r >= cq[b + 1]:
                raise ValueError(f"query row {r} lies outside every THD segment")
            base, nkeys = int(ck[b]), int(ck[b + 1] - ck[b])
        spans = [(0, m[0, r])] + [(m[i, r], m[i + 1, r]) for i in range(1, e_count, 2)]
        for lo, hi in spans:
            if not (0 <= lo <= nkeys and 0 <= hi <= nkeys):
                raise ValueError("interval mask endpoint outside its sequence")
        merged = []
        for lo, hi in sorted((lo, hi) for lo, hi in spans if hi > lo):
            if merged and lo <= merged[-1][1]:
                merged[-1][1] = max(merged[-1][1], hi)
            else:
                merged.append([lo, hi])
        if len(merged) > 2:
            raise NotImplementedError("more than two disjoint key intervals in a query row")
        for i, (lo, hi) in enumerate(merged):
            out[1 + 2 * i, r] = base + lo
            out[2 + 2 * i, r] = base + hi
    return out.astype(np.int32)
