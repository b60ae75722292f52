"""Integer THD metadata oracle (numpy). TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

Everything is one packed row. The functions without a `cp_` prefix are context-parallel degree 1
(local blocks == all blocks); `shard_positions`, `cp_math_visibility` and `cp_endpoints` restate
one rank's share at cp_size > 1.
"""

from __future__ import annotations

import numpy as np

MASK_VALUE = -1.0e30  # aspec/models/ops/direct_cp.py:20


def pack_documents(lengths, max_seq_length=None, pad_to_max_length=True):
    """Row layout of `DFlashPackingCollator.__call__` (aspec/data/utils.py:226-356, CP=1).

    Returns ctx_doc_ids [T] int64 (-1 on padding, utils.py:281), base_position_ids [T]
    (doc-local arange, utils.py:282; 0 on padding), attention_mask [T] and the build's
    cu_seqlens [ndoc+1] int32 = [0, cumsum(lengths)].
    """
    lengths = [int(x) for x in lengths]
    used = sum(lengths)
    if max_seq_length is None:
        max_seq_length = used
    if used <= 0 or used > max_seq_length:
        raise ValueError(f"Packed row has {used} tokens; expected 1..{max_seq_length}")
    pad = max_seq_length - used if pad_to_max_length else 0
    docs = np.concatenate([np.full(n, i, np.int64) for i, n in enumerate(lengths)] + [np.full(pad, -1, np.int64)])
    pos = np.concatenate([np.arange(n, dtype=np.int64) for n in lengths] + [np.zeros(pad, np.int64)])
    mask = np.concatenate([np.ones(used, np.int64), np.zeros(pad, np.int64)])
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    return docs, pos, mask, cu


def token_keep(anchors, keep, block, sequence_length):
    """`_token_keep` (direct_cp.py:370-379): block keep and in-row offsets, per query row."""
    anchors = np.asarray(anchors, np.int64)
    keep = np.asarray(keep, bool)
    offsets = np.tile(np.arange(block), anchors.size)
    a = np.repeat(anchors, block)
    k = np.repeat(keep, block)
    if sequence_length is None:
        return k
    return k & (a + offsets < sequence_length)


def query_metadata(anchors, keep, anchor_docs, block, sequence_length):
    """`_query_metadata` (thd_attention.py:25-39): (docs, blocks, anchors, keep) per query row."""
    anchors = np.asarray(anchors, np.int64)
    anchor_docs = np.asarray(anchor_docs, np.int64)
    blocks = np.arange(anchors.size, dtype=np.int64)
    qkeep = token_keep(anchors, keep, block, sequence_length) & (np.repeat(anchor_docs, block) >= 0)
    return (np.repeat(anchor_docs, block), np.repeat(blocks, block), np.repeat(anchors, block), qkeep)


def key_metadata(anchors, keep, anchor_docs, context_positions, context_docs, block, sequence_length):
    """`_key_metadata` (thd_attention.py:42-56): (docs, positions, blocks, keep) per key."""
    qdocs, qblocks, _, qkeep = query_metadata(anchors, keep, anchor_docs, block, sequence_length)
    context_docs = np.asarray(context_docs, np.int64)
    n = qdocs.size
    return (
        np.concatenate([context_docs, qdocs]),
        np.concatenate([np.asarray(context_positions, np.int64), -(np.arange(n) % block) - 1]),
        np.concatenate([np.full(context_docs.size, -1, np.int64), qblocks]),
        np.concatenate([context_docs >= 0, qkeep]),
    )


def thd_aux(anchors, keep, anchor_docs, context_positions, context_docs, block, sequence_length):
    """The eight int32 mask tensors in `fixed_aux` order (thd_attention.py:149-161)."""
    qd, qb, qa, qk = query_metadata(anchors, keep, anchor_docs, block, sequence_length)
    kd, kp, kb, kk = key_metadata(anchors, keep, anchor_docs, context_positions, context_docs, block,
                                  sequence_length)
    q = np.stack([qa, qk, qb, qd]).astype(np.int32)
    k = np.stack([kd, kp, kb, kk]).astype(np.int32)
    return q, k


def thd_visibility(qaux, kaux, block, context_window=None, query_window=None, draft_is_causal=False):
    """Brute-force dense mask of the THD mask_mod (thd_attention.py:77-131): [Nq, K] bool."""
    qa, qk, qb, qd = (np.asarray(x, np.int64)[:, None] for x in qaux)
    kd, kp, kb, kk = (np.asarray(x, np.int64)[None, :] for x in kaux)
    nq = qa.shape[0]
    visible_context = (kp >= 0) & (kp < qa)
    if context_window is not None:
        visible_context &= kp >= qa - context_window
    visible_draft = (kb >= 0) & (kb == qb)
    qoff = (np.arange(nq) % block)[:, None]
    doff = -kp - 1
    if query_window is not None:
        visible_context &= qa + qoff - kp < query_window
        dist = qoff - doff
        visible_draft &= (dist < query_window) & (dist > -query_window)
    if draft_is_causal:
        visible_draft &= doff <= qoff
    return (qd == kd) & (visible_context | visible_draft) & (qk > 0) & (kk > 0)


def math_visibility(anchors, keep, context_positions, context_docs, anchor_docs, block,
                    sequence_length, context_window=None, query_window=None, draft_is_causal=False):
    """`_visibility` of the math backend (direct_cp.py:382-425) at CP=1: [Nq, K] bool."""
    anchors = np.asarray(anchors, np.int64)
    n = anchors.size
    blocks = np.arange(n)
    qblocks = np.repeat(blocks, block)
    qa = anchors[qblocks]
    qkeep = token_keep(anchors, keep, block, sequence_length)
    cpos = np.asarray(context_positions, np.int64)
    vis_ctx = cpos[None, :] < qa[:, None]
    if context_window is not None:
        vis_ctx &= cpos[None, :] >= qa[:, None] - context_window
    if context_docs is not None:
        adocs = np.asarray(anchor_docs, np.int64)[qblocks]
        cdocs = np.asarray(context_docs, np.int64)
        vis_ctx &= (adocs[:, None] >= 0) & (cdocs[None, :] == adocs[:, None])
    qoff = np.tile(np.arange(block), n)
    if query_window is not None:
        vis_ctx &= (qa + qoff)[:, None] - cpos[None, :] < query_window
    vis_draft = qblocks[None, :] == qblocks[:, None]
    if draft_is_causal:
        vis_draft &= qoff[None, :] <= qoff[:, None]
    if query_window is not None:
        vis_draft &= np.abs(qoff[:, None] - qoff[None, :]) < query_window
    key_keep = np.concatenate([np.ones(cpos.size, bool), qkeep])
    return np.concatenate([vis_ctx, vis_draft], axis=1) & qkeep[:, None] & key_keep[None, :]


def endpoints(anchors, keep, anchor_docs, context_positions, context_docs, block, sequence_length,
              context_window=None, query_window=None, draft_is_causal=False):
    """`_build_cudnn_thd_mask` (direct_cp.py:750-900) at CP=1: int32 [5, Nq]
    = (0, context_begin, context_end, draft_begin, draft_end), zeros on dropped rows."""
    anchors = np.asarray(anchors, np.int64)
    n = anchors.size
    qblocks = np.repeat(np.arange(n), block)
    offsets = np.tile(np.arange(block), n)
    qa = anchors[qblocks]
    qkeep = token_keep(anchors, keep, block, sequence_length)
    cpos = np.asarray(context_positions, np.int64)
    T = cpos.size
    lower = np.zeros_like(qa)
    if context_window is not None:
        lower = np.maximum(lower, qa - context_window)
    if query_window is not None:
        lower = np.maximum(lower, qa + offsets - query_window + 1)
    cb = np.searchsorted(cpos, lower, side="left")
    ce = np.searchsorted(cpos, qa, side="left")
    if context_docs is not None:
        cdocs = np.asarray(context_docs, np.int64)
        adocs = np.asarray(anchor_docs, np.int64)[qblocks]
        sortable = np.where(cdocs >= 0, cdocs, np.iinfo(np.int64).max)
        cb = np.maximum(cb, np.searchsorted(sortable, adocs, side="left"))
        ce = np.minimum(ce, np.searchsorted(sortable, adocs, side="right"))
        qkeep = qkeep & (adocs >= 0)
    cb = np.minimum(cb, ce)
    base = T + qblocks * block
    valid = np.full_like(qa, block)
    if sequence_length is not None:
        valid = np.clip(sequence_length - qa, 0, block)
    db = base.copy()
    de = base + valid
    if draft_is_causal:
        de = np.minimum(de, base + offsets + 1)
    if query_window is not None:
        db = base + np.clip(offsets - query_window + 1, 0, None)
        de = np.minimum(de, base + np.clip(offsets + query_window, None, block))
    db = np.minimum(db, de)
    out = np.stack([np.zeros_like(cb), cb, ce, db, de])
    out = np.where(qkeep[None, :], out, 0)
    return out.astype(np.int32)


def endpoints_to_dense(ends, num_keys):
    """Dense [Nq, K] visibility of interval endpoints."""
    ends = np.asarray(ends, np.int64)
    k = np.arange(num_keys)[None, :]
    cb, ce, db, de = (ends[i][:, None] for i in range(1, 5))
    return ((k >= cb) & (k < ce)) | ((k >= db) & (k < de))


def tile_classes_dense(visible, tile_m, tile_n, pad_visible=True):
    """Brute-force tile classes (0 empty, 1 partial, 2 full) from a dense mask, with the padding
    convention of tests/test_thd_sparse_metadata.py:187-200: padding is invisible for "any" and
    visible for "all" (pad_visible) -- or invisible for both (pad_visible=False)."""
    visible = np.asarray(visible, bool)
    nq, nk = visible.shape
    qpad, kpad = (-nq) % tile_m, (-nk) % tile_n
    anyv = np.pad(visible, ((0, qpad), (0, kpad)), constant_values=False)
    allv = np.pad(visible, ((0, qpad), (0, kpad)), constant_values=bool(pad_visible))
    nm, nn = anyv.shape[0] // tile_m, anyv.shape[1] // tile_n
    a = anyv.reshape(nm, tile_m, nn, tile_n).any(axis=(1, 3))
    f = allv.reshape(nm, tile_m, nn, tile_n).all(axis=(1, 3))
    return np.where(a, np.where(f, 2, 1), 0).astype(np.int32)


def tile_classes_from_endpoints(ends, num_queries, num_keys, tile_m, tile_n, pad_visible=True):
    """Same classes computed per row from interval overlaps (sizes where the dense mask is too big)."""
    ends = np.asarray(ends, np.int64)
    nm = -(-num_queries // tile_m)
    nn = -(-num_keys // tile_n)
    k0 = np.arange(nn) * tile_n
    k1 = np.minimum(k0 + tile_n, num_keys)
    width = k1 - k0
    classes = np.zeros((nm, nn), np.int32)
    for m in range(nm):
        r0, r1 = m * tile_m, min((m + 1) * tile_m, num_queries)
        cb, ce, db, de = (ends[i, r0:r1][:, None] for i in range(1, 5))
        c = (np.maximum(np.minimum(k1[None], ce) - np.maximum(k0[None], cb), 0)
             + np.maximum(np.minimum(k1[None], de) - np.maximum(k0[None], db), 0))
        anyv = (c > 0).any(axis=0)
        allv = (c == width[None]).all(axis=0)
        if not pad_visible:
            allv &= (k0 + tile_n <= num_keys) & (r0 + tile_m <= num_queries)
        classes[m] = np.where(anyv, np.where(allv, 2, 1), 0)
    return classes


def dense_to_ordered(blocks):
    """`_dense_to_ordered` (fa4_sparse.py:84-91): per row, count and ascending indices, zero tail."""
    blocks = np.asarray(blocks, bool)
    cols = blocks.shape[-1]
    idx = np.broadcast_to(np.arange(cols, dtype=np.int32), blocks.shape)
    packed = np.sort(np.where(blocks, idx, idx + cols), axis=-1)
    packed = np.where(packed < cols, packed, 0).astype(np.int32)
    return blocks.sum(axis=-1).astype(np.int32), packed


def ordered_to_dense(counts, indices, columns):
    """`_ordered_to_dense` (fa4_sparse.py:75-81)."""
    counts = np.asarray(counts)
    indices = np.asarray(indices)
    slots = np.arange(indices.shape[-1])
    valid = slots < counts[..., None]
    dense = np.zeros(indices.shape[:-1] + (columns + 1,), bool)
    safe = np.where(valid, indices, columns)
    np.put_along_axis(dense, safe, valid, axis=-1)
    return dense[..., :columns]


def sparse_lists(classes):
    """Forward lists and transposed backward lists of a class matrix, as `build_thd_sparse_pair`
    (thd_sparse_metadata.py:149-186) returns them for equal forward/backward tiles."""
    classes = np.asarray(classes)
    fwd = dense_to_ordered(classes == 1) + dense_to_ordered(classes == 2)
    bwd = dense_to_ordered((classes == 1).T) + dense_to_ordered((classes == 2).T)
    return fwd, bwd


def visible_pairs(ends):
    """Visible (q, k) pairs of an endpoint array (the FLOP accounting of
    tools/performance/bench_dspark_b7_attention.py:173-193)."""
    ends = np.asarray(ends, np.int64)
    return int(np.sum(ends[2] - ends[1]) + np.sum(ends[4] - ends[3]))


def shard_positions(total, rank, cp, layout="contiguous", alignment=1):
    """`build_context_positions` (direct_cp.py:23-53; the contiguous bounds are
    `context_shard_bounds`, aspec/inference/context.py:30-55): int64 positions owned by `rank`."""
    if layout == "contiguous" or cp == 1:
        groups = total // alignment
        start = groups * rank // cp * alignment
        end = total if rank == cp - 1 else groups * (rank + 1) // cp * alignment
        return np.arange(start, end, dtype=np.int64)
    chunks = 2 * cp
    parts = [np.arange(total * c // chunks, total * (c + 1) // chunks, dtype=np.int64)
             for c in (rank, chunks - 1 - rank)]
    return np.concatenate(parts)


def cp_blocks(num_blocks, rank, cp, layout="contiguous"):
    """(collective block order, this rank's local blocks): `collective_block_ids` and
    `local_block_ids` (direct_cp.py:248-262)."""
    collective = np.concatenate([shard_positions(num_blocks, r, cp, layout) for r in range(cp)])
    return collective, shard_positions(num_blocks, rank, cp, layout)


def cp_math_visibility(anchors, keep, anchor_docs, context_positions, context_docs, block,
                       sequence_length, collective_blocks, local_blocks, context_window=None,
                       query_window=None, draft_is_causal=False):
    """`_visibility` (direct_cp.py:382-425) for one rank: [len(collective)*B, T_local + len(local)*B]
    bool. Queries: the collective blocks' rows; keys: the rank's context positions (global
    positions, with their documents), then its local blocks' draft keys."""
    anchors = np.asarray(anchors, np.int64)
    collective = np.asarray(collective_blocks, np.int64)
    local = np.asarray(local_blocks, np.int64)
    qblocks = np.repeat(collective, block)
    qa = anchors[qblocks]
    qkeep = token_keep(anchors[collective], np.asarray(keep, bool)[collective], block, sequence_length)
    cpos = np.asarray(context_positions, np.int64)
    vis_ctx = cpos[None, :] < qa[:, None]
    if context_window is not None:
        vis_ctx &= cpos[None, :] >= qa[:, None] - context_window
    if context_docs is not None:
        adocs = np.asarray(anchor_docs, np.int64)[qblocks]
        cdocs = np.asarray(context_docs, np.int64)
        vis_ctx &= (adocs[:, None] >= 0) & (cdocs[None, :] == adocs[:, None])
    qoff = np.tile(np.arange(block), collective.size)
    if query_window is not None:
        vis_ctx &= (qa + qoff)[:, None] - cpos[None, :] < query_window
    dblocks = np.repeat(local, block)
    doff = np.tile(np.arange(block), local.size)
    vis_draft = dblocks[None, :] == qblocks[:, None]
    if draft_is_causal:
        vis_draft &= doff[None, :] <= qoff[:, None]
    if query_window is not None:
        vis_draft &= np.abs(qoff[:, None] - doff[None, :]) < query_window
    key_keep = np.concatenate([np.ones(cpos.size, bool),
                               token_keep(anchors[local], np.asarray(keep, bool)[local], block, sequence_length)])
    return np.concatenate([vis_ctx, vis_draft], axis=1) & qkeep[:, None] & key_keep[None, :]


def cp_endpoints(anchors, keep, anchor_docs, context_positions, context_docs, block, sequence_length,
                 collective_blocks, local_blocks, context_window=None, query_window=None,
                 draft_is_causal=False):
    """`_build_cudnn_thd_mask` (direct_cp.py:750-878) for one rank: int32 [5, len(collective)*B]
    = (0, context_begin, context_end, draft_begin, draft_end) over the rank's keys; a block the
    rank does not own has both draft endpoints at the key length; zeros on dropped rows."""
    anchors = np.asarray(anchors, np.int64)
    collective = np.asarray(collective_blocks, np.int64)
    local = np.asarray(local_blocks, np.int64)
    qblocks = np.repeat(collective, block)
    offsets = np.tile(np.arange(block), collective.size)
    qa = anchors[qblocks]
    qkeep = token_keep(anchors[collective], np.asarray(keep, bool)[collective], block, sequence_length)
    cpos = np.asarray(context_positions, np.int64)
    T = cpos.size
    key_length = T + local.size * block
    lower = np.zeros_like(qa)
    if context_window is not None:
        lower = np.maximum(lower, qa - context_window)
    if query_window is not None:
        lower = np.maximum(lower, qa + offsets - query_window + 1)
    cb = np.searchsorted(cpos, lower, side="left")
    ce = np.searchsorted(cpos, qa, side="left")
    if context_docs is not None:
        cdocs = np.asarray(context_docs, np.int64)
        adocs = np.asarray(anchor_docs, np.int64)[qblocks]
        sortable = np.where(cdocs >= 0, cdocs, np.iinfo(np.int64).max)
        cb = np.maximum(cb, np.searchsorted(sortable, adocs, side="left"))
        ce = np.minimum(ce, np.searchsorted(sortable, adocs, side="right"))
        qkeep = qkeep & (adocs >= 0)
    cb = np.minimum(cb, ce)
    slot_of = np.full(anchors.size, -1, np.int64)
    slot_of[local] = np.arange(local.size)
    slots = slot_of[qblocks]
    owns = slots >= 0
    base = T + np.maximum(slots, 0) * block
    valid = np.full_like(qa, block)
    if sequence_length is not None:
        valid = np.clip(sequence_length - qa, 0, block)
    db = base.copy()
    de = base + valid
    if draft_is_causal:
        de = np.minimum(de, base + offsets + 1)
    if query_window is not None:
        db = base + np.clip(offsets - query_window + 1, 0, None)
        de = np.minimum(de, base + np.clip(offsets + query_window, None, block))
    db = np.minimum(db, de)
    db = np.where(owns, db, key_length)
    de = np.where(owns, de, key_length)
    out = np.stack([np.zeros_like(cb), cb, ce, db, de])
    out = np.where(qkeep[None, :], out, 0)
    return out.astype(np.int32)
