"""Pins the interval-union mask oracle (oracle/flex_mask.py) on the CPU: a hand-derived known answer,
the endpoints against the DFlash mask_mod brute force on the reference's own cases
(tests/test_cudnn_flex_attention.py:208-300), and the two-interval conversion against the
interval-union semantics by enumeration."""

import numpy as np
import pytest

from oracle import flex_mask as F


def test_known_answer_unpacked():
    # context 8, block 2, anchors 1 and 4: block 0 sees [0, 1) and its draft keys 8..9, block 1
    # sees [0, 4) and 10..11; three endpoints (context_end, draft_begin, draft_end) per row
    m = F.dspark_mla_mask([[1, 4]], [[True, True]], 8, 2)
    assert m.shape == (1, 3, 4)
    np.testing.assert_array_equal(m[0], [[1, 1, 4, 4], [8, 8, 10, 10], [10, 10, 12, 12]])
    # a dropped block has all-zero endpoints; a causal block ends at its own offset + 1
    m = F.dspark_mla_mask([[1, 4]], [[False, True]], 8, 2, is_causal=True)
    np.testing.assert_array_equal(m[0], [[0, 0, 4, 4], [0, 0, 10, 10], [0, 0, 11, 12]])


def _check_against_mask_mod(anchors, keep, ctx, block, **opts):
    m = F.dspark_mla_mask(anchors, keep, ctx, block, **opts)
    dense = F.dflash_mask_dense(anchors, keep, ctx, block, **opts)
    bsz, lq, nk = dense.shape
    keys = np.arange(nk)
    for b in range(bsz):
        for q in range(lq):
            np.testing.assert_array_equal(F.endpoint_visible(m, b * lq + q, keys), dense[b, q])
    return m


@pytest.mark.parametrize("block", (5, 7))
@pytest.mark.parametrize(("is_causal", "sliding_window"), ((False, None), (True, None), (False, 4), (True, 4)))
def test_endpoints_match_mask_mod(block, is_causal, sliding_window):
    """tests/test_cudnn_flex_attention.py:208-243: context 20, anchors [[3, 12], [7, 16]], one block
    dropped; three endpoints without a window, five with one."""
    m = _check_against_mask_mod([[3, 12], [7, 16]], [[True, False], [True, True]], 20, block,
                                is_causal=is_causal, sliding_window=sliding_window)
    assert m.shape[1] == (3 if sliding_window is None else 5)


@pytest.mark.parametrize("block", (5, 7))
def test_endpoints_match_packed_document_mask(block):
    """tests/test_cudnn_flex_attention.py:246-272."""
    docs = [[0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2, 2, 3, 3, 3]]
    _check_against_mask_mod([[3, 8, 16]], [[True, True, True]], 20, block, ctx_doc_ids=docs)


def test_endpoints_match_mask_mod_with_context_window_padding_and_unsorted_documents():
    # documents in contiguous runs but not ascending, a padding run (-1), and a context window on
    # top. The block anchored on padding is dropped: for a KEPT anchor on padding the reference's
    # own two forms disagree (the endpoints drop the row, cudnn_flex_attention.py:129; the mask_mod
    # keeps its draft block, dflash.py:105-125); validate_injected_anchors rejects such anchors.
    docs = [[2, 2, 2, 0, 0, 0, 0, 0, 5, 5, 5, 5, -1, -1, -1, -1],
            [1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 3, 3, 3, 3, 3, 3]]
    anchors = [[1, 6, 9, 13], [0, 4, 9, 12]]
    keep = [[True, True, True, False], [True, False, True, True]]
    for window in (None, 2, 5):
        _check_against_mask_mod(anchors, keep, 16, 3, ctx_doc_ids=docs, context_window=window)
        _check_against_mask_mod(anchors, keep, 16, 3, ctx_doc_ids=docs, context_window=window,
                                is_causal=True, sliding_window=3)


def test_invalid_geometry_matches_the_reference():
    """tests/test_cudnn_flex_attention.py:275-300."""
    keep = np.ones((1, 2), bool)
    with pytest.raises(ValueError, match="inside the context"):
        F.dspark_mla_mask([[1, 8]], keep, 8, 5)
    with pytest.raises(ValueError, match="sliding_window"):
        F.dspark_mla_mask([[1, 2]], keep, 8, 5, sliding_window=0)
    with pytest.raises(ValueError, match="contiguous run"):
        F.dspark_mla_mask([[1, 2]], keep, 8, 5, ctx_doc_ids=[[0, 0, 1, 1, 0, 0, 2, 2]])


def _union_visible(mask, rows_of, keys_of):
    """Dense [rows, all keys] visibility of an interval-union mask in the flattened key space."""
    m = np.asarray(mask)
    rows = m.shape[2]
    total = max(k1 for _, k1 in keys_of)
    out = np.zeros((rows, total), bool)
    for r in range(rows):
        k0, k1 = keys_of[rows_of(r)]
        local = np.arange(k1 - k0)
        out[r, k0:k1] = F.endpoint_visible(m, r, local)
    return out


def _two_interval_visible(ends, total):
    keys = np.arange(total)
    return (((keys[None] >= ends[1][:, None]) & (keys[None] < ends[2][:, None]))
            | ((keys[None] >= ends[3][:, None]) & (keys[None] < ends[4][:, None])))


def test_two_interval_form_equals_the_union_bshd_and_thd():
    rng = np.random.default_rng(0)
    # BSHD: batch 3, 6 query rows, 11 keys per sequence; random masks whose union is <= 2 intervals
    lq, lk, bsz = 6, 11, 3
    rows = bsz * lq
    for trial in range(200):
        e = np.zeros((1, 5, rows), np.int64)
        for r in range(rows):
            a, b_, c = sorted(rng.integers(0, lk + 1, 3))
            kind = rng.integers(0, 4)
            if kind == 0:    # [0, a) U [b, c)
                e[0, :, r] = [a, b_, c, 0, 0]
            elif kind == 1:  # [0, 0) U [a, b) U [b, c): touching, merges into one
                e[0, :, r] = [0, a, b_, b_, c]
            elif kind == 2:  # overlapping intervals in reverse order
                e[0, :, r] = [0, b_, c, a, max(b_, a)]
            else:            # empty everything, or inverted (empty) intervals
                e[0, :, r] = [0, c, a, c, b_]
        ends = F.intervals_to_endpoints(e, query_length=lq, key_length=lk)
        want = _union_visible(e, lambda r: r // lq, [(b * lk, (b + 1) * lk) for b in range(bsz)])
        np.testing.assert_array_equal(_two_interval_visible(ends, bsz * lk), want)
    # THD: three segments of 2, 5 and 3 rows with 4, 9 and 6 keys
    cq, ck = np.array([0, 2, 7, 10]), np.array([0, 4, 13, 19])
    seg = lambda r: int(np.searchsorted(cq, r, side="right")) - 1  # noqa: E731
    for trial in range(200):
        e = np.zeros((1, 3, 10), np.int64)
        for r in range(10):
            n = ck[seg(r) + 1] - ck[seg(r)]
            e[0, :, r] = sorted(rng.integers(0, n + 1, 3))
        ends = F.intervals_to_endpoints(e, cu_seqlens_q=cq, cu_seqlens_k=ck)
        want = _union_visible(e, seg, [(ck[s], ck[s + 1]) for s in range(3)])
        np.testing.assert_array_equal(_two_interval_visible(ends, 19), want)


def test_two_interval_form_rejects_what_it_cannot_hold():
    three = np.array([[[1], [2], [3], [5], [6]]])  # [0,1) U [2,3) U [5,6)
    with pytest.raises(NotImplementedError, match="two disjoint"):
        F.intervals_to_endpoints(three, query_length=1, key_length=8)
    with pytest.raises(ValueError, match="outside"):
        F.intervals_to_endpoints(np.array([[[9], [0], [0]]]), query_length=1, key_length=8)
