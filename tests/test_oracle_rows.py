"""CPU checks pinning the row-level oracle (packing, anchors, output blocks, DSpark targets)
against the reference's own test cases and closed forms, plus the host-side validation of the
product functions (which raises before any device work)."""

import numpy as np
import pytest
import torch

from oracle import rows as R


# ---------------------------------------------------------------- a1 packing (utils.py:199-356)
def _feature(n, hidden=3):
    return {"input_ids": np.arange(n, dtype=np.int64)[None], "loss_mask": np.ones((1, n), np.int64),
            "hidden_states": np.ones((1, n, hidden), np.float32),
            "last_hidden_states": np.ones((1, n, hidden), np.float32)}


def test_packing_matches_reference_known_answer():
    # tests/test_packing.py:71-81
    out = R.pack_row([_feature(3), _feature(2)], 8)
    assert out["input_ids"].shape == (1, 8)
    assert out["ctx_doc_ids"].tolist() == [[0, 0, 0, 1, 1, -1, -1, -1]]
    assert out["base_position_ids"].tolist() == [[0, 1, 2, 0, 1, 0, 0, 0]]
    assert out["attention_mask"].tolist() == [[1, 1, 1, 1, 1, 0, 0, 0]]
    assert out["input_ids"].tolist() == [[0, 1, 2, 0, 1, 0, 0, 0]]
    assert out["cu_seqlens"].tolist() == [0, 3, 5]
    assert out["hidden_states"].shape == (1, 8, 3)
    assert out["hidden_states"][0, 5:].sum() == 0 and out["hidden_states"][0, :5].min() == 1


def test_packing_overflow_and_unpadded_rows():
    with pytest.raises(ValueError, match="Packed row has"):   # tests/test_packing.py:84-86
        R.pack_row([_feature(3), _feature(2)], 4)
    out = R.pack_row([_feature(3), _feature(2)], 8, pad_to_max_length=False)
    assert out["input_ids"].shape == (1, 5)
    assert out["base_position_ids"][0, :5].tolist() == [0, 1, 2, 0, 1]


def test_context_shard_bounds_cover_each_document_once():
    for n in (0, 1, 7, 31, 64):
        for ws in (1, 2, 3, 4):
            for al in (1, 2, 4):
                b = [R.context_shard_bounds(n, r, ws, al) for r in range(ws)]
                assert b[0][0] == 0 and b[-1][1] == n
                assert all(b[i][1] == b[i + 1][0] for i in range(ws - 1))
                assert all(s % al == 0 for s, _ in b)


def test_collator_host_validation_fails_closed_without_gpu():
    from aspec_amd.collate import DFlashPackingCollator

    with pytest.raises(ValueError, match="max_seq_length > 0"):
        DFlashPackingCollator(0)
    with pytest.raises(ValueError, match="unpadded THD rows"):
        DFlashPackingCollator(8, context_parallel_size=2, context_parallel_rank=1)
    c = DFlashPackingCollator(4)
    feats = [{"input_ids": torch.zeros(1, 3, dtype=torch.long), "loss_mask": torch.ones(1, 3),
              "_aspec_work": {"execution_id": "a"}},
             {"input_ids": torch.zeros(1, 2, dtype=torch.long), "loss_mask": torch.ones(1, 2),
              "_aspec_work": {"execution_id": "b"}}]
    with pytest.raises(ValueError, match="Packed row has 5 tokens"):
        c(feats)
    with pytest.raises(ValueError, match="empty row"):
        c([])
    feats[1]["_aspec_work"] = {"execution_id": ""}
    with pytest.raises(ValueError, match="work identity"):
        DFlashPackingCollator(8)(feats)
    feats[1]["_aspec_work"] = {"execution_id": "b"}
    with pytest.raises(ValueError, match="on one GPU"):      # CPU features: no silent CPU path
        DFlashPackingCollator(8)(feats)


# ---------------------------------------------------------------- a2 anchors (anchors.py)
def test_document_anchor_slots_known_answers():
    # tests/test_sample_anchor_budget.py:83-86
    assert R.document_anchor_slots((33,) * 100, 512, 7, 4) == ((27,) * 100, 2700, 2700)
    assert R.document_anchor_slots((9, 13), 8, 7, 4) == ((3, 7), 10, 12)
    assert R.document_anchor_slots((3, 4), 512, 4) == ((0, 0), 0, 1)


def test_single_document_sampler_closed_form():
    # Fully supervised document of length L: candidates are 0 .. L-B (anchors.py:46-48), so
    # c = L-B+1, ordered = arange(c), and slot s picks (trunc(u*c) + s*stride) % c.
    L, B, A = 200, 16, 8
    for u in (0.0, 0.2345, 0.999999):
        anchors, keep = R.sample_document_anchors(np.ones(L), np.zeros(L, np.int64), (L,), A, B,
                                                   np.array([u], np.float32))
        c = L - B + 1
        stride = min(max(c // A, 1), B + 1)
        phase = int(np.float32(u) * np.float32(c))
        assert keep.all() and anchors.size == A
        assert anchors.tolist() == [(phase + s * stride) % c for s in range(A)]


def test_document_sampler_equals_native_sampler_per_document():
    # tests/test_sample_anchor_budget.py:38-61: segmented sampling == the per-sample sampler
    # applied to each document (same draws, offset by the document start).
    rng = np.random.default_rng(3)
    for lengths in ((9, 13, 30), (80,), (20, 51)):
        for A in (4, 512):
            masks = [np.ones(n) for n in lengths]
            for m in masks:
                m[2:5] = 0
            docs = np.concatenate([np.full(n, i) for i, n in enumerate(lengths)])
            u = rng.random(len(lengths)).astype(np.float32)
            actual, keep = R.sample_document_anchors(np.concatenate(masks), docs, lengths, A, 4, u)
            slots, total, padded = R.document_anchor_slots(lengths, A, 4)
            offset = cursor = 0
            for i, (m, n, s) in enumerate(zip(masks, lengths, slots)):
                expected, valid = R.sample_anchors(m[None], A, 4, u[i:i + 1])
                assert keep[cursor:cursor + s].tolist() == valid[0, :s].tolist()
                assert actual[cursor:cursor + s].tolist() == np.where(valid[0, :s], expected[0, :s] + offset, 0).tolist()
                offset += n
                cursor += s
            assert actual.size == padded == total


def test_document_sampler_budget_is_not_borrowed():
    # tests/test_sample_anchor_budget.py:64-80
    lengths = (3, 19, 4, 31)
    mask = np.ones(sum(lengths))
    mask[3:22] = 0
    docs = np.concatenate([np.full(n, i) for i, n in enumerate(lengths)])
    anchors, keep = R.sample_document_anchors(mask, docs, lengths, 8, 4, np.full(4, 0.5, np.float32), alignment=4)
    assert anchors.size % 4 == 0 and keep.sum() == 8
    assert (docs[anchors[keep]] == 3).all()
    empty_a, empty_k = R.sample_document_anchors(np.zeros_like(mask), docs, lengths, 8, 4, np.zeros(4, np.float32))
    assert not empty_k.any() and not empty_a.any()
    short = R.sample_document_anchors(np.ones(7), docs[:7], (3, 4), 512, 4, np.zeros(2, np.float32))
    assert short[0].shape == (1,) and not short[1].any()


def test_document_sampler_alignment_padding_known_answer():
    # tests/test_sample_anchor_budget.py:89-96
    docs = np.array([0] * 9 + [1] * 13)
    anchors, keep = R.sample_document_anchors(np.ones(22), docs, (9, 13), 8, 7, np.array([0.3, 0.7], np.float32),
                                              alignment=4)
    assert anchors.shape == keep.shape == (12,)
    assert keep.sum() == 10 and not keep[-2:].any() and not anchors[-2:].any()
    assert (docs[anchors[:3]] == 0).all() and (docs[anchors[3:10]] == 1).all()


def test_per_sample_sampler_gap_and_coverage():
    # anchors.py:214-229: with max_gap = 0 and enough budget, kept anchors are adjacent
    # supervised positions; each slot is kept iff s < valid count.
    mask = np.ones((2, 40))
    mask[1, 10:] = 0
    anchors, keep = R.sample_anchors(mask, 6, 4, np.array([0.0, 0.5], np.float32), max_gap=0)
    assert anchors[0].tolist() == list(range(6))
    # row 1: candidates 0..8 (c = 9), stride 1, offset trunc(0.5 * 9) = 4, wrapping modulo c
    assert keep[1].tolist() == [True] * 6
    assert anchors[1].tolist() == [4, 5, 6, 7, 8, 0]
    # short rows return the empty layout (anchors.py:253-254)
    a, k = R.sample_anchors(np.ones((1, 4)), 3, 4, np.zeros(1, np.float32))
    assert not k.any() and not a.any()


def test_validate_injected_anchors_messages_and_order():
    lm = np.ones((1, 10))
    lm[0, 5] = 0
    docs = np.array([[0] * 6 + [1] * 4])
    a, k = R.validate_injected_anchors([[1, 7]], [[True, False]], lm, 2, 4)
    assert a.tolist() == [[1, 0]]
    with pytest.raises(ValueError, match="in-bounds first prediction target"):
        R.validate_injected_anchors([[9, 0]], [[True, False]], lm, 2, 4)
    with pytest.raises(ValueError, match="must be supervised"):
        R.validate_injected_anchors([[4, 0]], [[True, False]], lm, 2, 4)
    with pytest.raises(ValueError, match="document boundaries"):
        R.validate_injected_anchors([[3, 0]], [[True, False]], lm, 2, 4, ctx_doc_ids=docs)
    # a partial last target may end exactly one token later (anchors.py:109)
    R.validate_injected_anchors([[2, 0]], [[True, False]], lm, 2, 4, ctx_doc_ids=docs,
                                allow_partial_last_target=True)


# ---------------------------------------------------------------- a11 output blocks
def test_output_block_counts_known_answer():
    # tests/test_dspark_output_compaction.py:57-60
    mask = [[True, True, False, False, False, True, False],
            [False, False, False, True, True, False, False]]
    assert R.output_block_counts(mask, 3) == [2, 2, 0]


def test_owner_indices_known_answers():
    # tests/test_dspark_output_compaction.py:109-113
    assert R.owner_block_indices(np.zeros((1, 24), bool), 4).tolist() == [[0, 6, 12, 18]]
    assert R.owner_block_indices(np.ones((1, 24), bool), 4) is None
    # tests/test_dspark_output_compaction.py:94-100
    for owners in (1, 2, 3, 4):
        m = np.zeros((2, owners * 6), bool)
        m[0, -2:] = True
        m[1, 1] = True
        idx = R.owner_block_indices(m, owners)
        assert idx.shape == (2, owners * 2)
        assert (idx // 6 == np.repeat(np.arange(owners), 2)[None]).all()


def test_block_order_is_stable_kept_first():
    rng = np.random.default_rng(0)
    keep = rng.random((3, 40)) < 0.4
    order = R.block_order(keep)
    for b in range(3):
        k = np.nonzero(keep[b])[0]
        d = np.nonzero(~keep[b])[0]
        assert order[b].tolist() == k.tolist() + d.tolist()
    # agrees with numpy's stable descending sort (what torch's stable argsort computes)
    ref = np.argsort(-keep.astype(np.int64), axis=1, kind="stable")
    assert (order == ref).all()


def test_prepare_block_layout_matches_parts():
    # tests/test_dspark_output_compaction.py:63-91
    for owners in (1, 2, 3, 4):
        for empty in (False, True):
            m = np.zeros((2, owners * 6), bool)
            if not empty:
                m[0, ::3] = True
                m[1, -2:] = True
            expected = R.owner_block_indices(m, owners)
            for rank in range(owners):
                idx, counts = R.prepare_block_layout(m, owners, rank, 4)
                assert counts == R.output_block_counts(m[:, rank * 6:(rank + 1) * 6], 4)
                assert (idx is None and expected is None) or (idx == expected).all()


# ---------------------------------------------------------------- a12 DSpark targets
def test_dspark_targets_known_answer():
    # Hand-derived from dspark.py:240-272: S=10, B=4, anchors 2 and 7, loss_mask 0 at 5.
    ids = np.arange(100, 110)[None]
    lm = np.ones((1, 10))
    lm[0, 5] = 0
    decay = R.decay_weights(4, 4.0)
    t = R.dspark_targets([[2, 7]], [[True, True]], ids, lm, 4, decay)
    assert t["label_index"].tolist() == [[[3, 4, 5, 6], [8, 9, 9, 9]]]
    assert t["eval_mask"].tolist() == [[[1, 1, 0, 0], [1, 1, 0, 0]]]
    assert t["target_ids"].tolist() == [[[103, 104, 105, 106], [108, 109, 109, 109]]]
    assert t["prev_ids"].tolist() == [[[102, 103, 104, 105], [107, 108, 109, 109]]]
    assert t["teacher_index"].tolist() == [[[2, 3, 4, 5], [7, 8, 8, 8]]]
    assert np.array_equal(t["weights"], t["eval_mask"] * decay)
    # a document boundary between 8 and 9 truncates the second block after one label
    docs = np.array([[0] * 9 + [1]])
    t = R.dspark_targets([[2, 7]], [[True, True]], ids, lm, 4, decay, ctx_doc_ids=docs)
    assert t["eval_mask"][0, 1].tolist() == [1, 0, 0, 0]
    # dropped blocks: zero labels and mask; prediction_start masks the leading slots
    t = R.dspark_targets([[2, 0]], [[True, False]], ids, lm, 4, decay, prediction_start=1)
    assert t["label_index"][0, 1].tolist() == [0, 0, 0, 0]
    assert t["eval_mask"].tolist() == [[[0, 1, 0, 0], [0, 0, 0, 0]]]


def test_decay_weights_closed_form():
    d = R.decay_weights(16, 4.0)
    assert d[0] == 1.0
    assert np.allclose(d, np.exp(-np.arange(16) / 4.0), rtol=1e-7, atol=0)
    assert (R.decay_weights(4, None) == 1).all()
    assert R.decay_weights(4, 2.0, prediction_start=2)[:3].tolist() == [1.0, 1.0, 1.0]
