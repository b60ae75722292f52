"""Pins the integer-metadata oracle (CPU): hand-derived golden fixtures from the reference's own
test cases, agreement of three independent restatements, and the tile-class spec."""

import numpy as np
import pytest

from aspec_amd import workloads as W
from oracle import metadata as M
from tests.conftest import load_golden


def _case(w, **masks):
    qaux, kaux = M.thd_aux(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                           w.block_size, w.sequence_length)
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length, **masks)
    return qaux, kaux, ends


def test_small_case_matches_hand_derived_fixture():
    g = load_golden("thd_small_case.json")
    docs, _, _, cu = M.pack_documents(g["lengths"], 40, pad_to_max_length=False)
    pos = np.arange(docs.size)  # context positions at CP=1 (thd_attention test: arange(33))
    anchors = np.array(g["anchors"])
    qaux, kaux = M.thd_aux(anchors, g["keep"], docs[anchors], pos, docs, g["block_size"], g["sequence_length"])
    eq = g["expected_query_aux"]
    ek = g["expected_key_aux"]
    np.testing.assert_array_equal(qaux, np.array([eq["anchors"], eq["keep"], eq["blocks"], eq["docs"]]))
    np.testing.assert_array_equal(kaux, np.array([ek["docs"], ek["positions"], ek["blocks"], ek["keep"]]))
    ends = M.endpoints(anchors, g["keep"], docs[anchors], pos, docs, g["block_size"], g["sequence_length"])
    np.testing.assert_array_equal(ends, np.array(g["expected_endpoints"]))
    np.testing.assert_array_equal(cu, [0, 9, 26, 33])


def test_dflash_truth_tables():
    g = load_golden("dflash_truth_tables.json")
    T, B = g["context_length"], g["block_size"]
    docs = np.zeros(T, np.int64)
    pos = np.arange(T)
    for case in g["cases"]:
        anchors = np.array(case["anchors"])
        qaux, kaux = M.thd_aux(anchors, case["keep"], np.zeros(anchors.size, np.int64), pos, docs, B, T)
        dense = M.thd_visibility(qaux, kaux, B)
        ends = M.endpoints(anchors, case["keep"], np.zeros(anchors.size, np.int64), pos, docs, B, T)
        from_ends = M.endpoints_to_dense(ends, T + anchors.size * B)
        np.testing.assert_array_equal(dense, from_ends)
        for q, keys in case["visible"]:
            assert dense[q, keys].all(), case["name"]
        for q, keys in case["invisible"]:
            assert not dense[q, keys].any(), case["name"]


LAYOUTS = [W.reference_test_layout(b) for b in (1, 7, 31, 257)] + [
    W.reference_test_layout(7, lengths=(257, 263, 19), drop_doc=False),
    W.config1(0), W.config1(3),
]
MASKS = [{}, {"query_window": 5}, {"query_window": 5, "draft_is_causal": True},
         {"draft_is_causal": True}, {"context_window": 40}]


@pytest.mark.parametrize("w", LAYOUTS, ids=lambda w: w.name)
@pytest.mark.parametrize("masks", MASKS, ids=str)
def test_three_restatements_agree(w, masks):
    """mask_mod brute force == endpoints == math `_visibility` (restricted to THD-kept rows)."""
    qaux, kaux, ends = _case(w, **masks)
    dense = M.thd_visibility(qaux, kaux, w.block_size, **masks)
    np.testing.assert_array_equal(M.endpoints_to_dense(ends, w.num_keys), dense)
    math = M.math_visibility(w.anchors, w.keep, w.context_positions, w.ctx_doc_ids, w.anchor_doc_ids,
                             w.block_size, w.sequence_length, **masks)
    # The math path's query keep omits the doc >= 0 test (direct_cp.py:370-379), the THD path has it
    # (thd_attention.py:33-35): they agree on every row whose anchor sits on a real document.
    real = np.repeat(w.anchor_doc_ids >= 0, w.block_size)
    key_real = np.concatenate([np.ones(w.context_length, bool), real])
    np.testing.assert_array_equal(math[real][:, key_real], dense[real][:, key_real])


@pytest.mark.parametrize("w", LAYOUTS[:5], ids=lambda w: w.name)
@pytest.mark.parametrize("tile", [(256, 128), (256, 80), (256, 64), (32, 64), (32, 128), (5, 3)])
@pytest.mark.parametrize("pad_visible", [True, False])
def test_tile_classes_from_endpoints_equal_bruteforce(w, tile, pad_visible):
    qaux, kaux, ends = _case(w, query_window=5, draft_is_causal=True)
    dense = M.thd_visibility(qaux, kaux, w.block_size, query_window=5, draft_is_causal=True)
    expected = M.tile_classes_dense(dense, *tile, pad_visible=pad_visible)
    got = M.tile_classes_from_endpoints(ends, w.num_queries, w.num_keys, *tile, pad_visible=pad_visible)
    np.testing.assert_array_equal(got, expected)


def test_tile_class_spec_padding_convention():
    # A 3x3 fully visible mask in 2x2 tiles: padding counts as visible for "full".
    vis = np.ones((3, 3), bool)
    np.testing.assert_array_equal(M.tile_classes_dense(vis, 2, 2, pad_visible=True), [[2, 2], [2, 2]])
    np.testing.assert_array_equal(M.tile_classes_dense(vis, 2, 2, pad_visible=False), [[2, 1], [1, 1]])
    vis[0, 0] = False
    np.testing.assert_array_equal(M.tile_classes_dense(vis, 2, 2), [[1, 2], [2, 2]])
    assert M.tile_classes_dense(np.zeros((2, 2), bool), 2, 2).tolist() == [[0]]


def test_ordered_lists_roundtrip_and_known_answer():
    blocks = np.array([[False, True, False, True], [False, False, False, False], [True, True, True, True]])
    cnt, idx = M.dense_to_ordered(blocks)
    np.testing.assert_array_equal(cnt, [2, 0, 4])
    np.testing.assert_array_equal(idx, [[1, 3, 0, 0], [0, 0, 0, 0], [0, 1, 2, 3]])
    np.testing.assert_array_equal(M.ordered_to_dense(cnt, idx, 4), blocks)


def test_config_pair_counts_match_flop_accounting():
    # Visible pairs per head of the benchmark configurations, reproduced by the seeded builders.
    assert M.visible_pairs(_case(W.config1(0))[2]) == 239360
    assert M.visible_pairs(_case(W.config2())[2]) == 16842752
    assert M.visible_pairs(_case(W.config4())[2]) == 537133056
    w = W.config2()
    # Closed form: sum over blocks of B * (anchor + B).
    assert M.visible_pairs(_case(w)[2]) == int(np.sum(w.block_size * (w.anchors + w.block_size)))


def test_packing_layout():
    docs, pos, mask, cu = M.pack_documents([3, 2], 7)
    np.testing.assert_array_equal(docs, [0, 0, 0, 1, 1, -1, -1])
    np.testing.assert_array_equal(pos, [0, 1, 2, 0, 1, 0, 0])
    np.testing.assert_array_equal(mask, [1, 1, 1, 1, 1, 0, 0])
    np.testing.assert_array_equal(cu, [0, 3, 5])
    with pytest.raises(ValueError):
        M.pack_documents([5, 5], 7)
