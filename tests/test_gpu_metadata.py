"""HIP integer metadata vs the oracle: bit-exact (aux tensors, endpoints, tile classes, lists)."""

import numpy as np
import pytest
import torch

from aspec_amd import workloads as W
from aspec_amd.direct_cp import thd_row_metadata
from aspec_amd.thd_sparse_metadata import build_thd_sparse_pair, tile_metadata
from oracle import metadata as M
from tests.conftest import load_golden

pytestmark = pytest.mark.gpu

LAYOUTS = [W.reference_test_layout(b) for b in (1, 7, 31, 257)] + [
    W.reference_test_layout(7, drop_doc=False), W.config1(0), W.config1(3),
]
MASKS = [{}, {"query_window": 5}, {"query_window": 5, "draft_is_causal": True},
         {"draft_is_causal": True}, {"context_window": 40}]


def _oracle(w, **masks):
    qaux, kaux = M.thd_aux(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                           w.block_size, w.sequence_length)
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length, **masks)
    return qaux, kaux, ends


def _hip_rows(w, device, **masks):
    meta = W.metadata_for(w, device, **masks)
    rows = thd_row_metadata(meta, device)
    torch.cuda.synchronize()
    return rows


def test_small_case_matches_hand_derived_fixture(gpu):
    g = load_golden("thd_small_case.json")
    anchors = np.array(g["anchors"])
    docs = np.concatenate([np.full(n, i) for i, n in enumerate(g["lengths"])])
    w = W.from_layout("small", g["lengths"], anchors, docs[anchors], g["block_size"], keep=g["keep"])
    rows = _hip_rows(w, gpu)
    eq, ek = g["expected_query_aux"], g["expected_key_aux"]
    np.testing.assert_array_equal(rows.query_aux.cpu().numpy(),
                                  np.array([eq["anchors"], eq["keep"], eq["blocks"], eq["docs"]]))
    np.testing.assert_array_equal(rows.key_aux.cpu().numpy(),
                                  np.array([ek["docs"], ek["positions"], ek["blocks"], ek["keep"]]))
    np.testing.assert_array_equal(rows.endpoints.cpu().numpy(), np.array(g["expected_endpoints"]))
    assert int(rows.flags.item()) == 0


def test_dflash_truth_tables(gpu):
    g = load_golden("dflash_truth_tables.json")
    T, B = g["context_length"], g["block_size"]
    for case in g["cases"]:
        anchors = np.array(case["anchors"])
        w = W.from_layout(case["name"], [T], anchors, np.zeros(anchors.size, np.int64), B,
                          keep=case["keep"])
        dense = M.endpoints_to_dense(_hip_rows(w, gpu).endpoints.cpu().numpy(), w.num_keys)
        for q, keys in case["visible"]:
            assert dense[q, keys].all(), case["name"]
        for q, keys in case["invisible"]:
            assert not dense[q, keys].any(), case["name"]


@pytest.mark.parametrize("w", LAYOUTS, ids=lambda w: w.name)
@pytest.mark.parametrize("masks", MASKS, ids=str)
def test_row_metadata_bit_exact(gpu, w, masks):
    qaux, kaux, ends = _oracle(w, **masks)
    rows = _hip_rows(w, gpu, **masks)
    np.testing.assert_array_equal(rows.query_aux.cpu().numpy(), qaux)
    np.testing.assert_array_equal(rows.key_aux.cpu().numpy(), kaux)
    np.testing.assert_array_equal(rows.endpoints.cpu().numpy(), ends)
    assert int(rows.flags.item()) == 0


@pytest.mark.parametrize("w", LAYOUTS, ids=lambda w: w.name)
@pytest.mark.parametrize("masks", MASKS, ids=str)
@pytest.mark.parametrize("tile", [(256, 128), (256, 80), (256, 64), (32, 64), (32, 128), (5, 3)])
def test_sparse_pair_from_aux_bit_exact(gpu, w, masks, tile, monkeypatch):
    """build_thd_sparse_pair on the eight mask tensors == brute-force any/all classes
    (tests/test_thd_sparse_metadata.py:187-200) turned into ordered lists."""
    from aspec_amd import thd_sparse_metadata as S

    monkeypatch.setattr(S, "sparse_block_sizes", lambda *a: (tile, tile))
    qaux, kaux, _ = _oracle(w)
    dense = M.thd_visibility(qaux, kaux, w.block_size, **masks)
    classes = M.tile_classes_dense(dense, *tile)
    (pc, pi, fc, fi), (bpc, bpi, bfc, bfi) = M.sparse_lists(classes)
    aux = [torch.as_tensor(x[None], device=gpu).contiguous() for x in list(qaux) + list(kaux)]
    pair = build_thd_sparse_pair(aux_tensors=aux, block_size=w.block_size,
                                 query_length=w.num_queries, key_length=w.num_keys,
                                 query_head_dim=128, value_head_dim=128, **masks)
    f, b = pair.forward, pair.backward
    for got, exp in ((f.mask_block_cnt, pc), (f.mask_block_idx, pi), (f.full_block_cnt, fc),
                     (f.full_block_idx, fi), (b.mask_block_cnt, bpc), (b.mask_block_idx, bpi),
                     (b.full_block_cnt, bfc), (b.full_block_idx, bfi)):
        np.testing.assert_array_equal(got[0, 0].cpu().numpy(), exp)


@pytest.mark.parametrize("w", [W.config1(0), W.config2(), W.config3(0, 0), W.config3(0, 1), W.config4()],
                         ids=lambda w: w.name)
def test_config_metadata_bit_exact(gpu, w):
    _, _, ends = _oracle(w)
    rows = _hip_rows(w, gpu)
    np.testing.assert_array_equal(rows.endpoints.cpu().numpy(), ends)
    for tile, pad in (((256, 128), True), ((32, 64), False), ((32, 128), False)):
        lists = tile_metadata(rows.endpoints, query_length=w.num_queries, key_length=w.num_keys,
                              tile_m=tile[0], tile_n=tile[1], pad_visible=pad)
        classes = M.tile_classes_from_endpoints(ends, w.num_queries, w.num_keys, *tile, pad_visible=pad)
        np.testing.assert_array_equal(lists["classes"].cpu().numpy(), classes)
        (pc, pi, fc, fi), (bpc, bpi, bfc, bfi) = M.sparse_lists(classes)
        for name, exp in (("fwd_partial_cnt", pc), ("fwd_partial_idx", pi), ("fwd_full_cnt", fc),
                          ("fwd_full_idx", fi), ("bwd_partial_cnt", bpc), ("bwd_partial_idx", bpi),
                          ("bwd_full_cnt", bfc), ("bwd_full_idx", bfi)):
            np.testing.assert_array_equal(lists[name].cpu().numpy(), exp, err_msg=name)


def test_layout_violations_fail_closed(gpu):
    w = W.config1(0)
    meta = W.metadata_for(w, gpu)
    meta.context_position_ids = meta.context_position_ids.flip(1)
    rows = thd_row_metadata(meta, gpu)
    with pytest.raises(ValueError, match="monotonically"):
        rows.check_layout()


@pytest.mark.parametrize("masks", MASKS, ids=str)
def test_batched_row_metadata_bit_exact(gpu, masks):
    """aspec_thd_batch_row_metadata over three packed rows of one common geometry (the
    DirectCPMetadata [batch, ...] form): each row's aux tensors and endpoints equal the oracle's for
    that row, the endpoints shifted into the flattened key space (row b's keys start at b*K) and
    dropped rows all zero."""
    from aspec_amd.direct_cp import DirectCPMetadata

    rows = [W.reference_test_layout(7), W.reference_test_layout(7, drop_doc=False),
            W.reference_test_layout(7, lengths=(100, 400, 39))]
    n, T = rows[0].num_blocks, rows[0].context_length
    assert all(w.num_blocks == n and w.context_length == T for w in rows)
    t = lambda key, dt: torch.as_tensor(np.stack([getattr(w, key) for w in rows]), dtype=dt, device=gpu)  # noqa: E731
    meta = DirectCPMetadata(t("anchors", torch.long), t("keep", torch.bool), t("context_positions", torch.long),
                            7, 0, 1, None, context_doc_ids=t("ctx_doc_ids", torch.long),
                            anchor_doc_ids=t("anchor_doc_ids", torch.long), sequence_length=T,
                            backend="cudnn_flex_attention", **masks)
    got = thd_row_metadata(meta, gpu)
    torch.cuda.synchronize()
    nq, nk = rows[0].num_queries, rows[0].num_keys
    assert got.num_queries == 3 * nq and got.num_keys == 3 * nk and int(got.flags.item()) == 0
    for b, w in enumerate(rows):
        qaux, kaux, ends = _oracle(w, **masks)
        np.testing.assert_array_equal(got.query_aux[:, b * nq:(b + 1) * nq].cpu().numpy(), qaux)
        np.testing.assert_array_equal(got.key_aux[:, b * nk:(b + 1) * nk].cpu().numpy(), kaux)
        kept = ends[2] > ends[1]
        kept |= ends[4] > ends[3]
        shifted = np.where(kept[None], ends + np.array([0, 1, 1, 1, 1])[:, None] * b * nk, 0)
        np.testing.assert_array_equal(got.endpoints[:, b * nq:(b + 1) * nq].cpu().numpy(), shifted)
