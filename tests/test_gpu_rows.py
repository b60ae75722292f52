"""HIP row-level operations vs the oracle, bit-exact: the packing collator, the anchor samplers
and injected-anchor validation, output-block layout and the DSpark targets."""

import numpy as np
import pytest
import torch

from aspec_amd import anchors as A
from aspec_amd import collate as C
from aspec_amd import targets as T
from aspec_amd import output_blocks as O
from oracle import rows as R

pytestmark = pytest.mark.gpu


def _np(t):
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.view(torch.int16)  # compare bit patterns
    return t.detach().cpu().numpy()


def _host(features):
    return [{k: (_np(v) if isinstance(v, torch.Tensor) else v) for k, v in f.items()} for f in features]


# ---------------------------------------------------------------- a1 packing
def _features(lengths, device, hidden=24, seed=0, dtype=torch.bfloat16, mask_dtype=torch.long):
    g = torch.Generator().manual_seed(seed)
    feats = []
    for i, n in enumerate(lengths):
        extra = 3  # the collator slices longer fields to the document length
        feats.append({
            "input_ids": torch.randint(0, 1000, (1, n), generator=g).to(device),
            "loss_mask": (torch.rand(1, n + extra, generator=g) > 0.3).to(mask_dtype).to(device),
            "hidden_states": torch.randn(1, n + extra, hidden, generator=g).to(dtype).to(device),
            "last_hidden_states": torch.randn(1, n, hidden, generator=g).to(dtype).to(device),
            "_aspec_work": {"execution_id": f"e{i}"},
        })
    return feats


@pytest.mark.parametrize("lengths,max_len,pad", [((3, 2), 8, True), ((910, 745, 649, 463), 4096, True),
                                                 ((5, 1, 7), 13, True), ((300, 17), 1024, False),
                                                 ((4096,), 4096, True)])
def test_collator_matches_oracle(gpu, lengths, max_len, pad):
    feats = _features(lengths, gpu, hidden=40 if len(lengths) != 1 else 4096)
    out = C.DFlashPackingCollator(max_len, pad_to_max_length=pad)(feats)
    torch.cuda.synchronize()
    ref = R.pack_row(_host(feats), max_len, pad_to_max_length=pad)
    for key in ("input_ids", "loss_mask", "ctx_doc_ids", "base_position_ids", "attention_mask",
                "cu_seqlens", "hidden_states", "last_hidden_states"):
        np.testing.assert_array_equal(_np(out[key]), ref[key], err_msg=key)
    assert out["packed_document_lengths"] == tuple(lengths)
    assert [w["execution_id"] for w in out["_aspec_work"]] == [f"e{i}" for i in range(len(lengths))]


def test_collator_context_parallel_shards(gpu):
    lengths = (37, 64, 9)
    for rank in range(3):
        bounds = [C.context_shard_bounds(n, rank, 3, alignment=4) for n in lengths]
        feats = _features(lengths, gpu, hidden=8)
        for f, (s, e) in zip(feats, bounds):
            f["hidden_states"] = f["hidden_states"][:, s:e].contiguous()
            f["last_hidden_states"] = f["last_hidden_states"][:, s:e].contiguous()
        out = C.DFlashPackingCollator(256, pad_to_max_length=False, context_parallel_rank=rank,
                                      context_parallel_size=3, context_shard_alignment=4)(feats)
        ref = R.pack_row(_host(feats), 256, pad_to_max_length=False, cp_rank=rank, cp_size=3,
                         cp_alignment=4)
        np.testing.assert_array_equal(_np(out["hidden_states"]), ref["hidden_states"])
        np.testing.assert_array_equal(_np(out["input_ids"]), ref["input_ids"])
        np.testing.assert_array_equal(_np(out["packed_context_positions"]), ref["packed_context_positions"])


# ---------------------------------------------------------------- a2 anchors
def _row(lengths, seed, hole=0.2):
    rng = np.random.default_rng(seed)
    mask = (rng.random(sum(lengths)) > hole).astype(np.float32)
    docs = np.concatenate([np.full(n, i) for i, n in enumerate(lengths)]).astype(np.int64)
    return mask, docs


@pytest.mark.parametrize("lengths,anchors,block,align", [
    ((9, 13, 30), 4, 4, 1), ((80,), 512, 4, 1), ((20, 51), 512, 4, 4), ((3, 19, 4, 31), 8, 4, 4),
    ((910, 745, 649, 463), 512, 16, 1), ((4096,), 512, 16, 8), (tuple([33] * 100), 512, 7, 4),
])
def test_document_sampler_matches_oracle(gpu, lengths, anchors, block, align):
    for seed in range(3):
        mask, docs = _row(lengths, seed)
        gen = torch.Generator(device=gpu).manual_seed(seed)
        a, k = A.sample_document_anchor_positions(torch.from_numpy(mask)[None].to(gpu),
                                                  torch.from_numpy(docs)[None].to(gpu), lengths,
                                                  anchors, block, generator=gen, alignment=align)
        gen.manual_seed(seed)
        u = _np(torch.rand(len(lengths), device=gpu, generator=gen))
        ra, rk = R.sample_document_anchors(mask, docs, lengths, anchors, block, u, alignment=align)
        np.testing.assert_array_equal(_np(a)[0], ra)
        np.testing.assert_array_equal(_np(k)[0], rk)


def test_document_sampler_mask_dtypes_agree(gpu):
    lengths = (40, 70)
    mask, docs = _row(lengths, 5)
    results = []
    for dt in (torch.float32, torch.long, torch.int32, torch.bool, torch.bfloat16, torch.float16):
        gen = torch.Generator(device=gpu).manual_seed(11)
        a, k = A.sample_document_anchor_positions(torch.from_numpy(mask)[None].to(gpu).to(dt),
                                                  torch.from_numpy(docs)[None].to(gpu), lengths, 8, 4,
                                                  generator=gen)
        results.append((_np(a), _np(k)))
    for a, k in results[1:]:
        np.testing.assert_array_equal(a, results[0][0])
        np.testing.assert_array_equal(k, results[0][1])


@pytest.mark.parametrize("batch,seq,anchors,block,gap,with_attn", [
    (1, 40, 6, 4, 0, False), (2, 300, 16, 16, None, False), (3, 4096, 512, 16, None, True),
    (2, 17, 8, 16, 2, False), (4, 1000, 64, 8, 3, True),
])
def test_per_sample_sampler_matches_oracle(gpu, batch, seq, anchors, block, gap, with_attn):
    rng = np.random.default_rng(seq)
    mask = (rng.random((batch, seq)) > 0.25).astype(np.float32)
    attn = None
    if with_attn:
        attn = np.ones((batch, seq), np.int64)
        attn[:, seq - seq // 7:] = 0
    gen = torch.Generator(device=gpu).manual_seed(7)
    a, k = A.sample_anchor_positions(seq, torch.from_numpy(mask).to(gpu), anchors, block, gpu,
                                     max_gap=gap, generator=gen,
                                     attention_mask=None if attn is None else torch.from_numpy(attn).to(gpu))
    gen.manual_seed(7)
    u = _np(torch.rand(batch, 1, device=gpu, generator=gen))[:, 0]
    ra, rk = R.sample_anchors(mask, anchors, block, u, max_gap=gap, attention_mask=attn)
    np.testing.assert_array_equal(_np(a), ra)
    np.testing.assert_array_equal(_np(k), rk)


def test_validate_injected_anchors_matches_oracle(gpu):
    lm = np.ones((2, 64), np.float32)
    lm[0, 20] = 0
    docs = np.zeros((2, 64), np.int64)
    docs[:, 40:] = 1
    t = lambda x: torch.from_numpy(np.asarray(x)).to(gpu)  # noqa: E731
    good = np.array([[0, 5, 21, 44], [3, 9, 50, 60]])
    keep = np.array([[True, True, True, False], [True, False, True, True]])
    a, k = A.validate_injected_anchors(t(good), t(keep), loss_mask=t(lm), num_anchors=4, block_size=4,
                                       ctx_doc_ids=t(docs))
    ra, _ = R.validate_injected_anchors(good, keep, lm, 4, 4, ctx_doc_ids=docs)
    np.testing.assert_array_equal(_np(a), ra)
    cases = [
        (np.array([[63, 0, 0, 0], [0, 0, 0, 0]]), "in-bounds first prediction target"),
        (np.array([[19, 0, 0, 0], [0, 0, 0, 0]]), "must be supervised"),
        (np.array([[37, 0, 0, 0], [0, 0, 0, 0]]), "document boundaries"),
    ]
    for bad, msg in cases:
        kp = np.zeros((2, 4), bool)
        kp[0, 0] = True
        with pytest.raises(ValueError, match=msg):
            R.validate_injected_anchors(bad, kp, lm, 4, 4, ctx_doc_ids=docs)
        with pytest.raises(ValueError, match=msg):
            A.validate_injected_anchors(t(bad), t(kp), loss_mask=t(lm), num_anchors=4, block_size=4,
                                        ctx_doc_ids=t(docs))
    # nothing kept: returns zeros without the later checks
    a, k = A.validate_injected_anchors(t(cases[1][0]), t(np.zeros((2, 4), bool)), loss_mask=t(lm),
                                       num_anchors=4, block_size=4)
    assert not _np(a).any() and not _np(k).any()


# ---------------------------------------------------------------- a11 output blocks
@pytest.mark.parametrize("batch,slots,owners,p", [(1, 6, 1, 0.5), (2, 7, 1, 0.4), (2, 24, 4, 0.3),
                                                  (3, 512, 1, 0.9), (2, 2048, 8, 0.2), (1, 24, 4, 0.0),
                                                  (2, 300, 3, 1.0)])
def test_output_block_layout_matches_oracle(gpu, batch, slots, owners, p):
    rng = np.random.default_rng(slots + owners)
    keep = rng.random((batch, slots)) < p
    tk = torch.from_numpy(keep).to(gpu)
    for chunk in (1, 3, 4, 512):
        assert O.output_block_counts(tk, chunk) == R.output_block_counts(keep, chunk)
    got = O.output_block_indices(tk)
    ref = R.output_block_indices(keep)
    assert (got is None) == (ref is None)
    if ref is not None:
        np.testing.assert_array_equal(_np(got), ref)
    got = O.owner_block_indices(tk, owners)
    ref = R.owner_block_indices(keep, owners)
    assert (got is None) == (ref is None)
    if ref is not None:
        np.testing.assert_array_equal(_np(got), ref)
    for rank in range(owners):
        gi, gc = O.prepare_block_layout(tk, owners, rank, 4)
        ri, rc = R.prepare_block_layout(keep, owners, rank, 4)
        assert gc == rc
        assert (gi is None) == (ri is None)
        if ri is not None:
            np.testing.assert_array_equal(_np(gi), ri)


def test_select_and_restore_round_trip(gpu):
    keep = torch.tensor([[True, False, True, False], [False, True, False, False]], device=gpu)
    idx = O.output_block_indices(keep)
    value = torch.randn(2, 4, 3, 5, device=gpu)
    sel = O.select_blocks(value, idx)
    restored = O.restore_blocks(sel, idx, 4)
    torch.testing.assert_close(restored[keep], value[keep])


# ---------------------------------------------------------------- a12 DSpark targets
@pytest.mark.parametrize("batch,seq,blocks,block,ps,gamma,with_docs", [
    (1, 10, 2, 4, 0, 4.0, False), (1, 4096, 512, 16, 0, 4.0, True), (2, 700, 40, 16, 1, 2.5, True),
    (3, 64, 9, 7, 0, None, False), (1, 4096, 512, 16, 0, 0.0, False),
])
def test_dspark_targets_match_oracle(gpu, batch, seq, blocks, block, ps, gamma, with_docs):
    rng = np.random.default_rng(seq + blocks)
    ids = rng.integers(0, 32000, (batch, seq))
    lm = (rng.random((batch, seq)) > 0.1).astype(np.float32)
    anchors = np.sort(rng.integers(0, seq, (batch, blocks)), axis=1)
    keep = rng.random((batch, blocks)) > 0.2
    docs = np.cumsum(rng.random((batch, seq)) < 0.01, axis=1) if with_docs else None
    t = lambda x: None if x is None else torch.from_numpy(np.asarray(x)).to(gpu)  # noqa: E731
    out = T.dspark_targets(t(anchors), t(keep), t(ids), t(lm), block, loss_decay_gamma=gamma,
                           prediction_start=ps, ctx_doc_ids=t(docs))
    decay = _np(T.decay_weights(block, gamma, ps, gpu)).reshape(-1)
    ref = R.dspark_targets(anchors, keep, ids, lm, block, decay, ctx_doc_ids=docs, prediction_start=ps)
    for key in ("label_index", "target_ids", "prev_ids", "teacher_index"):
        np.testing.assert_array_equal(_np(getattr(out, key)), ref[key], err_msg=key)
    for key in ("eval_mask", "weights"):
        np.testing.assert_array_equal(_np(getattr(out, key)).view(np.int32), ref[key].view(np.int32),
                                      err_msg=key)
    # the decay table is the reference's own torch expression: exp(-k / gamma) to a few float32 ulp
    if gamma:
        ks = np.maximum(np.arange(block) - ps, 0)
        np.testing.assert_allclose(decay, np.exp(-ks / gamma), rtol=1e-6, atol=0)  # float32 exp of a float32 quotient
