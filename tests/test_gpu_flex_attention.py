"""The cuDNN FlexAttention surface (aspec_amd.cudnn_flex_attention) and batch > 1 Direct-CP rows on
the GPU.

- `build_dspark_mla_mask` (HIP) bit-exact against the oracle restatement (oracle/flex_mask.py,
  pinned against the reference's mask_mod brute force) on the reference's own cases, plus padded,
  unsorted and windowed documents; the reference's errors.
- The interval-union -> two-interval conversion (HIP) bit-exact against the oracle for BSHD and THD
  masks, and its errors.
- `cudnn_flex_attention` called exactly as aspec/models/draft/dflash.py:932-942 calls it, on a
  2-row padded BSHD batch at BASELINE config-1 geometry (GQA 32/8 x 128, block 16, an anchor every
  64 document tokens), against the dense fp32 math oracle with the mask_mod's visibility; the same
  data as THD with cu_seqlens gives bitwise the same result.
- `DirectCPMetadata` with batch 2: unpacked rows, and packed rows on the cuDNN backend at the
  reference's own CP1 test geometry (tests/test_cudnn_flex_attention.py:402-458) with its bars.
Attention tolerances: the reference's bf16-vs-math bars, atol = rtol = 0.025 (O, LSE) and 0.04
(gradients) (tests/test_thd_attention.py:218-225), or the cuDNN route's 0.025 / 0.035 and
0.06 / 0.08 where the reference's cuDNN test uses them.
"""

import numpy as np
import pytest
import torch

from aspec_amd import workloads as W
from aspec_amd.cudnn_flex_attention import CudnnFlexMask, build_dspark_mla_mask, cudnn_flex_attention
from aspec_amd.direct_cp import DirectCPMetadata, direct_cp_attention, direct_cp_attention_from_kv
from oracle import attention as A
from oracle import flex_mask as F
from oracle import metadata as M

pytestmark = pytest.mark.gpu


def _report(name, got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    err = (got - ref).abs().max().item() if got.numel() else 0.0
    rel = ((got - ref).norm() / ref.norm().clamp_min(1e-30)).item()
    print(f"{name}: max_abs={err:.3e} rel_l2={rel:.3e}", flush=True)


def _mask_gpu(gpu, anchors, keep, ctx, block, docs=None, **opts):
    t = lambda x, dt: torch.as_tensor(np.asarray(x), dtype=dt, device=gpu)  # noqa: E731
    return build_dspark_mla_mask(anchor_positions=t(anchors, torch.long), block_keep_mask=t(keep, torch.bool),
                                 context_length=ctx, block_size=block,
                                 ctx_doc_ids=None if docs is None else t(docs, torch.long), **opts)


@pytest.mark.parametrize("block", (5, 7))
@pytest.mark.parametrize(("is_causal", "sliding_window"), ((False, None), (True, None), (False, 4), (True, 4)))
def test_mla_mask_bit_exact_reference_cases(gpu, block, is_causal, sliding_window):
    anchors, keep = [[3, 12], [7, 16]], [[True, False], [True, True]]
    got = _mask_gpu(gpu, anchors, keep, 20, block, is_causal=is_causal, sliding_window=sliding_window)
    want = F.dspark_mla_mask(anchors, keep, 20, block, is_causal=is_causal, sliding_window=sliding_window)
    assert got.mask_func.dtype == torch.int32
    np.testing.assert_array_equal(got.mask_func.cpu().numpy(), want)


@pytest.mark.parametrize("window", (None, 2, 5))
@pytest.mark.parametrize("causal_sliding", (False, True))
def test_mla_mask_bit_exact_documents(gpu, window, causal_sliding):
    cases = [
        ([[3, 8, 16]], [[True] * 3], [[0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2, 2, 3, 3, 3]], 20, 5),
        ([[1, 6, 9, 13], [0, 4, 9, 12]], [[True, True, True, True], [True, False, True, True]],
         [[2, 2, 2, 0, 0, 0, 0, 0, 5, 5, 5, 5, -1, -1, -1, -1], [1] * 10 + [3] * 6], 16, 3),
    ]
    opts = dict(context_window=window)
    if causal_sliding:
        opts.update(is_causal=True, sliding_window=3)
    for anchors, keep, docs, ctx, block in cases:
        got = _mask_gpu(gpu, anchors, keep, ctx, block, docs, **opts)
        want = F.dspark_mla_mask(anchors, keep, ctx, block, ctx_doc_ids=docs, **opts)
        np.testing.assert_array_equal(got.mask_func.cpu().numpy(), want)


def test_mla_mask_long_rows_many_runs(gpu):
    """Document runs across several 1024-token scan chunks of the run-start kernel (two batch rows
    of 5000 tokens, 300 and 7 runs, a padding tail)."""
    rng = np.random.default_rng(5)
    docs = np.full((2, 5000), -1, np.int64)
    cuts = np.sort(rng.choice(np.arange(1, 4800), 299, replace=False))
    docs[0, :4800] = np.searchsorted(cuts, np.arange(4800), side="right")
    docs[1, :] = np.repeat(rng.permutation(7), [700, 800, 900, 600, 500, 1000, 500])
    anchors = np.sort(rng.choice(4790, (2, 64)), axis=1)
    keep = rng.random((2, 64)) < 0.8
    got = _mask_gpu(gpu, anchors, keep, 5000, 7, docs)
    np.testing.assert_array_equal(got.mask_func.cpu().numpy(),
                                  F.dspark_mla_mask(anchors, keep, 5000, 7, ctx_doc_ids=docs))


def test_mla_mask_errors_match_the_reference(gpu):
    keep = [[True, True]]
    with pytest.raises(ValueError, match="inside the context"):
        _mask_gpu(gpu, [[1, 8]], keep, 8, 5)
    with pytest.raises(ValueError, match="sliding_window"):
        _mask_gpu(gpu, [[1, 2]], keep, 8, 5, sliding_window=0)
    with pytest.raises(ValueError, match="contiguous run"):
        _mask_gpu(gpu, [[1, 2]], keep, 8, 5, [[0, 0, 1, 1, 0, 0, 2, 2]])
    with pytest.raises(ValueError, match="context_window"):
        _mask_gpu(gpu, [[1, 2]], keep, 8, 5, context_window=0)
    with pytest.raises(ValueError, match="identical"):
        _mask_gpu(gpu, [[1, 2]], [[True]], 8, 5)


def _random_union_mask(rng, rows, keys_of_row, ends):
    e = np.zeros((1, ends, rows), np.int64)
    for r in range(rows):
        n = keys_of_row(r)
        a, b, c = sorted(rng.integers(0, n + 1, 3))
        if ends == 3:
            e[0, :, r] = [a, b, c]
        else:
            e[0, :, r] = [[a, b, c, 0, 0], [0, a, b, b, c], [0, b, c, a, max(a, b)], [0, c, a, c, b]][r % 4]
    return e


def test_interval_conversion_bit_exact_bshd_and_thd(gpu):
    rng = np.random.default_rng(11)
    q = torch.empty(3, 40, 2, 128, device=gpu, dtype=torch.bfloat16)
    k = torch.empty(3, 90, 1, 128, device=gpu, dtype=torch.bfloat16)
    for ends in (3, 5):
        e = _random_union_mask(rng, 120, lambda r: 90, ends)
        mask = CudnnFlexMask(mask_func=torch.as_tensor(e, dtype=torch.int32, device=gpu))
        plan = mask.plan_for(q, k, k)
        np.testing.assert_array_equal(plan.endpoints.cpu().numpy(),
                                      F.intervals_to_endpoints(e, query_length=40, key_length=90))
        assert mask.plan_for(q, k, k) is plan  # cached per geometry
    cq, ck = np.array([0, 7, 50, 51, 80]), np.array([0, 20, 130, 131, 200])
    seg = lambda r: int(np.searchsorted(cq, r, side="right")) - 1  # noqa: E731
    e = _random_union_mask(rng, 80, lambda r: ck[seg(r) + 1] - ck[seg(r)], 5)
    i32 = lambda x: torch.as_tensor(x, dtype=torch.int32, device=gpu)  # noqa: E731
    mask = CudnnFlexMask(mask_func=i32(e), cu_seqlens_q=i32(cq), cu_seqlens_k=i32(ck), max_seqlen_q=43,
                         max_seqlen_k=110)
    plan = mask.plan_for(torch.empty(80, 2, 128, device=gpu), torch.empty(200, 1, 128, device=gpu),
                         torch.empty(200, 1, 128, device=gpu))
    np.testing.assert_array_equal(plan.endpoints.cpu().numpy(),
                                  F.intervals_to_endpoints(e, cu_seqlens_q=cq, cu_seqlens_k=ck))


def test_interval_conversion_errors(gpu):
    q = torch.empty(1, 1, 2, 128, device=gpu, dtype=torch.bfloat16)
    k = torch.empty(1, 8, 1, 128, device=gpu, dtype=torch.bfloat16)
    three = CudnnFlexMask(mask_func=torch.tensor([[[1], [2], [3], [5], [6]]], dtype=torch.int32, device=gpu))
    with pytest.raises(NotImplementedError, match="two disjoint"):
        three.plan_for(q, k, k)
    outside = CudnnFlexMask(mask_func=torch.tensor([[[9], [0], [0]]], dtype=torch.int32, device=gpu))
    with pytest.raises(ValueError, match="inside their sequence"):
        outside.plan_for(q, k, k)
    wrong_rows = CudnnFlexMask(mask_func=torch.zeros(1, 3, 2, dtype=torch.int32, device=gpu))
    with pytest.raises(ValueError, match="query rows"):
        wrong_rows.plan_for(q, k, k)


def _padded_config1_batch(seeds=(0, 1), T=4096):
    """Two config-1 rows (4 documents each, lengths seeded in [256, 1024]) padded to T tokens with
    document id -1, their anchor lists padded with dropped slots to one common length."""
    rows = [W.config1(s) for s in seeds]
    n = max(w.num_blocks for w in rows)
    anchors = np.zeros((len(rows), n), np.int64)
    keep = np.zeros((len(rows), n), bool)
    docs = np.full((len(rows), T), -1, np.int64)
    for b, w in enumerate(rows):
        docs[b, :w.context_length] = w.ctx_doc_ids
        anchors[b, :w.num_blocks] = w.anchors
        keep[b, :w.num_blocks] = True
    return anchors, keep, docs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_cudnn_flex_attention_dflash_call_padded_bshd_batch(gpu, dtype):
    """The Draft layer's own call (dflash.py:932-942): BSHD Q/K/V, mask from build_dspark_mla_mask
    with packed documents, pack_gqa=False, physical_gqa=True; forward, LSE and all gradients of a
    2-row padded batch against the fp32 oracle under the mask_mod's dense visibility, in bf16 and
    in fp16 (the reference's cuDNN route takes both, cudnn_flex_attention.py:353-356)."""
    anchors, keep, docs = _padded_config1_batch()
    T, block = docs.shape[1], 16
    mask = _mask_gpu(gpu, anchors, keep, T, block, docs)
    np.testing.assert_array_equal(mask.mask_func.cpu().numpy(),
                                  F.dspark_mla_mask(anchors, keep, T, block, ctx_doc_ids=docs))
    bsz, lq, nk = anchors.shape[0], anchors.shape[1] * block, T + anchors.shape[1] * block
    g = torch.Generator().manual_seed(17)
    q = (torch.randn(bsz, lq, 32, 128, generator=g) * 0.5).to(dtype)
    k = (torch.randn(bsz, nk, 8, 128, generator=g) * 0.5).to(dtype)
    v = (torch.randn(bsz, nk, 8, 128, generator=g) * 0.5).to(dtype)
    dout = torch.randn(bsz, lq, 32, 128, generator=g).to(dtype)
    dlse = torch.randn(bsz, 32, lq, generator=g) * 0.1
    results = {}
    for mode in ("auto", "internal"):
        qd, kd, vd = (t.to(gpu).requires_grad_() for t in (q, k, v))
        out, lse = cudnn_flex_attention(qd, kd, vd, mask=mask, scale=128 ** -0.5, pack_gqa=False,
                                        physical_gqa=True, gqa_mode=mode, return_lse=True)
        assert out.shape == (bsz, lq, 32, 128) and lse.shape == (bsz, 32, lq) and out.dtype == dtype
        ((out.float() * dout.to(gpu).float()).sum() + (lse * dlse.to(gpu)).sum()).backward()
        torch.cuda.synchronize()
        results[mode] = [x.detach().cpu() for x in (out, lse, qd.grad, kd.grad, vd.grad)]
    for a, b in zip(results["auto"], results["internal"]):
        assert torch.equal(a, b)  # every GQA policy runs the same kernels
    out, lse, dq, dk, dv = results["auto"]
    dense = F.dflash_mask_dense(anchors, keep, T, block, ctx_doc_ids=docs)
    for b in range(bsz):
        r_out, r_lse, (r_dq, r_dk, r_dv) = A.attention(
            q[b].transpose(0, 1).float(), k[b].transpose(0, 1).float(), v[b].transpose(0, 1).float(),
            dense[b], 128 ** -0.5, dout=dout[b].transpose(0, 1).float(), dlse=dlse[b], dtype=torch.float32)
        row_keep = torch.as_tensor(dense[b].any(-1))
        for name, got, ref, tol in (("O", out[b].transpose(0, 1), r_out, 0.025),
                                    ("dQ", dq[b].transpose(0, 1), r_dq, 0.04),
                                    ("dK", dk[b].transpose(0, 1), r_dk, 0.04),
                                    ("dV", dv[b].transpose(0, 1), r_dv, 0.04)):
            _report(f"row {b} {name}", got.float(), ref)
            torch.testing.assert_close(got.float(), ref, atol=tol, rtol=tol)
        _report(f"row {b} LSE", lse[b][:, row_keep], r_lse[:, row_keep])
        torch.testing.assert_close(lse[b][:, row_keep], r_lse[:, row_keep], atol=0.025, rtol=0.025)
        assert not out[b].transpose(0, 1)[:, ~row_keep].any()
        assert torch.all(lse[b][:, ~row_keep] == A.MASK_VALUE)
    # the same data as THD with cu_seqlens: bitwise the same outputs and gradients
    i32 = lambda x: torch.as_tensor(x, dtype=torch.int32, device=gpu)  # noqa: E731
    thd = CudnnFlexMask(mask_func=mask.mask_func, cu_seqlens_q=i32([0, lq, 2 * lq]),
                        cu_seqlens_k=i32([0, nk, 2 * nk]), max_seqlen_q=lq, max_seqlen_k=nk)
    qd, kd, vd = (t.to(gpu).flatten(0, 1).requires_grad_() for t in (q, k, v))
    out_t, lse_t = cudnn_flex_attention(qd, kd, vd, mask=thd, scale=128 ** -0.5, return_lse=True)
    assert out_t.shape == (bsz * lq, 32, 128) and lse_t.shape == (32, bsz * lq)
    ((out_t.float() * dout.to(gpu).flatten(0, 1).float()).sum()
     + (lse_t * dlse.to(gpu).transpose(0, 1).reshape(32, -1)).sum()).backward()
    assert torch.equal(out_t.detach().cpu().view(bsz, lq, 32, 128), out)
    assert torch.equal(lse_t.detach().cpu().view(32, bsz, lq).transpose(0, 1), lse)
    for got, ref in zip((qd.grad, kd.grad, vd.grad), (dq, dk, dv)):
        assert torch.equal(got.cpu().view(ref.shape), ref)


def test_cudnn_flex_attention_rejects_what_the_reference_rejects(gpu):
    mask = _mask_gpu(gpu, [[1, 4]], [[True, True]], 8, 2)
    q = torch.zeros(1, 4, 2, 128, device=gpu, dtype=torch.bfloat16)
    k = torch.zeros(1, 12, 1, 128, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="CudnnFlexMask"):
        cudnn_flex_attention(q, k, k, mask=mask.mask_func, scale=1.0)
    with pytest.raises(ValueError, match="CUDA"):
        cudnn_flex_attention(q.cpu(), k.cpu(), k.cpu(), mask=mask, scale=1.0)
    with pytest.raises(TypeError, match="FP16 or BF16"):
        cudnn_flex_attention(q.float(), k.float(), k.float(), mask=mask, scale=1.0)
    with pytest.raises(ValueError, match="rank-4 BSHD or rank-3 THD"):
        cudnn_flex_attention(q[0, 0], k[0, 0], k[0, 0], mask=mask, scale=1.0)
    with pytest.raises(ValueError, match="cumulative sequence lengths"):
        cudnn_flex_attention(q[0], k[0], k[0], mask=mask, scale=1.0)
    with pytest.raises(ValueError, match="divisible"):
        cudnn_flex_attention(torch.zeros(1, 4, 3, 128, device=gpu, dtype=torch.bfloat16),
                             torch.zeros(1, 12, 2, 128, device=gpu, dtype=torch.bfloat16),
                             torch.zeros(1, 12, 2, 128, device=gpu, dtype=torch.bfloat16), mask=mask, scale=1.0)
    with pytest.raises(ValueError, match=r"\(Dqk,Dv\)"):
        cudnn_flex_attention(q[..., :64], k[..., :64], k[..., :64], mask=mask, scale=1.0)
    with pytest.raises(ValueError, match="GQA mode"):
        cudnn_flex_attention(q, k, k, mask=mask, scale=1.0, gqa_mode="bogus")
    with pytest.raises(TypeError, match="same dtype"):
        cudnn_flex_attention(q, k.half(), k.half(), mask=mask, scale=1.0)


def _direct_cp_oracle(anchors, keep, positions, docs, adocs, block, seq, q, k, v, dout, dlse, b):
    ends = M.endpoints(anchors[b], keep[b], adocs[b] if adocs is not None else np.zeros(anchors.shape[1]),
                       positions[b], docs[b] if docs is not None else np.zeros(positions.shape[1], np.int64),
                       block, seq)
    vis = M.endpoints_to_dense(ends, positions.shape[1] + anchors.shape[1] * block)
    return A.attention(q[b].float(), k[b].float(), v[b].float(), vis, 128 ** -0.5, dout=dout[b].float(),
                       dlse=dlse[b], dtype=torch.float32), vis


def test_direct_cp_unpacked_batch_of_two(gpu):
    """Unpacked rows (no documents), batch 2, the default FA4 backend name: the reference serves
    these through FA4's batch dimension (direct_cp.py:585-747)."""
    rng = np.random.default_rng(3)
    T, n, block = 700, 24, 16
    anchors = np.sort(rng.choice(T - block, (2, n), replace=False), axis=1)
    keep = rng.random((2, n)) < 0.85
    positions = np.broadcast_to(np.arange(T), (2, T)).copy()
    t = lambda x, dt: torch.as_tensor(x, dtype=dt, device=gpu)  # noqa: E731
    meta = DirectCPMetadata(t(anchors, torch.long), t(keep, torch.bool), t(positions, torch.long), block,
                            0, 1, None, sequence_length=T)
    g = torch.Generator().manual_seed(8)
    nq, nk = n * block, T + n * block
    q = (torch.randn(2, 8, nq, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(2, 2, nk, 128, generator=g) * 0.5).bfloat16()
    v = (torch.randn(2, 2, nk, 128, generator=g) * 0.5).bfloat16()
    dout = torch.randn(2, 8, nq, 128, generator=g).bfloat16()
    dlse = torch.randn(2, 8, nq, generator=g) * 0.1
    # token-major storage, as DFlashAttention hands the op its [B, H, L, D] views
    dev = lambda x: x.transpose(1, 2).contiguous().to(gpu).transpose(1, 2).requires_grad_()  # noqa: E731
    qd, kd, vd = dev(q), dev(k), dev(v)
    out, lse = direct_cp_attention_from_kv(qd, kd, vd, meta)
    assert out.shape == (2, 8, nq, 128) and lse.shape == (2, 8, nq)
    ((out.float() * dout.to(gpu).float()).sum() + (lse * dlse.to(gpu)).sum()).backward()
    for b in range(2):
        (r_out, r_lse, (r_dq, r_dk, r_dv)), vis = _direct_cp_oracle(
            anchors, keep, positions, None, None, block, T, q, k, v, dout, dlse, b)
        row_keep = torch.as_tensor(vis.any(-1))
        torch.testing.assert_close(out[b].detach().float().cpu(), r_out, atol=0.025, rtol=0.025)
        torch.testing.assert_close(lse[b].detach().cpu()[:, row_keep], r_lse[:, row_keep], atol=0.025, rtol=0.025)
        for name, got, ref in (("dQ", qd.grad[b], r_dq), ("dK", kd.grad[b], r_dk), ("dV", vd.grad[b], r_dv)):
            _report(f"unpacked row {b} {name}", got.float().cpu(), ref)
            torch.testing.assert_close(got.float().cpu(), ref, atol=0.04, rtol=0.04)


def test_direct_cp_packed_batch_of_two_cudnn_backend(gpu):
    """tests/test_cudnn_flex_attention.py:402-458: batch 2, GQA 4/2, context 128 of four 32-token
    documents, block 5, head-major inputs through direct_cp_attention on the cuDNN backend, forward
    and LSE within 0.025 / 0.035 and gradients within 0.06 / 0.08 of the math path. The FA4 backend
    keeps the reference's one-row rule for packed rows."""
    anchors = np.array([[17, 49, 81, 113], [19, 51, 83, 115]])
    keep = np.ones_like(anchors, bool)
    block, T = 5, 128
    docs = np.broadcast_to(np.repeat(np.arange(4), 32), (2, T)).copy()
    adocs = np.take_along_axis(docs, anchors, 1)
    positions = np.broadcast_to(np.arange(T), (2, T)).copy()
    t = lambda x: torch.as_tensor(x, device=gpu)  # noqa: E731
    common = dict(anchor_positions=t(anchors), block_keep_mask=t(keep), context_position_ids=t(positions),
                  context_doc_ids=t(docs), anchor_doc_ids=t(adocs), block_size=block, cp_rank=0, cp_size=1,
                  group=None, sequence_length=T)
    g = torch.Generator().manual_seed(821)
    nq = anchors.shape[1] * block
    shapes = ((2, 4, nq, 128), (2, 2, T, 128), (2, 2, T, 128), (2, 2, nq, 128), (2, 2, nq, 128))
    inputs = [torch.randn(s, generator=g).bfloat16() for s in shapes]
    dev = [x.to(gpu).requires_grad_() for x in inputs]
    out, lse = direct_cp_attention(*dev, DirectCPMetadata(**common, backend="cudnn_flex_attention"))
    dout = torch.randn(out.shape, generator=g)
    dlse = torch.randn(lse.shape, generator=g)
    ((out.float() * dout.to(gpu)).sum() + 0.01 * (lse * dlse.to(gpu)).sum()).backward()
    k = torch.cat((inputs[1], inputs[3]), 2)
    v = torch.cat((inputs[2], inputs[4]), 2)
    for b in range(2):
        (r_out, r_lse, (r_dq, r_dk, r_dv)), _ = _direct_cp_oracle(
            anchors, keep, positions, docs, adocs, block, T, inputs[0], k, v, dout, 0.01 * dlse, b)
        torch.testing.assert_close(out[b].detach().float().cpu(), r_out, atol=0.025, rtol=0.035)
        torch.testing.assert_close(lse[b].detach().cpu(), r_lse, atol=0.025, rtol=0.035)
        grads = (dev[0].grad[b], dev[1].grad[b], dev[2].grad[b], dev[3].grad[b], dev[4].grad[b])
        refs = (r_dq, r_dk[:, :T], r_dv[:, :T], r_dk[:, T:], r_dv[:, T:])
        for got, ref in zip(grads, refs):
            torch.testing.assert_close(got.float().cpu(), ref, atol=0.06, rtol=0.08)
    with pytest.raises(ValueError, match="one controller-owned row"):
        direct_cp_attention(*[x.detach() for x in dev], DirectCPMetadata(**common, backend="fa4"))


def _grads_fresh(fn, inputs, dout):
    out = fn(*inputs)
    return torch.autograd.grad(out, inputs, dout)


def test_cudnn_flex_attention_multiple_live_autograd_graphs(gpu):
    """Two pending graphs over one mask, consumed in reverse order (the reference's
    tests/test_cudnn_internal_gqa_gpu.py:93-123): each call owns its scratch, so each graph's
    gradients equal a fresh forward + backward of the same inputs bit for bit (the HIP backward
    is deterministic), for both GQA modes."""
    torch.manual_seed(330)
    qshape, kshape = (1, 71, 8, 128), (1, 229, 2, 128)
    ends = torch.full((71,), 229, device=gpu, dtype=torch.int32)
    zeros = torch.zeros_like(ends)
    mask = CudnnFlexMask(torch.stack((zeros, zeros, ends, ends, ends))[None])
    for mode in ("internal", "native"):
        inputs = [[torch.randn(shape, device=gpu, dtype=torch.bfloat16).requires_grad_()
                   for shape in (qshape, kshape, kshape)] for _ in range(2)]
        dout = [torch.randn(qshape, device=gpu, dtype=torch.bfloat16) for _ in inputs]
        fn = lambda q, k, v: cudnn_flex_attention(q, k, v, mask=mask, scale=128 ** -0.5, gqa_mode=mode)  # noqa: E731
        outputs = [fn(*values) for values in inputs]
        actual = [None, None]
        for index in (1, 0):
            actual[index] = torch.autograd.grad(outputs[index], inputs[index], dout[index])
        for values, grads, d in zip(inputs, actual, dout):
            expected = _grads_fresh(fn, values, d)
            for got, ref in zip(grads, expected):
                assert torch.equal(got, ref)
                assert torch.isfinite(got).all()


def test_direct_cp_multiple_live_autograd_graphs(gpu):
    """The same for `direct_cp_attention_from_kv`: two pending graphs sharing one metadata object
    (and so one cached plan), consumed in reverse order, each equal bit for bit to a fresh
    forward + backward, and the first also within the reference's bars of the oracle."""
    w = W.config1(0)
    w.q_heads, w.kv_heads = 8, 2
    meta = W.metadata_for(w, gpu)
    g = torch.Generator(device=gpu).manual_seed(331)

    def rows(n, h):
        return torch.randn(1, n, h, w.head_dim, device=gpu, generator=g).to(torch.bfloat16).transpose(1, 2)

    inputs = [[rows(w.num_queries, 8).requires_grad_(), rows(w.num_keys, 2).requires_grad_(),
               rows(w.num_keys, 2).requires_grad_()] for _ in range(2)]
    dout = [rows(w.num_queries, 8) for _ in inputs]
    fn = lambda q, k, v: direct_cp_attention_from_kv(q, k, v, meta)[0]  # noqa: E731
    outputs = [fn(*values) for values in inputs]
    actual = [None, None]
    for index in (1, 0):
        actual[index] = torch.autograd.grad(outputs[index], inputs[index], dout[index])
    for values, grads, d in zip(inputs, actual, dout):
        expected = _grads_fresh(fn, values, d)
        for got, ref in zip(grads, expected):
            assert torch.equal(got, ref)
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length)
    vis = M.endpoints_to_dense(ends, w.num_keys)
    q, k, v = (x.detach()[0].float().cpu() for x in inputs[0])
    _, _, ref = A.attention(q, k, v, vis, w.head_dim ** -0.5, dout=dout[0][0].float().cpu(),
                            dtype=torch.float32)
    for got, r in zip(actual[0], ref):
        torch.testing.assert_close(got[0].float().cpu(), r, atol=0.04, rtol=0.04)
