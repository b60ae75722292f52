"""The one-layer DSpark training step on the GPU: RMSNorm (with the fused residual add), SwiGLU and
the fused AdamW against the fp64 oracle (bf16 tolerances stated per test), the composed layer
and its parameter gradients against the fp64 layer oracle at a reduced geometry and, on sampled
rows, against the fp32 row-restricted layer oracle at the full Qwen3-8B geometry (config 5), and
three full steps at that geometry."""

import numpy as np
import pytest
import torch

from aspec_amd import workloads as W
from aspec_amd.draft_layer import (DSparkDraftLayerModel, FusedBF16Optimizer, dspark_layer_step,
                                   layer_batch, rms_norm, swiglu, warmup_decay_lr)
from oracle import layer as ol
from oracle import loss as oloss
from oracle import metadata as M

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().double().cpu().numpy()


def _close(name, got, want, rel_l2, atol_frac):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want).max()
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    frac = err / max(np.abs(want).max(), 1e-30)
    print(f"{name}: max_abs={err:.3e} ({frac:.3e} of the largest value) rel_l2={rel:.3e}")
    assert rel < rel_l2, name
    assert err <= atol_frac * max(np.abs(want).max(), 1e-30), name


@pytest.mark.parametrize("hidden,residual", [(4096, False), (4096, True), (1000, True), (8192, False)])
def test_rmsnorm_matches_oracle(gpu, hidden, residual):
    g = torch.Generator(device=gpu).manual_seed(hidden)
    rows = 96
    x = (torch.randn(rows, hidden, device=gpu, generator=g) * 2).to(torch.bfloat16).requires_grad_()
    r = (torch.randn(rows, hidden, device=gpu, generator=g)).to(torch.bfloat16).requires_grad_() if residual else None
    w = (1 + 0.1 * torch.randn(hidden, device=gpu, generator=g)).to(torch.bfloat16).requires_grad_()
    out = rms_norm(x, w, 1e-6, residual=r)
    y, n = out if residual else (x, out)
    dn = torch.randn(rows, hidden, device=gpu, generator=g).to(torch.bfloat16)
    dy = torch.randn(rows, hidden, device=gpu, generator=g).to(torch.bfloat16) if residual else None
    outs, grads = ((y, n), (dy, dn)) if residual else ((n,), (dn,))
    torch.autograd.backward(outs, grads)
    ry, rn = ol.rms_norm(_np(x), _np(w), 1e-6, residual=None if r is None else _np(r))
    if residual:
        # y is bf16(x + r): compare exactly against the rounded oracle sum
        np.testing.assert_array_equal(_np(y), _np(torch.as_tensor(ry).to(torch.bfloat16)))
        ry = _np(y)
    _close("rmsnorm out", _np(n), ol.rms_norm(ry, _np(w), 1e-6)[1], 1e-2, 1e-2)
    gdy, gdw = ol.rms_norm_grad(ry, _np(w), 1e-6, _np(dn), None if dy is None else _np(dy))
    _close("rmsnorm dx", _np(x.grad), gdy, 1e-2, 2e-2)
    if residual:
        np.testing.assert_array_equal(_np(r.grad), _np(x.grad))
    _close("rmsnorm dw", _np(w.grad), gdw, 1e-2, 2e-2)


def test_swiglu_matches_oracle(gpu):
    g = torch.Generator(device=gpu).manual_seed(7)
    gu = (torch.randn(64, 2 * 12288, device=gpu, generator=g) * 2).to(torch.bfloat16).requires_grad_()
    out = swiglu(gu)
    d = torch.randn(out.shape, device=gpu, generator=g).to(torch.bfloat16)
    out.backward(d)
    _close("swiglu out", _np(out), ol.swiglu(_np(gu)), 1e-2, 1e-2)
    _close("swiglu dgu", _np(gu.grad), ol.swiglu_grad(_np(gu), _np(d)), 1e-2, 2e-2)


class _Params(torch.nn.Module):
    def __init__(self, gpu):
        super().__init__()
        g = torch.Generator(device=gpu).manual_seed(11)
        self.a = torch.nn.Parameter(torch.randn(1000, 37, device=gpu, generator=g).to(torch.bfloat16))
        self.b = torch.nn.Parameter(torch.randn(513, device=gpu, generator=g).to(torch.bfloat16))
        self.frozen = torch.nn.Parameter(torch.randn(9, device=gpu).to(torch.bfloat16), requires_grad=False)


def test_fused_adamw_matches_oracle_with_clip_skip_and_missing_gradients(gpu):
    """Five steps: gradients accumulated in place into the flat buffer (zero_grad(set_to_none=False))
    or left where autograd puts them (the default), a non-finite step (skipped), a clipped step, and
    a step in which `b` has no gradient (b untouched, and its bias corrections count its own
    steps)."""
    mod = _Params(gpu)
    opt = FusedBF16Optimizer(mod, lr=1e-2, weight_decay=0.1, max_grad_norm=5.0, total_steps=10,
                             warmup_ratio=0.2)
    p0 = _np(torch.cat([mod.a.detach().reshape(-1), mod.b.detach().reshape(-1)]).float())
    na, nb = mod.a.numel(), mod.b.numel()
    g = torch.Generator(device=gpu).manual_seed(12)
    grads, lrs, actives = [], [], []
    for step in range(5):
        in_place = step in (0, 2)
        opt.zero_grad(set_to_none=not in_place)
        ga = torch.randn(mod.a.shape, device=gpu, generator=g) * (0.05 if step != 2 else 3.0)
        gb = torch.randn(mod.b.shape, device=gpu, generator=g) * 0.05
        if step == 1:
            gb[5] = float("nan")  # a non-finite step: skipped
        (mod.a * ga.to(torch.bfloat16)).sum().backward()
        b_has_grad = step != 3
        if b_has_grad:
            (mod.b * gb.to(torch.bfloat16)).sum().backward()
        assert (mod.a.grad.data_ptr() == opt.grads.data_ptr()) == in_place  # accumulated in place
        grads.append(_np(torch.cat([mod.a.grad.reshape(-1),
                                    mod.b.grad.reshape(-1) if b_has_grad else torch.zeros_like(mod.b).reshape(-1)])))
        actives.append(np.concatenate([np.ones(na, bool), np.full(nb, b_has_grad)]))
        lrs.append(opt.get_learning_rate())
        b_before = _np(mod.b).copy()
        norm = opt.step()
        assert mod.a.grad is None and mod.b.grad is None  # consumed, as the reference's step does
        want_p, want_norms, want_t = ol.adamw_steps(p0, grads, lrs=lrs, weight_decay=0.1, max_grad_norm=5.0,
                                                    active=actives)
        got = _np(opt.master[: p0.size])
        print(f"step {step}: lr={lrs[-1]:.3e} norm={float(norm):.4f} oracle={want_norms[-1]:.4f}")
        if np.isfinite(want_norms[-1]):
            assert float(norm) == pytest.approx(want_norms[-1], rel=1e-4)
        else:
            assert not np.isfinite(float(norm))
        np.testing.assert_allclose(got, want_p[-1], rtol=1e-5, atol=1e-6)
        np.testing.assert_array_equal(_np(mod.a).reshape(-1), _np(opt.master[:na].to(torch.bfloat16)))
        if not b_has_grad:
            np.testing.assert_array_equal(_np(mod.b), b_before)
    assert opt.optimizer_steps() == 4
    assert lrs == [warmup_decay_lr(i, max_lr=1e-2, total_steps=10, warmup_steps=2) for i in range(5)]


class _OddParams(torch.nn.Module):
    """A parameter of 37 elements ahead of another: the segment table needs multiples of 8, so the
    optimizer takes its gathered path."""

    def __init__(self, gpu):
        super().__init__()
        g = torch.Generator(device=gpu).manual_seed(13)
        self.a = torch.nn.Parameter(torch.randn(37, device=gpu, generator=g).to(torch.bfloat16))
        self.b = torch.nn.Parameter(torch.randn(513, device=gpu, generator=g).to(torch.bfloat16))


def test_fused_adamw_gathered_path_matches_oracle_and_refuses_a_missing_gradient(gpu):
    """The gathered path (a parameter whose size is not a multiple of 8): with every gradient
    present it follows the optimizer oracle; a step in which one parameter has no gradient raises
    NotImplementedError before any state changes (it cannot skip the parameter as the reference's
    AdamW does); a step with no gradient at all leaves everything untouched."""
    mod = _OddParams(gpu)
    opt = FusedBF16Optimizer(mod, lr=1e-2, weight_decay=0.1, max_grad_norm=5.0, total_steps=10,
                             warmup_ratio=0.0)
    assert not opt._segments_ok
    p0 = _np(torch.cat([mod.a.detach().reshape(-1), mod.b.detach().reshape(-1)]).float())
    g = torch.Generator(device=gpu).manual_seed(14)
    grads, lrs = [], []
    for step in range(2):
        ga = torch.randn(mod.a.shape, device=gpu, generator=g) * 0.05
        gb = torch.randn(mod.b.shape, device=gpu, generator=g) * 0.05
        ((mod.a * ga.to(torch.bfloat16)).sum() + (mod.b * gb.to(torch.bfloat16)).sum()).backward()
        grads.append(_np(torch.cat([mod.a.grad.reshape(-1), mod.b.grad.reshape(-1)])))
        lrs.append(opt.get_learning_rate())
        norm = opt.step()
        want_p, want_norms, _ = ol.adamw_steps(p0, grads, lrs=lrs, weight_decay=0.1, max_grad_norm=5.0)
        assert float(norm) == pytest.approx(want_norms[-1], rel=1e-4)
        np.testing.assert_allclose(_np(opt.master[: p0.size]), want_p[-1], rtol=1e-5, atol=1e-6)
    master, exp_avg, state = opt.master.clone(), opt.exp_avg.clone(), opt.state.clone()
    (mod.a.float().sum()).backward()  # b has no gradient
    with pytest.raises(NotImplementedError, match="cannot skip"):
        opt.step()
    torch.cuda.synchronize()
    assert torch.equal(opt.master, master) and torch.equal(opt.exp_avg, exp_avg)
    assert torch.equal(opt.state, state)
    opt.zero_grad()
    before = _np(opt.master).copy()
    assert float(opt.step()) == 0.0  # nothing to update
    np.testing.assert_array_equal(_np(opt.master), before)


def test_adamw_segments_match_the_flat_step_bit_for_bit(gpu):
    """aspec_adamw_step_segments over three gradient tensors (the last of odd size) against
    aspec_adamw_step over the same gradients gathered into one buffer, through the C ABI: master
    weights, moments, bf16 parameters and the norm are bitwise equal after each of three steps
    (the second one non-finite, hence skipped)."""
    import ctypes

    from aspec_amd import _lib

    lib = _lib.load()
    sizes = [8000, 296, 5]
    n = sum(sizes)
    g = torch.Generator(device=gpu).manual_seed(21)
    p0 = torch.randn(n, device=gpu, generator=g).to(torch.bfloat16)
    size = ctypes.c_size_t()
    _lib.call("aspec_adamw_workspace_bytes", ctypes.byref(size))

    def fresh():
        return {"flat": p0.clone(), "master": p0.float(), "m": torch.zeros(n, device=gpu),
                "v": torch.zeros(n, device=gpu),
                "state": torch.zeros(lib.aspec_adamw_state_bytes(), dtype=torch.uint8, device=gpu),
                "ws": torch.empty(size.value, dtype=torch.uint8, device=gpu)}

    seg, flat = fresh(), fresh()
    numel = (ctypes.c_int64 * 3)(*sizes)
    stream = _lib.stream_handle(torch.device(gpu))
    for step in range(3):
        parts = [torch.randn(k, device=gpu, generator=g).to(torch.bfloat16) for k in sizes]
        if step == 1:
            parts[2][4] = float("inf")
        gathered = torch.cat(parts)
        hyper = (1e-2, 0.05, 0.9, 0.999, 1e-8, 1.0)
        ptrs = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in parts])
        _lib.call("aspec_adamw_step_segments", _lib.ptr(seg["flat"]), _lib.ptr(seg["master"]),
                  _lib.ptr(seg["m"]), _lib.ptr(seg["v"]), ptrs, numel, 3, *hyper,
                  _lib.ptr(seg["state"]), _lib.ptr(seg["ws"]), stream)
        _lib.call("aspec_adamw_step", _lib.ptr(flat["flat"]), _lib.ptr(flat["master"]),
                  _lib.ptr(flat["m"]), _lib.ptr(flat["v"]), _lib.ptr(gathered), n, *hyper,
                  _lib.ptr(flat["state"]), _lib.ptr(flat["ws"]), stream)
        torch.cuda.synchronize()
        for key in ("flat", "master", "m", "v"):
            assert torch.equal(seg[key], flat[key]), (step, key)
        assert torch.equal(seg["state"][:40], flat["state"][:40]), step
        assert seg["state"][24:28].view(torch.float32).isfinite().item() == (step != 1)
    with pytest.raises(ValueError, match="multiple of 8"):
        bad = (ctypes.c_int64 * 3)(7, 289, 5)
        _lib.call("aspec_adamw_step_segments", _lib.ptr(seg["flat"]), _lib.ptr(seg["master"]),
                  _lib.ptr(seg["m"]), _lib.ptr(seg["v"]), ptrs, bad, 3, *hyper,
                  _lib.ptr(seg["state"]), _lib.ptr(seg["ws"]), stream)


def _small_model(gpu, seed=0, draft_vocab=300):
    return DSparkDraftLayerModel(hidden=256, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=700,
                                 draft_vocab=draft_vocab, max_positions=512, device=gpu, seed=seed)


def test_layer_forward_and_gradients_match_oracle(gpu):
    model = _small_model(gpu)
    w = W.from_layout("small", [150, 106], np.array([0, 40, 96, 150, 190]), np.array([0, 0, 0, 1, 1]), 16)
    batch = layer_batch(model, w, seed=5)
    hidden = model(batch["target_hidden"], batch["draft_input_ids"], batch["context_positions"],
                   batch["draft_positions"], batch["metadata"])
    G = torch.randn(hidden.shape, device=gpu, generator=torch.Generator(device=gpu).manual_seed(9))
    hidden.backward(G.to(hidden.dtype))
    names = [n for n, p in model.named_parameters()]
    P = {n: torch.tensor(_np(p), requires_grad=p.requires_grad) for n, p in model.named_parameters()}
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length)
    visible = M.endpoints_to_dense(ends, w.num_keys)
    ref = ol.layer_forward(P, _np(batch["target_hidden"]), batch["draft_input_ids"].cpu().numpy(),
                           batch["context_positions"].cpu().numpy(), batch["draft_positions"].cpu().numpy(),
                           visible, _np(model.rope_cos), _np(model.rope_sin), model.eps)
    (ref * torch.as_tensor(_np(G.to(hidden.dtype)))).sum().backward()
    # Measured: hidden rel-L2 5.7e-3 (max error 0.9% of the largest value), parameter gradients
    # rel-L2 5.6e-3 .. 8.4e-3 (max error <= 1.1%); bars at about twice that.
    _close("layer hidden", _np(hidden), ref.detach().numpy(), 1.2e-2, 2e-2)
    for n, p in model.named_parameters():
        if not p.requires_grad:
            continue
        _close(f"grad {n}", _np(p.grad), P[n].grad.numpy(), 1.8e-2, 2.5e-2)
    assert len(names) == len(P)


@pytest.mark.parametrize("draft_vocab", [304, 300])
def test_layer_step_loss_and_gradients_match_oracle(gpu, draft_vocab):
    """The step's loss, every parameter gradient and the pre-clip gradient norm against the fp64
    oracle (layer oracle + CE/L1 oracle gradients pushed back through the frozen head). A draft
    vocabulary of 304 runs the fused vocabulary-GEMM + loss + dlogits pass, 300 (not a multiple
    of 8) the logits-then-loss path."""
    model = _small_model(gpu, seed=1, draft_vocab=draft_vocab)
    opt = FusedBF16Optimizer(model, lr=1e-3, total_steps=100, warmup_ratio=0.0)
    w = W.from_layout("small", [150, 106], np.array([0, 40, 96, 150, 190]), np.array([0, 0, 0, 1, 1]), 16)
    batch = layer_batch(model, w, seed=6)
    params_before = {n: _np(p) for n, p in model.named_parameters()}
    seen = {}  # the gradients the optimizer step consumes (it leaves every grad None)
    step = opt.step

    def keep_and_step(closure=None):
        seen.update({n: _np(p.grad) for n, p in model.named_parameters() if p.requires_grad})
        return step(closure)

    opt.step = keep_and_step
    loss, norm = dspark_layer_step(model, opt, batch)
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length)
    visible = M.endpoints_to_dense(ends, w.num_keys)
    P = {n: torch.tensor(v, requires_grad=p.requires_grad)
         for (n, v), p in zip(params_before.items(), model.parameters())}
    hidden_t = ol.layer_forward(P, _np(batch["target_hidden"]), batch["draft_input_ids"].cpu().numpy(),
                                batch["context_positions"].cpu().numpy(),
                                batch["draft_positions"].cpu().numpy(), visible, _np(model.rope_cos),
                                _np(model.rope_sin), model.eps)
    hidden = hidden_t.detach().numpy()
    head = params_before["lm_head"]
    logits = hidden @ head.T
    teacher = (_np(batch["teacher_hidden"]).reshape(-1, head.shape[1]) @ head.T)
    t = batch["targets"]
    tgt = t.target_ids.reshape(-1).cpu().numpy()
    tidx = t.teacher_index.reshape(-1).cpu().numpy()
    wts = t.weights.reshape(-1).cpu().numpy().astype(np.float64)
    y = teacher[np.clip(tidx, 0, None)]
    ce = oloss.cross_entropy(logits, tgt)
    l1 = oloss.l1(logits, y)
    scale = 1.0 / max(wts.sum(), 1e-6)
    ref = (0.1 * (ce * wts).sum() + 0.9 * (l1 * wts).sum()) * scale
    dlogits = (oloss.cross_entropy_grad(logits, tgt, 0.1 * wts * scale)
               + oloss.l1_grad(logits, y, 0.9 * wts * scale))
    (hidden_t * torch.as_tensor(dlogits @ head)).sum().backward()
    ref_norm = np.sqrt(sum((P[n].grad.numpy() ** 2).sum() for n in P if P[n].requires_grad))
    print(f"layer step loss: got={float(loss):.6f} oracle={ref:.6f} grad_norm={float(norm):.5f} "
          f"oracle={ref_norm:.5f}")
    assert float(loss) == pytest.approx(ref, rel=2e-3)
    assert float(norm) == pytest.approx(ref_norm, rel=1e-2)
    # Measured: parameter gradients rel-L2 1.3e-2 .. 3.9e-2, max error <= 5.6% of the largest
    # value; bars at about twice that. They are looser than the layer test's because the L1 term
    # (weight 0.9) has the gradient p (sign(p - q) - sum p sign(p - q)): wherever p ~ q, the bf16
    # logits' error flips the sign against the fp64 oracle, and dh = dlogits W sums rows of
    # dlogits that nearly cancel. The loss and the gradient norm stay within 0.1% / 0.3%.
    bad = []
    for n, p in model.named_parameters():
        if p.requires_grad:
            try:
                _close(f"grad {n}", seen[n], P[n].grad.numpy(), 8e-2, 1.2e-1)
            except AssertionError:
                bad.append(n)
    assert not bad, bad
    assert opt.optimizer_steps() == 1
    moved = [n for n, p in model.named_parameters() if p.requires_grad
             and not np.array_equal(_np(p), params_before[n])]
    assert "q_proj" in moved and "down_proj" in moved


def test_config5_full_geometry_steps(gpu):
    model = DSparkDraftLayerModel(device=gpu)
    opt = FusedBF16Optimizer(model, lr=1e-4, total_steps=1000, warmup_ratio=0.0)
    batch = layer_batch(model, W.config5(), seed=0)
    q0 = model.q_proj.detach().clone()
    losses = []
    for _ in range(3):
        loss, norm = dspark_layer_step(model, opt, batch)
        losses.append(float(loss))
        assert np.isfinite(float(norm))
    print(f"config5 losses: {losses}")
    assert all(np.isfinite(losses))
    assert opt.optimizer_steps() == 3
    assert not torch.equal(q0, model.q_proj.detach())


def test_config5_full_geometry_layer_rows_and_gradients_match_oracle(gpu):
    """At the full Qwen3-8B geometry of config 5 (H = 4096, GQA 32/8, FFN 12288, 3 documents of
    4096 context tokens, 507 anchors x 16): the layer's final-normed hidden states on ~50 sampled
    query rows (every document, first and last rows, every block offset), and every parameter
    gradient for an upstream gradient carried by those rows only, against the fp32 row-restricted
    layer oracle (keys and values of every token; pinned to the dense oracle on the CPU)."""
    torch.manual_seed(0)
    model = DSparkDraftLayerModel(device=gpu)
    w = W.config5()
    batch = layer_batch(model, w, seed=2)
    hidden = model(batch["target_hidden"], batch["draft_input_ids"], batch["context_positions"],
                   batch["draft_positions"], batch["metadata"])
    H = hidden.shape[-1]
    nq = hidden.numel() // H
    rows = np.unique(np.concatenate([np.arange(0, nq, nq // 40), [nq - 1], np.arange(16)]))
    g = torch.zeros(nq, H, device=gpu)
    g_rows = torch.randn(len(rows), H, generator=torch.Generator().manual_seed(7))
    g[torch.as_tensor(rows, device=gpu)] = g_rows.to(gpu)
    hidden.backward(g.reshape(hidden.shape).to(hidden.dtype))

    f32 = lambda t: t.detach().float().cpu()  # noqa: E731
    P = {n: f32(p).requires_grad_(p.requires_grad) for n, p in model.named_parameters()}
    ends = M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                       w.block_size, w.sequence_length)
    vis_rows = M.endpoints_to_dense(ends[:, rows], w.num_keys)
    ref = ol.layer_forward_rows(P, f32(batch["target_hidden"]), batch["draft_input_ids"].cpu(),
                                batch["context_positions"].cpu(), batch["draft_positions"].cpu(),
                                vis_rows, rows, f32(model.rope_cos), f32(model.rope_sin), model.eps,
                                dtype=torch.float32)
    (ref * g_rows.to(hidden.dtype).float()).sum().backward()
    # Measured: hidden rows rel-L2 8.8e-3 (max error 1.0% of the largest value), parameter
    # gradients rel-L2 8.7e-3 .. 1.2e-2 (max error <= 1.4%); bars at about twice that.
    _close("config5 hidden rows", _np(hidden.reshape(nq, H)[torch.as_tensor(rows, device=gpu)]),
           ref.detach().double().numpy(), 1.8e-2, 2.5e-2)
    checked = 0
    for n, p in model.named_parameters():
        if not p.requires_grad or P[n].grad is None:
            continue
        _close(f"config5 grad {n}", _np(p.grad), P[n].grad.double().numpy(), 2.5e-2, 3e-2)
        checked += 1
    assert checked >= 10
