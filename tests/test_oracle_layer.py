"""Pins the one-layer step oracle (oracle/layer.py) against closed forms and finite differences
(CPU only)."""

import math

import numpy as np
import pytest
import torch

from oracle import layer as ol


def _rng(seed=0):
    return np.random.default_rng(seed)


def test_rms_norm_constant_rows_normalise_to_the_weight():
    w = np.array([0.5, -2.0, 3.0, 1.0])
    for c in (-3.0, 0.25, 7.0):
        _, out = ol.rms_norm(np.full((2, 4), c), w, eps=0.0)
        np.testing.assert_allclose(out, np.sign(c) * np.broadcast_to(w, (2, 4)), rtol=1e-14)


def test_rms_norm_residual_is_added_first():
    r = _rng(1)
    x, res, w = r.standard_normal((3, 8)), r.standard_normal((3, 8)), r.standard_normal(8)
    y, out = ol.rms_norm(x, w, 1e-6, residual=res)
    np.testing.assert_allclose(y, x + res)
    np.testing.assert_allclose(out, ol.rms_norm(x + res, w, 1e-6)[1])


def test_rms_norm_gradients_match_finite_differences():
    r = _rng(2)
    y, w, g, extra = (r.standard_normal((3, 6)), r.standard_normal(6), r.standard_normal((3, 6)),
                      r.standard_normal((3, 6)))
    eps = 1e-5
    dy, dw = ol.rms_norm_grad(y, w, eps, g, dy_extra=extra)
    f = lambda y_, w_: float((g * ol.rms_norm(y_, w_, eps)[1]).sum() + (extra * y_).sum())
    h = 1e-6
    fd_y = np.zeros_like(y)
    for i in np.ndindex(y.shape):
        a, b = y.copy(), y.copy()
        a[i] += h
        b[i] -= h
        fd_y[i] = (f(a, w) - f(b, w)) / (2 * h)
    fd_w = np.zeros_like(w)
    for i in range(w.size):
        a, b = w.copy(), w.copy()
        a[i] += h
        b[i] -= h
        fd_w[i] = (f(y, a) - f(y, b)) / (2 * h)
    np.testing.assert_allclose(dy, fd_y, rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(dw, fd_w, rtol=1e-6, atol=1e-8)


def test_swiglu_special_values_and_gradient():
    gu = np.array([[0.0, 50.0, -50.0, 2.0, 3.0, 4.0]])
    out = ol.swiglu(gu)
    # silu(0) = 0, silu(50) -> 50, silu(-50) -> 0
    np.testing.assert_allclose(out, [[0.0, 50.0 * 3.0, 0.0]], atol=1e-12)
    r = _rng(3)
    gu = r.standard_normal((2, 8))
    d = r.standard_normal((2, 4))
    grad = ol.swiglu_grad(gu, d)
    h = 1e-6
    fd = np.zeros_like(gu)
    for i in np.ndindex(gu.shape):
        a, b = gu.copy(), gu.copy()
        a[i] += h
        b[i] -= h
        fd[i] = ((d * ol.swiglu(a)).sum() - (d * ol.swiglu(b)).sum()) / (2 * h)
    np.testing.assert_allclose(grad, fd, rtol=1e-6, atol=1e-8)


def test_adamw_first_step_closed_form_and_clip():
    p0 = np.array([1.0, -2.0, 0.5])
    g = np.array([0.1, -0.2, 0.0])
    lr, wd, eps = 1e-2, 0.1, 1e-8
    out, norms, t = ol.adamw_steps(p0, [g], lrs=[lr], weight_decay=wd, eps=eps, max_grad_norm=10.0)
    # fresh state: m_hat = g, v_hat = g^2, so the step is lr * g / (|g| + eps) after the decay
    want = p0 * (1 - lr * wd) - lr * g / (np.abs(g) + eps)
    np.testing.assert_allclose(out[0], want, rtol=1e-12)
    assert norms[0] == pytest.approx(math.sqrt(0.05))
    assert t == 1
    # a clipped gradient takes the same first step direction (the ratio is scale free) ...
    clipped, _, _ = ol.adamw_steps(p0, [g], lrs=[lr], weight_decay=wd, eps=0.0, max_grad_norm=1e-3)
    np.testing.assert_allclose(clipped[0][:2], (p0 * (1 - lr * wd) - lr * np.sign(g))[:2], rtol=1e-12)
    # ... and a non-finite gradient skips the step entirely
    skipped, _, t2 = ol.adamw_steps(p0, [np.array([np.nan, 0.0, 0.0]), g], lrs=[lr, lr])
    np.testing.assert_array_equal(skipped[0], p0)
    assert t2 == 1


def test_adamw_oracle_matches_torch_adamw_with_missing_gradients():
    """Per-parameter activity: a parameter whose grad is None is skipped by torch's AdamW (no decay,
    no moment update) and keeps its own step count for the bias corrections; the clip norm covers
    the parameters that have gradients."""
    r = _rng(3)
    sizes = [5, 3, 4]
    p0 = [r.standard_normal(n) for n in sizes]
    tp = [torch.tensor(x, requires_grad=True) for x in p0]
    opt = torch.optim.AdamW(tp, lr=1e-2, weight_decay=0.1, foreach=False)
    has = [[True, True, True], [True, False, True], [False, True, True], [True, True, False],
           [False, False, True]]
    grads, actives, lrs = [], [], []
    for k, on in enumerate(has):
        gs = [r.standard_normal(n) * 0.4 for n in sizes]
        for x, g, h in zip(tp, gs, on):
            x.grad = torch.tensor(g) if h else None
        torch.nn.utils.clip_grad_norm_([x for x in tp if x.grad is not None], 1.0)
        lr = 1e-2 * (k + 1)
        opt.param_groups[0]["lr"] = lr
        opt.step()
        grads.append(np.concatenate(gs))
        actives.append(np.concatenate([np.full(n, h) for n, h in zip(sizes, on)]))
        lrs.append(lr)
    out, _, t = ol.adamw_steps(np.concatenate(p0), grads, lrs=lrs, weight_decay=0.1,
                               max_grad_norm=1.0, active=actives)
    np.testing.assert_allclose(out[-1], np.concatenate([x.detach().numpy() for x in tp]),
                               rtol=1e-12, atol=1e-14)
    assert t == len(has)
    # a parameter that never had a gradient is untouched
    out2, _, _ = ol.adamw_steps(np.concatenate(p0), grads[:1], lrs=lrs[:1], weight_decay=0.1,
                                active=[np.concatenate([np.zeros(5, bool), np.ones(7, bool)])])
    np.testing.assert_array_equal(out2[0][:5], p0[0])


def test_layer_forward_is_differentiable_and_row_local():
    """The oracle layer runs in fp64 with autograd; a draft query whose only visible keys are its
    own block does not see the context."""
    r = _rng(4)
    H, D, hq, hkv, F, T, nq, V = 16, 8, 2, 1, 32, 6, 4, 20
    params = {
        "embed_tokens": r.standard_normal((V, H)), "context_proj": r.standard_normal((H, 3 * H)) * 0.1,
        "context_norm": np.ones(H), "input_layernorm": np.ones(H), "q_proj": r.standard_normal((hq * D, H)),
        "k_proj": r.standard_normal((hkv * D, H)), "v_proj": r.standard_normal((hkv * D, H)),
        "q_norm": np.ones(D), "k_norm": np.ones(D), "o_proj": r.standard_normal((H, hq * D)) * 0.1,
        "post_attention_layernorm": np.ones(H), "gate_up_proj": r.standard_normal((2 * F, H)) * 0.1,
        "down_proj": r.standard_normal((H, F)) * 0.1, "final_norm": np.ones(H)}
    P = {k: torch.tensor(v, requires_grad=True) for k, v in params.items()}
    th = r.standard_normal((1, T, 3 * H))
    vis = np.zeros((nq, T + nq), bool)
    vis[:, T:] = True  # draft-only visibility
    cos, sin = np.ones((16, D)), np.zeros((16, D))
    out = ol.layer_forward(P, th, [1, 2, 3, 4], np.arange(T), np.arange(nq), vis, cos, sin, 1e-6)
    out.sum().backward()
    assert P["context_proj"].grad is not None
    # keys of the context are masked: the context projection receives no gradient through attention
    assert float(P["context_proj"].grad.abs().max()) == 0.0
    assert float(P["q_proj"].grad.abs().max()) > 0.0


def _layer_params(H, D, hq, hkv, F, V, *, scale=0.1, seed=5):
    r = _rng(seed)
    return {
        "embed_tokens": r.standard_normal((V, H)), "context_proj": r.standard_normal((H, 3 * H)) * scale,
        "context_norm": np.ones(H), "input_layernorm": np.ones(H), "q_proj": r.standard_normal((hq * D, H)),
        "k_proj": r.standard_normal((hkv * D, H)), "v_proj": r.standard_normal((hkv * D, H)),
        "q_norm": np.ones(D), "k_norm": np.ones(D), "o_proj": r.standard_normal((H, hq * D)) * scale,
        "post_attention_layernorm": np.ones(H), "gate_up_proj": r.standard_normal((2 * F, H)) * scale,
        "down_proj": r.standard_normal((H, F)) * scale, "final_norm": np.ones(H)}


def _run_layer(params, th, ids, T, nq, vis, D, eps):
    cos, sin = np.ones((64, D)), np.zeros((64, D))
    out = ol.layer_forward(params, th, ids, np.arange(T), np.arange(nq), vis, cos, sin, eps)
    return out.detach().numpy()


def test_layer_forward_without_attention_and_mlp_is_final_norm_of_the_embedding():
    """o_proj = 0 and down_proj = 0 remove both sublayers: both residual adds leave the embedding
    row as is, so the output is final_norm(embed[id]). Constant embedding rows c give sign(c) * w
    (RMSNorm of a constant row). A missing residual gives 0, a missing final norm gives c."""
    H, D, hq, hkv, F, T, nq, V = 8, 4, 2, 1, 16, 5, 3, 6
    P = _layer_params(H, D, hq, hkv, F, V)
    P["o_proj"][:] = 0.0
    P["down_proj"][:] = 0.0
    consts = np.array([3.0, -0.5, 2.0, -7.0, 1.5, 0.25])
    P["embed_tokens"] = np.repeat(consts[:, None], H, axis=1)
    w = np.linspace(-2.0, 2.0, H)
    P["final_norm"] = w
    vis = _rng(6).random((nq, T + nq)) < 0.5
    vis[:, T:] = True
    ids = [3, 1, 4]
    out = _run_layer(P, _rng(7).standard_normal((1, T, 3 * H)), ids, T, nq, vis, D, 1e-12)
    np.testing.assert_allclose(out, np.sign(consts[ids])[:, None] * w[None], rtol=1e-9, atol=1e-12)


def test_layer_forward_single_visible_key_routes_that_keys_value_row():
    """Each query sees exactly one context key j(r). Its softmax weight is then 1, so the
    attention output of query head h is the value row of key j(r) under KV head h // group.
    One-hot target features and context_proj = sqrt(H) [I | 0 | 0] make the context rows
    ctx[j] = sqrt(H) e_j exactly (their RMS is 1), so v_j = sqrt(H) v_proj[:, j]. With zero
    embedding rows, o_proj = I and down_proj = 0, the output row is RMSNorm of the concatenated
    head outputs. A wrong key, a wrong query-head to KV-head map or a lost residual changes it."""
    H, D, hq, hkv, F, T, nq, V = 8, 2, 4, 2, 16, 6, 4, 3
    P = _layer_params(H, D, hq, hkv, F, V)
    P["embed_tokens"][:] = 0.0
    P["context_proj"] = np.sqrt(H) * np.concatenate([np.eye(H), np.zeros((H, 2 * H))], axis=1)
    M = np.array([[1, -2, 3, 0, 2, -1, 4, 1], [0, 1, -1, 2, 3, 1, -2, 2],
                  [2, 0, 1, -3, 1, 2, 1, -1], [-1, 3, 0, 1, -2, 1, 2, 3]], np.float64)
    P["v_proj"] = M
    P["o_proj"] = np.eye(H)
    P["down_proj"][:] = 0.0
    th = np.zeros((1, T, 3 * H))
    for j in range(T):
        th[0, j, j] = 1.0
    keys = [4, 1, 5, 0]  # the one visible context key of each query row
    vis = np.zeros((nq, T + nq), bool)
    for r, j in enumerate(keys):
        vis[r, j] = True
    eps = 1e-12
    out = _run_layer(P, th, [0, 1, 2, 0], T, nq, vis, D, eps)
    group = hq // hkv
    for r, j in enumerate(keys):
        v = np.sqrt(H) * M[:, j]  # [hkv * D]
        y = np.concatenate([v[(h // group) * D:(h // group + 1) * D] for h in range(hq)])
        want = y / np.sqrt((y * y).mean() + eps)
        np.testing.assert_allclose(out[r], want, rtol=1e-9, atol=1e-12)


def test_layer_forward_swiglu_gates_with_the_first_half():
    """gate_up_proj rows [gate; up]: with the attention removed, constant positive embedding rows
    normalise to ones, so gate = -50 and up = 1 for every unit. silu(-50) * 1 is ~1e-20, so the MLP
    adds nothing and the output is final_norm(ones) = ones; gate and up swapped would add
    silu(1) * -50 * sum(down) per dimension. With gate = 1 and up = 2 instead, the MLP adds
    2 silu(1) (= 2 / (1 + e^-1)) times each down_proj row sum."""
    H, D, hq, hkv, F, T, nq, V = 8, 4, 2, 1, 4, 3, 2, 2
    P = _layer_params(H, D, hq, hkv, F, V)
    P["embed_tokens"][:] = 2.0
    P["o_proj"][:] = 0.0
    down = _rng(8).standard_normal((H, F))
    P["down_proj"] = down
    vis = np.ones((nq, T + nq), bool)
    th = _rng(9).standard_normal((1, T, 3 * H))
    P["gate_up_proj"] = np.concatenate([np.full((F, H), -50.0 / H), np.full((F, H), 1.0 / H)])
    out = _run_layer(P, th, [0, 1], T, nq, vis, D, 1e-12)
    np.testing.assert_allclose(out, np.ones((nq, H)), rtol=1e-12)
    P["gate_up_proj"] = np.concatenate([np.full((F, H), 1.0 / H), np.full((F, H), 2.0 / H)])
    out = _run_layer(P, th, [0, 1], T, nq, vis, D, 1e-12)
    y = 2.0 + 2.0 / (1.0 + math.exp(-1.0)) * down.sum(axis=1)
    want = y / np.sqrt((y * y).mean() + 1e-12)
    np.testing.assert_allclose(out, np.broadcast_to(want, (nq, H)), rtol=1e-12)


def test_layer_forward_rows_equals_the_dense_layer_rows_values_and_gradients():
    """The row-restricted oracle (full-size GPU parity) equals the dense layer oracle on the chosen
    rows, and with an upstream gradient carried by those rows only, every parameter gradient equals
    the dense layer's (the other rows contribute nothing). Random visibility with some empty rows,
    real RoPE tables, non-unit norm weights."""
    r = _rng(11)
    H, D, hq, hkv, F, T, nq, V = 32, 8, 4, 2, 48, 12, 10, 30
    params = _layer_params(H, D, hq, hkv, F, V, scale=0.3, seed=12)
    for name in ("context_norm", "input_layernorm", "q_norm", "k_norm", "post_attention_layernorm",
                 "final_norm"):
        params[name] = 1.0 + 0.2 * r.standard_normal(params[name].shape)
    th = r.standard_normal((1, T, 3 * H))
    ids = r.integers(0, V, nq)
    vis = r.random((nq, T + nq)) < 0.5
    vis[3] = False  # a row without visible keys
    ang = np.outer(np.arange(64), 1.0 / (100.0 ** (np.arange(D // 2) / (D // 2))))
    cos = np.concatenate([np.cos(ang)] * 2, axis=1)
    sin = np.concatenate([np.sin(ang)] * 2, axis=1)
    ctx_pos, draft_pos = np.arange(T), r.integers(0, 40, nq)
    rows = np.array([0, 3, 7, 9])
    g = r.standard_normal((len(rows), H))

    Pd = {k: torch.tensor(v, requires_grad=True) for k, v in params.items()}
    dense = ol.layer_forward(Pd, th, ids, ctx_pos, draft_pos, vis, cos, sin, 1e-6)
    (dense[torch.as_tensor(rows)] * torch.as_tensor(g)).sum().backward()
    Pr = {k: torch.tensor(v, requires_grad=True) for k, v in params.items()}
    sub = ol.layer_forward_rows(Pr, th, ids, ctx_pos, draft_pos, vis[rows], rows, cos, sin, 1e-6)
    (sub * torch.as_tensor(g)).sum().backward()

    np.testing.assert_allclose(sub.detach().numpy(), dense.detach().numpy()[rows], rtol=1e-12, atol=1e-12)
    for name in params:
        a, b = Pr[name].grad, Pd[name].grad
        assert (a is None) == (b is None), name
        if a is not None:
            np.testing.assert_allclose(a.numpy(), b.numpy(), rtol=1e-10, atol=1e-12, err_msg=name)
    assert float(Pd["context_proj"].grad.abs().max()) > 0.0  # the check reaches the key path
