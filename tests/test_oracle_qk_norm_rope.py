"""CPU checks pinning the Q/K RMSNorm + RoPE oracle (oracle/qk_norm_rope.py) against closed forms
and finite differences, plus the product wrapper's host-side validation."""

import numpy as np
import pytest
import torch

from oracle import qk_norm_rope as Q


def _angles(rng, rows, d):
    half = rng.standard_normal((rows, d // 2))
    ang = np.concatenate([half, half], axis=-1)  # cat(freqs, freqs), dflash.py:228
    return np.cos(ang), np.sin(ang)


def test_hand_computed_known_answer():
    # D = 4, x = (1, 2, 3, 4), eps = 0, w = 1: mean(x^2) = 7.5; angle pi/2 -> out = rotate_half(a)
    x = np.array([[[1.0, 2.0, 3.0, 4.0]]])
    cos = np.zeros((1, 4))
    sin = np.ones((1, 4))
    out, rstd = Q.norm_rope(x, np.ones(4), cos, sin, np.array([0]), 0.0)
    np.testing.assert_allclose(rstd, [[1 / np.sqrt(7.5)]])
    np.testing.assert_allclose(out[0, 0], np.array([-3.0, -4.0, 1.0, 2.0]) / np.sqrt(7.5))


def test_identity_rotation_is_weighted_rms_norm():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 3, 128))
    w = rng.standard_normal(128)
    out, _ = Q.norm_rope(x, w, np.ones((7, 128)), np.zeros((7, 128)), rng.integers(0, 7, 5), 1e-6)
    expect = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(out, expect, rtol=1e-12)


def test_constant_rows_normalize_to_unit_magnitude():
    x = np.full((2, 1, 128), -3.0)
    out, _ = Q.norm_rope(x, np.ones(128), np.ones((1, 128)), np.zeros((1, 128)), np.zeros(2, int), 0.0)
    np.testing.assert_allclose(out, -1.0, rtol=1e-12)


def test_rotation_preserves_each_pair_norm():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 2, 128))
    cos, sin = _angles(rng, 9, 128)
    pos = rng.integers(0, 9, 6)
    out, rstd = Q.norm_rope(x, np.ones(128), cos, sin, pos, 1e-6)
    a = x * rstd[..., None]
    np.testing.assert_allclose(out[..., :64] ** 2 + out[..., 64:] ** 2, a[..., :64] ** 2 + a[..., 64:] ** 2,
                               rtol=1e-10)


def test_keys_are_context_then_draft_per_batch_row():
    rng = np.random.default_rng(2)
    b, lc, ld, h = 2, 3, 2, 1
    ctx = rng.standard_normal((b, lc, h, 128))
    drf = rng.standard_normal((b, ld, h, 128))
    q = rng.standard_normal((b, ld, 2, 128))
    cos, sin = _angles(rng, 8, 128)
    pq, pc, pd = rng.integers(0, 8, (b, ld)), rng.integers(0, 8, (b, lc)), rng.integers(0, 8, (b, ld))
    _, k, _, rk = Q.prepare_qk(q, ctx, drf, np.ones(128), np.ones(128), cos, sin, pq, pc, pd, 1e-6)
    kc, _ = Q.norm_rope(ctx, np.ones(128), cos, sin, pc, 1e-6)
    kd, _ = Q.norm_rope(drf, np.ones(128), cos, sin, pd, 1e-6)
    np.testing.assert_array_equal(k[:, :lc], kc)
    np.testing.assert_array_equal(k[:, lc:], kd)
    assert k.shape == (b, lc + ld, h, 128) and rk.shape == (b, lc + ld, h)


def test_rotate_half_transpose():
    rng = np.random.default_rng(3)
    a, v = rng.standard_normal(128), rng.standard_normal(128)
    assert np.isclose(np.dot(Q.rotate_half(a), v), np.dot(a, Q.rotate_half_t(v)))


def test_gradients_match_finite_differences():
    rng = np.random.default_rng(4)
    d = 8  # the formulas hold for any even width
    x = rng.standard_normal((2, 3, d))
    w = rng.standard_normal(d)
    cos, sin = _angles(rng, 5, d)
    pos = rng.integers(0, 5, 2)
    g = rng.standard_normal((2, 3, d))
    eps = 1e-3
    dx, dw = Q.norm_rope_grad(x, w, cos, sin, pos, eps, g)

    def f(xx, ww):
        return (Q.norm_rope(xx, ww, cos, sin, pos, eps)[0] * g).sum()

    h = 1e-6
    num_dx = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        e = np.zeros_like(x)
        e[idx] = h
        num_dx[idx] = (f(x + e, w) - f(x - e, w)) / (2 * h)
    num_dw = np.array([(f(x, w + h * np.eye(d)[i]) - f(x, w - h * np.eye(d)[i])) / (2 * h) for i in range(d)])
    np.testing.assert_allclose(dx, num_dx, rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(dw, num_dw, rtol=1e-6, atol=1e-8)


def test_wrapper_validates_on_the_host_before_any_device_work():
    from aspec_amd.dspark_qk_norm_rope import dspark_qk_norm_rope

    q = torch.zeros(1, 3, 2 * 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 5, 128, dtype=torch.bfloat16)
    kd = torch.zeros(1, 3, 128, dtype=torch.bfloat16)
    w = torch.ones(128, dtype=torch.bfloat16)
    cs = torch.ones(1, 1, 8, 128, dtype=torch.bfloat16)
    p3, p5 = torch.zeros(1, 3, dtype=torch.long), torch.zeros(1, 5, dtype=torch.long)
    with pytest.raises(ValueError, match="requires CUDA tensors"):
        dspark_qk_norm_rope(q, k, kd, w, w, 1e-6, cs, cs, p3, p5, p3, 2, 1, 128)
    with pytest.raises(ValueError, match="must be contiguous"):
        dspark_qk_norm_rope(q.transpose(1, 2), k, kd, w, w, 1e-6, cs, cs, p3, p5, p3, 2, 1, 128)
