"""Pins the DSpark head-term oracle (oracle/dspark_head.py) against closed forms, hand-stated
answers and finite differences (CPU only)."""

import math

import numpy as np
import pytest

from oracle import dspark_head as odh
from oracle import loss as oloss


def _rng(seed=0):
    return np.random.default_rng(seed)


def test_markov_logits_reduce_to_head_projection_without_w2():
    r = _rng()
    h, w = r.standard_normal((5, 7)), r.standard_normal((11, 7))
    w1, w2 = r.standard_normal((11, 3)), np.zeros((11, 3))
    prev = r.integers(0, 11, 5)
    np.testing.assert_allclose(odh.markov_logits(h, w, prev, w1, w2), h @ w.T, rtol=0, atol=0)


def test_markov_logits_one_hot_embedding_selects_a_w2_column():
    r = _rng(1)
    V, R = 9, 4
    w1 = np.zeros((V, R))
    w1[np.arange(V), np.arange(V) % R] = 1.0  # token v embeds to e_{v mod R}
    w2 = r.standard_normal((V, R))
    prev = np.array([0, 5, 7, 2])
    got = odh.markov_logits(np.zeros((4, 6)), np.zeros((V, 6)), prev, w1, w2)
    for i, p in enumerate(prev):
        np.testing.assert_array_equal(got[i], w2[:, p % R])


def test_markov_gradients_match_finite_differences():
    r = _rng(2)
    rows, H, V, R = 3, 4, 6, 2
    h, w = r.standard_normal((rows, H)), r.standard_normal((V, H))
    w1, w2 = r.standard_normal((V, R)), r.standard_normal((V, R))
    prev = np.array([1, 1, 4])  # a repeated token: its w1 gradient accumulates
    g = r.standard_normal((rows, V))
    dh, dw1, dw2 = odh.markov_logits_grad(h, w, prev, w1, w2, g)
    f = lambda h_, w1_, w2_: float((g * odh.markov_logits(h_, w, prev, w1_, w2_)).sum())
    eps = 1e-6
    for arr, grad, which in ((h, dh, 0), (w1, dw1, 1), (w2, dw2, 2)):
        fd = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            plus, minus = [a.copy() for a in (h, w1, w2)], [a.copy() for a in (h, w1, w2)]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            fd[idx] = (f(*plus) - f(*minus)) / (2 * eps)
        np.testing.assert_allclose(grad, fd, rtol=1e-6, atol=1e-8)


def test_argmax_follows_torch_rules():
    nan, inf = float("nan"), float("inf")
    rows = [
        ([3.0, 1.0, 3.0, 2.0], 0),          # tie: first maximum
        ([1.0, nan, 5.0, nan], 1),          # NaN counts as the largest: first NaN
        ([-inf, -inf, -inf], 0),            # all -inf: index 0
        ([1.0, inf, 2.0, inf], 1),          # first +inf
        ([-inf, -2.0, -inf, -2.0], 1),      # masked entries, tied finite maximum
        ([0.0, -0.0, 0.0], 0),              # signed zeros compare equal
    ]
    for values, expected in rows:
        assert int(odh.argmax(np.array(values))) == expected, values


def test_bce_with_logits_closed_forms():
    z = np.array([0.0, 0.3, 1.0])
    np.testing.assert_allclose(odh.bce_with_logits(np.zeros(3), z), np.full(3, math.log(2.0)))
    # d/dx = sigmoid(x) - z
    x = np.array([-3.0, -0.5, 0.7, 4.0])
    zz = np.array([0.2, 0.9, 0.0, 1.0])
    eps = 1e-6
    fd = (odh.bce_with_logits(x + eps, zz) - odh.bce_with_logits(x - eps, zz)) / (2 * eps)
    np.testing.assert_allclose(fd, 1 / (1 + np.exp(-x)) - zz, rtol=1e-7, atol=1e-9)


def test_acceptance_statistics_hand_computed():
    accept = np.array([[[0.5, 0.5, 0.5], [0.9, 0.1, 0.3]]])
    mask = np.array([[[1, 1, 0], [0, 0, 0]]], np.float64)  # second block entirely masked
    stats = odh.acceptance_statistics(accept, mask)
    # block 0: alpha = [0.5, 0.5, 0] -> tau = 1 + 0.5 + 0.25 + 0 = 1.75; block 1 contributes nothing
    np.testing.assert_allclose(stats, [[0.5, 0.5, 0.0, 1.75], [1.0, 1.0, 0.0, 1.0]])


def test_prediction_terms_compose_the_reference_terms():
    r = _rng(3)
    B, N, K, H, V, R = 1, 2, 3, 5, 7, 2
    h = r.standard_normal((B, N, K, H))
    w = r.standard_normal((V, H))
    th = r.standard_normal((B, N, K, H))
    w1, w2 = r.standard_normal((V, R)), r.standard_normal((V, R))
    tgt = r.integers(0, V, (B, N, K))
    prev = r.integers(0, V, (B, N, K))
    mask = np.ones((B, N, K))
    mask[0, 1, 2] = 0
    weights = mask * np.exp(-np.arange(K) / 4.0)
    cw = r.standard_normal(H + R)
    out = odh.prediction_terms(h, tgt, prev, w, th, mask, weights, w1=w1, w2=w2, conf_w=cw, conf_b=0.1,
                               conf_alpha=1.0)
    logits = odh.markov_logits(h.reshape(-1, H), w, prev.reshape(-1), w1, w2)
    teacher = th.reshape(-1, H) @ w.T
    ce = oloss.cross_entropy(logits, tgt.reshape(-1)).reshape(B, N, K)
    l1 = oloss.l1(logits, teacher).reshape(B, N, K)
    assert out[0] == pytest.approx((ce * weights).sum(), rel=1e-12)
    assert out[1] == pytest.approx((l1 * weights).sum(), rel=1e-12)
    np.testing.assert_allclose(out[3], (ce * mask).sum((0, 1)), rtol=1e-12)
    assert out[5].shape == (2, K + 1)


def test_prediction_terms_conf_num_and_position_correct_hand_computed():
    """One batch, two blocks of three positions, V = H = 3, W = I (logits = h). By hand:
    - argmax of the rows: block 0 -> [0, 1, 2], block 1 -> [2, 2, 0]; targets [0, 0, 2] and
      [2, 1, 0]; eval mask [1, 1, 1] and [1, 1, 0], so the correct-and-evaluated counts per
      position are [1 + 1, 0 + 0, 1 + 0] = [2, 0, 1];
    - the teacher equals the draft on positions 0 and 1 (L1 = 0, accept = 1) and is a far one-hot
      elsewhere on position 2 (L1 = 2 up to e^-60, accept = 0);
    - the confidence head reads [h | w1[prev]] with weight (0, 0, 0 | 1, 0) and bias 0.5, and
      w1[t] = (t, 0), so its logit is prev + 0.5; BCE(x, 1) = log(1 + e^-x), BCE(x, 0) =
      log(1 + e^x); conf_num = sum of weights x BCE."""
    big = 60.0
    h = np.array([[[[big, 0, 0], [0, big, 0], [0, 0, big]],
                   [[0, 1, big], [0, 0, big], [big, 0, 0]]]], np.float64)
    teacher = h.copy()
    teacher[0, 0, 2] = [big, 0, 0]
    teacher[0, 1, 2] = [0, big, 0]
    w = np.eye(3)
    tgt = np.array([[[0, 0, 2], [2, 1, 0]]])
    prev = np.array([[[1, 2, 0], [0, 1, 2]]])
    mask = np.array([[[1.0, 1.0, 1.0], [1.0, 1.0, 0.0]]])
    weights = mask * np.array([1.0, 0.5, 0.25])
    w1 = np.array([[0.0, 0.0], [1.0, 0.0], [2.0, 0.0]])
    w2 = np.zeros((3, 2))
    cw = np.array([0.0, 0.0, 0.0, 1.0, 0.0])
    out = odh.prediction_terms(h, tgt, prev, w, teacher, mask, weights, w1=w1, w2=w2, conf_w=cw,
                               conf_b=0.5, conf_alpha=1.0)
    np.testing.assert_array_equal(out[4], [2.0, 0.0, 1.0])
    x = prev + 0.5
    accept = np.array([[[1, 1, 0], [1, 1, 0]]], np.float64)
    bce = np.where(accept == 1, np.log1p(np.exp(-x)), np.log1p(np.exp(x)))
    assert out[2] == pytest.approx(float((bce * weights).sum()), rel=1e-12, abs=1e-12)
    # without the Markov features the logit is the bias alone
    out_plain = odh.prediction_terms(h, tgt, prev, w, teacher, mask, weights, w1=w1, w2=w2,
                                     conf_w=cw[:3], conf_b=0.5, conf_alpha=1.0, conf_with_markov=False)
    bce0 = np.where(accept == 1, math.log1p(math.exp(-0.5)), math.log1p(math.exp(0.5)))
    assert out_plain[2] == pytest.approx(float((bce0 * weights).sum()), rel=1e-12)
    # the acceptance totals see alpha = accept * mask: per position [2, 2, 0] and tau = 1 + 1 + 1
    # for both blocks (the cumulative product stops at position 2)
    np.testing.assert_allclose(out[5], [[2.0, 2.0, 0.0, 6.0], [2.0, 2.0, 1.0, 2.0]], atol=1e-12)


def test_prediction_terms_teacher_logits_equal_projected_teacher():
    r = _rng(9)
    B, N, K, H, V = 1, 2, 3, 4, 6
    h, th = r.standard_normal((B, N, K, H)), r.standard_normal((B, N, K, H))
    w = r.standard_normal((V, H))
    tgt, prev = r.integers(0, V, (B, N, K)), r.integers(0, V, (B, N, K))
    mask = np.ones((B, N, K))
    a = odh.prediction_terms(h, tgt, prev, w, th, mask, mask)
    b = odh.prediction_terms(h, tgt, prev, w, None, mask, mask, teacher_logits=th.reshape(-1, H) @ w.T)
    for x, y in zip(a, b):
        np.testing.assert_allclose(x, y, rtol=1e-12)
