"""Pins of the sampled-L1 oracle (oracle/sampling.py), CPU only.

* the reference's own known answers for the joint filter (tests/test_dspark_l1_sampling.py:56-67);
* agreement with a second, independent restatement written as the reference test's scalar
  loops (tests/test_dspark_l1_sampling.py:34-51: Python sort by (-value, index), a running sum
  compared with top_p) on the reference test's sampling cases and random rows;
* closed forms: a temperature alone is softmax(x / T); top_k = 1 and a tiny top_p keep the first
  maximum; inactive filters give the plain softmax; identical rows give zero L1 and gradient;
* the L1 gradient against central finite differences (fp64, away from the support's boundary).
"""

import math

import numpy as np
import pytest
from scipy.special import softmax

from oracle import sampling as S

DEFAULT = (1.0, 1.0, -1)
TARGET = (0.8, 0.85, 5)
DRAFT = (1.2, 0.9, 7)
CASES = [DEFAULT, (0.4, 1.0, -1), (1.0, 1.0, 1), (1.0, 1.0, 100), (1.0, 0.5, 10**30), (1.0, 0.5, -1),
         TARGET, DRAFT]


def scalar_probs(row, sampling):
    """The reference test's independent oracle, as scalar Python (one row)."""
    temperature, top_p, top_k = sampling
    maximum = max(row)
    values = [math.exp((v - maximum) / temperature) for v in row]
    total = sum(values)
    p = [v / total for v in values]
    order = sorted(range(len(row)), key=lambda i: (-row[i], i))
    keep = [False] * len(row)
    cumulative = 0.0
    for rank, i in enumerate(order):
        keep[i] = (top_k == -1 or rank < top_k) and (top_p == 1.0 or cumulative <= top_p)
        cumulative += p[i]
    z = [(v - maximum) / temperature if k else -math.inf for v, k in zip(row, keep)]
    zmax = max(z)
    e = [math.exp(v - zmax) if v != -math.inf else 0.0 for v in z]
    s = sum(e)
    return [v / s for v in e]


def test_reference_known_answers():
    x = np.log(np.array([[0.4, 0.3, 0.2, 0.1]], dtype=np.float32))
    np.testing.assert_allclose(S.probs(x, (1.0, 0.5, 2)), [[4 / 7, 3 / 7, 0.0, 0.0]], atol=1e-6)
    np.testing.assert_allclose(S.probs(np.zeros((1, 4)), (1.0, 0.5, -1)), [[1 / 3, 1 / 3, 1 / 3, 0.0]],
                               atol=1e-12)
    tiny = S.probs(np.array([[1e30, 0.0, -1e30]]), (1e-10, 0.1, 1))
    np.testing.assert_allclose(tiny, [[1.0, 0.0, 0.0]], atol=0)


@pytest.mark.parametrize("sampling", CASES)
def test_matches_scalar_restatement(sampling):
    rng = np.random.default_rng(7)
    rows = [[3.0, -2.0, 1.0, 0.0], [0.0, 0.0, 0.0, 0.0]]
    got = S.probs(np.array(rows), sampling)
    want = np.array([scalar_probs(r, sampling) for r in rows])
    np.testing.assert_allclose(got, want, atol=1e-7)
    x = rng.standard_normal((8, 37)) * 2.0
    got = S.probs(x, sampling, np.float64)
    want = np.array([scalar_probs(list(r), sampling) for r in x])
    np.testing.assert_allclose(got, want, atol=1e-12)
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=1e-12)


def test_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 50))
    x[0, [3, 17]] = x[0].max() + 1.0  # a tied maximum: the first index wins
    np.testing.assert_allclose(S.probs(x, (0.37, 1.0, -1), np.float64), softmax(x / 0.37, axis=-1),
                               atol=1e-12)
    for sampling in ((1.0, 1.0, 1), (1.0, 1e-9, -1), (2.0, 1e-9, 3)):
        p = S.probs(x, sampling)
        onehot = np.zeros_like(p)
        onehot[np.arange(6), np.argmax(x, axis=-1)] = 1.0
        np.testing.assert_array_equal(p, onehot)
    for sampling in ((1.0, 1.0, -1), (1.0, 1.0, 50), (1.0, 1.0, 10**9)):
        np.testing.assert_allclose(S.probs(x, sampling), softmax(x, axis=-1), atol=1e-7)
    # the top_p support is the shortest prefix of the order whose preceding mass stays <= top_p
    for top_p in (0.3, 0.6, 0.95):
        keep = S.support(x, (1.0, top_p, -1), np.float64)
        p = softmax(x, axis=-1)
        for r in range(6):
            order = np.argsort(-x[r], kind="stable")
            before = np.concatenate([[0.0], np.cumsum(p[r][order])[:-1]])
            np.testing.assert_array_equal(keep[r][order], before <= np.float32(top_p))
    # nested supports
    a = S.support(x, (1.0, 0.4, -1))
    b = S.support(x, (1.0, 0.8, -1))
    assert not (a & ~b).any()


@pytest.mark.parametrize("target,draft", [(DEFAULT, DRAFT), (TARGET, DEFAULT), (TARGET, DRAFT),
                                          ((1.0, 1.0, -1), (0.5, 1.0, -1))])
def test_identical_rows_and_gradient(target, draft):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5, 23)) * 1.5
    y = rng.standard_normal((5, 23)) * 1.5
    assert np.all(S.sampled_l1(x, x, draft, draft) == 0.0)
    assert np.all(S.sampled_l1_grad(x, x, np.ones(5), draft, draft) == 0.0)
    g = rng.random(5)
    grad = S.sampled_l1_grad(x, y, g, target, draft, np.float64)
    eps = 1e-6
    fd = np.zeros_like(x)
    for r in range(5):
        for v in range(23):
            xp, xm = x.copy(), x.copy()
            xp[r, v] += eps
            xm[r, v] -= eps
            # the support must not move under the step (the boundary is away from every token)
            assert np.array_equal(S.support(xp, draft, np.float64), S.support(xm, draft, np.float64))
            fd[r, v] = g[r] * (S.sampled_l1(xp, y, target, draft, np.float64)[r]
                               - S.sampled_l1(xm, y, target, draft, np.float64)[r]) / (2 * eps)
    np.testing.assert_allclose(grad, fd, atol=1e-7, rtol=1e-5)


def test_sampling_logits_gradient_finite_differences():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 11))
    w = rng.standard_normal((3, 11))
    for sampling in ((1.0, 0.7, 4), (0.6, 0.9, -1)):
        keep = S.support(x, sampling)

        def f(z):
            out = S.scaled_values(z, sampling, np.float64)
            return (np.where(keep, out, 0.0) * w).sum()

        grad = S.sampling_logits_grad(x, w, sampling)
        eps = 1e-6
        fd = np.zeros_like(x)
        for r in range(3):
            for v in range(11):
                xp, xm = x.copy(), x.copy()
                xp[r, v] += eps
                xm[r, v] -= eps
                fd[r, v] = (f(xp) - f(xm)) / (2 * eps)
        np.testing.assert_allclose(grad, fd, atol=1e-6, rtol=1e-4)
