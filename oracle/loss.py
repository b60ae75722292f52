"""Loss oracle in float64 (numpy). TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

L1: sum_v |softmax(x)_v - softmax(y)_v| per row, the objective of `tiled_l1_from_logits`
(aspec/models/ops/tiled_l1.py:176-209) and `compiled_l1_from_logits` (aspec/models/ops/loss.py:84-91).
Its gradient w.r.t. x is p * (sign(p - q) - E_p[sign(p - q)]) (tiled_l1.py:107-127 states the
cancellation-free form of the same quantity).
CE: logsumexp(x) - x[target], `F.cross_entropy(reduction="none")` (aspec/models/dspark.py:568-570),
ignore_index rows give 0.
"""

from __future__ import annotations

import numpy as np


def softmax(x):
    x = np.asarray(x, np.float64)
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)


def l1(x, y):
    return np.abs(softmax(x) - softmax(y)).sum(axis=-1)


def l1_grad(x, y, g):
    p, q = softmax(x), softmax(y)
    sign = np.sign(p - q)
    centered = sign - (p * sign).sum(axis=-1, keepdims=True)
    return p * centered * np.asarray(g, np.float64)[..., None]


def cross_entropy(x, targets, ignore_index=-100):
    x = np.asarray(x, np.float64)
    t = np.asarray(targets, np.int64)
    m = np.max(x, axis=-1)
    lse = m + np.log(np.exp(x - m[..., None]).sum(axis=-1))
    safe = np.where(t == ignore_index, 0, t)
    picked = np.take_along_axis(x, safe[..., None], axis=-1)[..., 0]
    return np.where(t == ignore_index, 0.0, lse - picked)


def cross_entropy_grad(x, targets, g, ignore_index=-100):
    p = softmax(x)
    t = np.asarray(targets, np.int64)
    onehot = np.zeros_like(p)
    valid = t != ignore_index
    np.put_along_axis(onehot, np.where(valid, t, 0)[..., None], 1.0, axis=-1)
    grad = (p - onehot) * np.asarray(g, np.float64)[..., None]
    return np.where(valid[..., None], grad, 0.0)
