"""CPU restatement of the reference's sampled L1 (test infrastructure: only tests/, smoke() and
bench.py's baseline leg use it; the product never imports it).

Follows aspec/models/ops/loss.py:57-80 (`sampling_logits`) and :83-89 (`compiled_l1_from_logits`):

  scaled = (x - max x) * float32(1 / float32(T))   when T != 1, else x    (fp32, from bf16 x)
  order  = scaled descending, ties by token index (a stable sort)
  remove = (exclusive cumulative mass > top_p) if top_p < 1;  rank >= top_k if 0 < top_k < V
  p      = softmax over the kept tokens;   l1 = sum |p_draft - p_teacher|

The scaled values are computed in fp32 exactly as PyTorch's CUDA path does (division of a
tensor by a Python scalar multiplies by the fp32 reciprocal), so the ties and the order match the
reference's. The masses, softmax, L1 and gradients are fp64; the cumulative mass is compared with
float32(top_p), as torch compares an fp32 tensor with a Python float.

Pinned by tests/test_oracle_sampling.py against the reference's own known answers
(tests/test_dspark_l1_sampling.py:56-67), against a second restatement written as the
reference test's scalar loops (:34-51), against closed forms (temperature only, top_k = 1,
inactive filters, identical rows) and, for the gradient, against finite differences.
"""

from __future__ import annotations

import numpy as np

DEFAULT = (1.0, 1.0, -1)


def scaled_values(x, sampling, dtype=np.float32):
    """[rows, V] values the order is taken over (x: values of bf16 logits). dtype float32 is the
    reference's arithmetic; float64 (x / T exactly) serves analytic checks such as finite
    differences."""
    temperature = sampling[0]
    xs = np.asarray(x, dtype=dtype)
    if temperature != 1.0:
        rcp = dtype(1.0) / dtype(temperature)
        with np.errstate(over="ignore"):
            return (xs - xs.max(axis=-1, keepdims=True)) * rcp
    return xs


def support(x, sampling, dtype=np.float32):
    """Boolean [rows, V] mask of the kept tokens."""
    temperature, top_p, top_k = sampling
    s = scaled_values(x, sampling, dtype).astype(np.float64)
    rows, vocab = s.shape
    keep = np.ones((rows, vocab), dtype=bool)
    if top_p == 1.0 and (top_k == -1 or top_k >= vocab):
        return keep
    order = np.argsort(-s, axis=-1, kind="stable")  # descending, ties by index
    srt = np.take_along_axis(s, order, axis=-1)
    remove = np.zeros_like(srt, dtype=bool)
    if top_p < 1.0:
        # the mass before each token in unnormalised terms (exp(s - max s), exact for tie groups of
        # equal tokens), against top_p times the row's total
        e = np.exp(srt - srt[:, :1])
        before = np.cumsum(e, axis=-1) - e
        remove |= before > float(np.float32(top_p)) * e.sum(axis=-1, keepdims=True)
    if 0 < top_k < vocab:
        remove |= np.arange(vocab)[None, :] >= top_k
    np.put_along_axis(keep, order, ~remove, axis=-1)
    return keep


def top_p_margin(x, sampling, dtype=np.float32):
    """Per row, the distance between top_p and the nearest preceding-mass value of any token,
    relative to the row's mass (inf without a top-p filter): a row within the rounding of its
    exp values (about 1e-7) may keep or drop its boundary token either way."""
    temperature, top_p, top_k = sampling
    s = scaled_values(x, sampling, dtype).astype(np.float64)
    if top_p == 1.0:
        return np.full(s.shape[0], np.inf)
    srt = -np.sort(-s, axis=-1)
    e = np.exp(srt - srt[:, :1])
    total = e.sum(axis=-1, keepdims=True)
    before = np.cumsum(e, axis=-1) - e
    return (np.abs(before - float(np.float32(top_p)) * total) / total).min(axis=-1)


def sampling_logits(x, sampling):
    """The filtered logits: fp32 scaled values, -inf outside the support."""
    if tuple(sampling) == DEFAULT:
        return np.asarray(x, dtype=np.float64)
    s = scaled_values(x, sampling).astype(np.float64)
    return np.where(support(x, sampling), s, -np.inf)


def probs(x, sampling, dtype=np.float32):
    s = scaled_values(x, sampling, dtype).astype(np.float64)
    keep = support(x, sampling, dtype)
    z = np.where(keep, s, -np.inf)
    e = np.exp(z - z.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def sampled_l1(x, y, target_sampling=DEFAULT, draft_sampling=DEFAULT, dtype=np.float32):
    return np.abs(probs(x, draft_sampling, dtype) - probs(y, target_sampling, dtype)).sum(axis=-1)


def sampled_l1_grad(x, y, g, target_sampling=DEFAULT, draft_sampling=DEFAULT, dtype=np.float32):
    """d(sum_r g_r l1_r)/dx: g / T * p * (sign(p - q) - sum p sign(p - q)) on the draft support."""
    p = probs(x, draft_sampling, dtype)
    q = probs(y, target_sampling, dtype)
    sign = np.sign(p - q)
    centered = sign - (p * sign).sum(axis=-1, keepdims=True)
    temperature = draft_sampling[0]
    scale = float(dtype(1.0) / dtype(temperature)) if temperature != 1.0 else 1.0
    return p * centered * np.asarray(g, dtype=np.float64)[:, None] * scale


def sampling_logits_grad(x, grad_out, sampling):
    """d(sum grad_out * sampling_logits(x))/dx: keep * g / T, minus, with a temperature, the kept
    gradient's sum / T shared evenly by the tokens equal to the row max (amax's gradient)."""
    temperature = sampling[0]
    g = np.asarray(grad_out, dtype=np.float64)
    keep = support(x, sampling)
    if temperature == 1.0:
        return np.where(keep, g, 0.0)
    rcp = float(np.float32(1.0) / np.float32(temperature))
    d = np.where(keep, g, 0.0) * rcp
    x64 = np.asarray(x, dtype=np.float64)
    is_max = x64 == x64.max(axis=-1, keepdims=True)
    share = d.sum(axis=-1, keepdims=True) / is_max.sum(axis=-1, keepdims=True)
    return d - np.where(is_max, share, 0.0)
