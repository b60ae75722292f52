"""DSpark head-term oracle in float64 (numpy). TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

Restates the head side of `DSparkModel._prediction_terms` (aspec/models/dspark.py:553-636):
  logits   = h W^T + markov_w2 markov_w1[prev]^T       (dspark.py:560-566; draft/dspark.py:97-114)
  ce, l1   = oracle.loss cross_entropy / l1              (dspark.py:568-570, 596-612)
  accept   = clamp(1 - l1 / 2, 0, 1)                     (dspark.py:613)
  conf     = BCE-with-logits(c . [h | markov_w1[prev]] + b, accept) (dspark.py:615-623)
  argmax   = first NaN, else first maximum, as torch.argmax (dspark.py:625)
  acceptance statistics                                  (aspec/models/ops/acceptance.py:15-30)
Pinned by tests/test_oracle_dspark_head.py: Markov logits reduce to h W^T when w2 = 0 and to a
column of w2 for a one-hot w1 row; argmax against hand-stated indices for ties, NaN, +-inf rows;
acceptance statistics against a hand-computed block; BCE against its value log 2 at 0 and its
closed-form gradient; the Markov gradients against finite differences.
"""

from __future__ import annotations

import numpy as np

from . import loss as oloss


def markov_logits(h, w, prev, w1, w2):
    """h [rows, H] W^T + w1[prev] w2^T, rows x V."""
    h = np.asarray(h, np.float64)
    e = np.asarray(w1, np.float64)[np.asarray(prev, np.int64)]
    return h @ np.asarray(w, np.float64).T + e @ np.asarray(w2, np.float64).T


def markov_logits_grad(h, w, prev, w1, w2, g):
    """(dh, dw1, dw2) of sum(g * markov_logits)."""
    g = np.asarray(g, np.float64)
    prev = np.asarray(prev, np.int64)
    e = np.asarray(w1, np.float64)[prev]
    dh = g @ np.asarray(w, np.float64)
    de = g @ np.asarray(w2, np.float64)
    dw1 = np.zeros(np.shape(w1), np.float64)
    np.add.at(dw1, prev, de)
    dw2 = g.T @ e
    return dh, dw1, dw2


def argmax(x):
    """torch.argmax over the last axis: NaN counts as the largest value (first NaN wins), else
    the first index of the maximum (an all -inf row gives 0). numpy's argmax follows the same
    rules."""
    return np.argmax(np.asarray(x, np.float64), axis=-1)


def bce_with_logits(x, z):
    """max(x, 0) - x z + log(1 + exp(-|x|)) (the stable form of -z log s(x) - (1-z) log(1-s(x)))."""
    x = np.asarray(x, np.float64)
    z = np.asarray(z, np.float64)
    return np.maximum(x, 0.0) - x * z + np.log1p(np.exp(-np.abs(x)))


def acceptance_statistics(accept, mask):
    """[[alpha summed per position..., sum over valid blocks of tau],
        [mask count per position..., valid block count]] with alpha = accept * mask and
    tau = 1 + sum_k prod_{j<=k} alpha_j (aspec/models/ops/acceptance.py:15-30)."""
    mask = np.asarray(mask, np.float64)
    alpha = np.asarray(accept, np.float64) * mask
    valid = (mask != 0).any(axis=-1)
    tau = 1.0 + np.cumprod(alpha, axis=-1).sum(axis=-1)
    num = np.concatenate([alpha.sum(axis=(0, 1)), [(tau * valid).sum()]])
    den = np.concatenate([mask.sum(axis=(0, 1)), [valid.sum()]])
    return np.stack([num, den])


def prediction_terms(h, target_ids, prev_ids, w, teacher_h, eval_mask, weights, *, w1=None, w2=None,
                     conf_w=None, conf_b=0.0, conf_with_markov=True, l1_alpha=1.0, conf_alpha=0.0,
                     prediction_start=0, teacher_logits=None):
    """(ce_num, l1_num, conf_num, position_loss, position_correct, acceptance_totals) for
    h [B, N, K, H] (dspark.py:553-636, unsampled L1 path, teacher = teacher_h W^T, or the
    given teacher_logits rows [B*N*K, V] when teacher_h is None)."""
    h = np.asarray(h, np.float64)
    shape = h.shape[:-1]
    rows = h.reshape(-1, h.shape[-1])
    prev = np.asarray(prev_ids, np.int64).reshape(-1)
    if w1 is not None:
        logits = markov_logits(rows, w, prev, w1, w2)
    else:
        logits = rows @ np.asarray(w, np.float64).T
    t = np.asarray(target_ids, np.int64).reshape(-1)
    weights = np.asarray(weights, np.float64)
    eval_mask = np.asarray(eval_mask, np.float64)
    ce = oloss.cross_entropy(logits, t).reshape(shape)
    ce_num = (ce * weights).sum()
    l1_num = 0.0
    accept = None
    if teacher_h is not None or teacher_logits is not None:
        if teacher_h is not None:
            teacher = np.asarray(teacher_h, np.float64).reshape(-1, h.shape[-1]) @ np.asarray(w, np.float64).T
        else:
            teacher = np.asarray(teacher_logits, np.float64).reshape(logits.shape)
        l1 = oloss.l1(logits, teacher).reshape(shape)
        if l1_alpha > 0:
            l1_num = (l1 * weights).sum()
        accept = np.clip(1.0 - 0.5 * l1, 0.0, 1.0)
    conf_num = 0.0
    if conf_w is not None and conf_alpha > 0:
        feats = rows
        if conf_with_markov:
            feats = np.concatenate([rows, np.asarray(w1, np.float64)[prev]], axis=1)
        pred = (feats @ np.asarray(conf_w, np.float64) + conf_b).reshape(shape)
        conf_num = (bce_with_logits(pred, accept) * weights).sum()
    correct = (argmax(logits).reshape(shape) == np.asarray(target_ids)) & (eval_mask > 0.5)
    position_loss = (ce * eval_mask).sum(axis=(0, 1))
    position_correct = correct.astype(np.float64).sum(axis=(0, 1))
    if accept is not None:
        stats = acceptance_statistics(accept[..., prediction_start:], eval_mask[..., prediction_start:])
        totals = np.pad(stats, ((0, 0), (prediction_start, 0)))
    else:
        totals = np.zeros((2, shape[-1] + 1))
    return ce_num, l1_num, conf_num, position_loss, position_correct, totals
