"""Q/K RMSNorm + RoPE oracle in float64 (numpy). TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.

Restates `_prepare_dflash_qk` (aspec/models/draft/dflash.py:296-327) with `_dflash_rms_norm`
(dflash.py:280-293) and `_rotate_half` (dflash.py:248-251), per head row of width D:
    n = x / sqrt(mean(x^2) + eps),  a = n * w,
    out = a * cos[pos] + rotate_half(a) * sin[pos],  rotate_half(a) = (-a[D/2:], a[:D/2]).
Keys are the context keys followed by the draft keys of each batch row (dflash.py:316). The
reference's fused kernel evaluates this in fp32 and rounds once
(aspec/kernels/cutedsl/dspark_qk_norm_rope.py:10); here everything stays float64 and the test
compares against it with the reference's tolerances (tests/test_dspark_qk_cutedsl.py:238-309).

The backward is the transpose of the same three steps:
    da = g * cos + rotate_half^T(g * sin),  rotate_half^T(v) = (v[D/2:], -v[:D/2]),
    dw = sum over rows of da * n,  dn = da * w,  dx = (dn - n * mean(dn * n)) / sqrt(mean(x^2) + eps).
"""

from __future__ import annotations

import numpy as np


def rotate_half(a):
    h = a.shape[-1] // 2
    return np.concatenate([-a[..., h:], a[..., :h]], axis=-1)


def rotate_half_t(v):
    """Transpose of rotate_half: <rotate_half(a), v> == <a, rotate_half_t(v)>."""
    h = v.shape[-1] // 2
    return np.concatenate([v[..., h:], -v[..., :h]], axis=-1)


def norm_rope(x, w, cos, sin, positions, eps):
    """x [..., tokens, heads, D] float64, positions [..., tokens] -> (out, rstd [..., tokens, heads])."""
    x = np.asarray(x, np.float64)
    rstd = 1.0 / np.sqrt((x * x).mean(-1) + eps)
    a = x * rstd[..., None] * np.asarray(w, np.float64)
    c = np.asarray(cos, np.float64)[positions][..., None, :]
    s = np.asarray(sin, np.float64)[positions][..., None, :]
    return a * c + rotate_half(a) * s, rstd


def norm_rope_grad(x, w, cos, sin, positions, eps, g):
    """Gradients (dx, dw) of sum(g * norm_rope(x)) for one tensor (dw summed over all rows)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    g = np.asarray(g, np.float64)
    rstd = 1.0 / np.sqrt((x * x).mean(-1) + eps)
    n = x * rstd[..., None]
    c = np.asarray(cos, np.float64)[positions][..., None, :]
    s = np.asarray(sin, np.float64)[positions][..., None, :]
    da = g * c + rotate_half_t(g * s)
    dw = (da * n).reshape(-1, x.shape[-1]).sum(0)
    dn = da * w
    dx = rstd[..., None] * (dn - n * (dn * n).mean(-1, keepdims=True))
    return dx, dw


def prepare_qk(query, context_key, draft_key, wq, wk, cos, sin, pos_q, pos_ctx, pos_draft, eps):
    """query [B, Ld, Hq, D], context_key [B, Lc, Hkv, D], draft_key [B, Ld, Hkv, D] ->
    (q [B, Ld, Hq, D], k [B, Lc + Ld, Hkv, D], rstd_q, rstd_k)."""
    q, rq = norm_rope(query, wq, cos, sin, pos_q, eps)
    kc, rc = norm_rope(context_key, wk, cos, sin, pos_ctx, eps)
    kd, rd = norm_rope(draft_key, wk, cos, sin, pos_draft, eps)
    return q, np.concatenate([kc, kd], axis=1), rq, np.concatenate([rc, rd], axis=1)


def prepare_qk_grad(query, context_key, draft_key, wq, wk, cos, sin, pos_q, pos_ctx, pos_draft,
                    eps, grad_q, grad_k):
    """(dquery, dcontext_key, ddraft_key, dwq, dwk) for upstream grad_q [B, Ld, Hq, D] and
    grad_k [B, Lc + Ld, Hkv, D]."""
    lc = np.asarray(context_key).shape[1]
    dq, dwq = norm_rope_grad(query, wq, cos, sin, pos_q, eps, grad_q)
    dc, dwc = norm_rope_grad(context_key, wk, cos, sin, pos_ctx, eps, np.asarray(grad_k)[:, :lc])
    dd, dwd = norm_rope_grad(draft_key, wk, cos, sin, pos_draft, eps, np.asarray(grad_k)[:, lc:])
    return dq, dc, dd, dwq, dwc + dwd
