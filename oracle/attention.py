"""Math-path attention oracle (CPU torch, fp32/fp64). TEST INFRASTRUCTURE ONLY -- see
oracle/__init__.py.

Restates `_expand_kv_heads` + `_math_partial` + `_apply_block_keep`
(aspec/models/ops/direct_cp.py:428-477): dense scores, masked to MASK_VALUE, logsumexp, softmax,
P.V; rows without a visible key get O = 0 and LSE = MASK_VALUE. Gradients come from autograd, as
in the reference's math backend. Work is chunked over KV-head groups, which is mathematically
identical and bounds the [heads, Nq, K] score tensor.
"""

from __future__ import annotations

import numpy as np
import torch

MASK_VALUE = -1.0e30  # aspec/models/ops/direct_cp.py:20


def _group_forward(q, k, v, visible, scale, dtype):
    # q [G, Nq, D]; k, v [K, D]: one KV head and its G query heads.
    scores = torch.matmul(q.to(dtype), k.to(dtype).transpose(-1, -2)) * scale
    scores = torch.where(visible[None], scores, torch.full_like(scores, MASK_VALUE))
    lse = torch.logsumexp(scores, dim=-1)
    p = torch.exp(scores - lse.unsqueeze(-1))
    out = torch.matmul(p, v.to(dtype))
    row_keep = visible.any(dim=-1)
    out = torch.where(row_keep[None, :, None], out, torch.zeros_like(out))
    lse = torch.where(row_keep[None], lse, torch.full_like(lse, MASK_VALUE))
    return out, lse


def attention(q, k, v, visible, scale, *, dout=None, dlse=None, dtype=torch.float64):
    """q [Hq, Nq, D], k/v [Hkv, K, D] (any float dtype, CPU), visible [Nq, K] bool.

    Returns (out [Hq,Nq,D], lse [Hq,Nq]) and, when dout is given, (dq, dk, dv) of
    sum(out*dout) + sum(lse*dlse). Everything is computed in `dtype`.
    """
    hq, nq, d = q.shape
    hkv = k.shape[0]
    if hq % hkv:
        raise ValueError("query heads must be divisible by the matching KV head count")
    group = hq // hkv
    visible = torch.as_tensor(np.asarray(visible), dtype=torch.bool)
    out = torch.empty((hq, nq, v.shape[-1]), dtype=dtype)
    lse = torch.empty((hq, nq), dtype=dtype)
    grads = None
    if dout is not None:
        grads = (torch.zeros((hq, nq, d), dtype=dtype), torch.zeros(k.shape, dtype=dtype),
                 torch.zeros(v.shape, dtype=dtype))
    for h in range(hkv):
        sl = slice(h * group, (h + 1) * group)
        qq = q[sl].detach().to(dtype).requires_grad_(dout is not None)
        kk = k[h].detach().to(dtype).requires_grad_(dout is not None)
        vv = v[h].detach().to(dtype).requires_grad_(dout is not None)
        with torch.set_grad_enabled(dout is not None):
            o, l = _group_forward(qq, kk, vv, visible, scale, dtype)
            if dout is not None:
                obj = (o * dout[sl].to(dtype)).sum()
                if dlse is not None:
                    obj = obj + (l * dlse[sl].to(dtype)).sum()
                gq, gk, gv = torch.autograd.grad(obj, (qq, kk, vv))
                grads[0][sl] = gq
                grads[1][h] = gk
                grads[2][h] = gv
        out[sl] = o.detach()
        lse[sl] = l.detach()
    if grads is None:
        return out, lse
    return out, lse, grads


def attention_row_loop(q, k, v, visible, scale, head, row):
    """One output row by an explicit float64 loop over visible keys (independent restatement
    used to pin `attention`): returns (out [D], lse). `visible` is the dense [Nq, K] mask or just
    this row's [K] mask."""
    group = q.shape[0] // k.shape[0]
    kv = head // group
    vis = np.asarray(visible)
    keys = np.nonzero(vis if vis.ndim == 1 else vis[row])[0]
    if keys.size == 0:
        return np.zeros(v.shape[-1]), MASK_VALUE
    qv = q[head, row].double().numpy()
    s = np.array([float(np.dot(qv, k[kv, j].double().numpy())) * scale for j in keys])
    m = s.max()
    w = np.exp(s - m)
    total = w.sum()
    out = sum(w[i] * v[kv, j].double().numpy() for i, j in enumerate(keys)) / total
    return out, m + np.log(total)
