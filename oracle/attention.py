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


def attention(q, k, v, visible, scale, *, dout=None, dlse=None, dtype=torch.float64, kv_heads=None):
    """q [Hq, Nq, D], k/v [Hkv, K, D] (any float dtype, CPU), visible [Nq, K] bool.

    Returns (out [Hq,Nq,D], lse [Hq,Nq]) and, when dout is given, (dq, dk, dv) of
    sum(out*dout) + sum(lse*dlse). Everything is computed in `dtype`. `kv_heads` restricts the
    work to those KV heads and their query heads (the other rows of every output stay zero).
    """
    hq, nq, d = q.shape
    hkv = k.shape[0]
    if hq % hkv:
        raise ValueError("query heads must be divisible by the matching KV head count")
    group = hq // hkv
    visible = torch.as_tensor(np.asarray(visible), dtype=torch.bool)
    out = torch.zeros((hq, nq, v.shape[-1]), dtype=dtype)
    lse = torch.zeros((hq, nq), dtype=dtype)
    grads = None
    if dout is not None:
        grads = (torch.zeros((hq, nq, d), dtype=dtype), torch.zeros(k.shape, dtype=dtype),
                 torch.zeros(v.shape, dtype=dtype))
    for h in (range(hkv) if kv_heads is None else kv_heads):
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


def _chunk_windows(e):
    """Disjoint ascending key windows [(lo, hi)] covering every interval of the rows of `e`
    ([5, rows] endpoints): the context intervals' span and the draft intervals' span, merged
    when they touch."""
    spans = []
    for b, t in ((1, 2), (3, 4)):
        nonempty = e[t] > e[b]
        if nonempty.any():
            spans.append((int(e[b][nonempty].min()), int(e[t][nonempty].max())))
    spans.sort()
    merged = []
    for lo, hi in spans:
        if merged and lo <= merged[-1][1]:
            merged[-1] = (merged[-1][0], max(merged[-1][1], hi))
        else:
            merged.append((lo, hi))
    return merged


def attention_group_sampled(q, k, v, ends, scale, dout, dlse=None, *, dq_rows=(), key_ranges=(),
                            chunk=512, dtype=torch.float32):
    """One KV group at sizes where the dense [G, Nq, K] scores do not fit: the same math as
    `attention` (direct_cp.py:428-477), streamed over chunks of query rows. Each chunk computes
    scores only over the key windows its rows' intervals span (keys outside every interval of the
    chunk have zero weight in all its rows, so this is exact).

    q, dout [G, Nq, D] (the group's query heads), k, v [K, D], ends [5, Nq] interval endpoints
    (row r sees keys [ends[1], ends[2]) and [ends[3], ends[4])), dlse [G, Nq] or None.
    Returns a dict with out [G, Nq, D] and lse [G, Nq] for every row; dq [G, len(dq_rows), D] for
    the listed rows; and per key range (k0, k1) the exact dk, dv [k1 - k0, D] summed over all
    query rows of the group. Gradients are those of sum(out*dout) + sum(lse*dlse), written out
    as the textbook softmax backward: P = exp(S - lse), delta = rowsum(dout*out) - dlse,
    dS = P (dout V^T - delta), dQ = scale dS K, dK = scale dS^T Q, dV = P^T dout.
    """
    q, k, v, dout = (torch.as_tensor(x).to(dtype) for x in (q, k, v, dout))
    g, nq, d = q.shape
    ends = np.asarray(ends)
    dlse = None if dlse is None else torch.as_tensor(dlse).to(dtype)
    out = torch.zeros((g, nq, v.shape[-1]), dtype=dtype)
    lse = torch.full((g, nq), MASK_VALUE, dtype=dtype)
    dq_rows = np.asarray(dq_rows, np.int64)
    dq = torch.zeros((g, dq_rows.size, d), dtype=dtype)
    dkv = [(torch.zeros((k1 - k0, d), dtype=dtype), torch.zeros((k1 - k0, v.shape[-1]), dtype=dtype))
           for k0, k1 in key_ranges]
    for r0 in range(0, nq, chunk):
        r1 = min(nq, r0 + chunk)
        e = ends[:, r0:r1].astype(np.int64)
        windows = _chunk_windows(e)
        if not windows:
            continue
        cols = torch.cat([torch.arange(lo, hi) for lo, hi in windows])
        et = torch.as_tensor(e)
        vis = (((cols[None] >= et[1, :, None]) & (cols[None] < et[2, :, None]))
               | ((cols[None] >= et[3, :, None]) & (cols[None] < et[4, :, None])))
        row_keep = vis.any(-1)
        kc, vc = k[cols], v[cols]
        s = torch.matmul(q[:, r0:r1], kc.T) * scale
        s.masked_fill_(~vis[None], float("-inf"))
        m = s.amax(-1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = torch.exp(s - m)
        del s
        l = p.sum(-1, keepdim=True)
        p = p / torch.where(l > 0, l, torch.ones_like(l))
        o = torch.matmul(p, vc)
        lr = (m + torch.log(l)).squeeze(-1)
        out[:, r0:r1] = torch.where(row_keep[None, :, None], o, torch.zeros_like(o))
        lse[:, r0:r1] = torch.where(row_keep[None], lr, torch.full_like(lr, MASK_VALUE))
        delta = (dout[:, r0:r1] * out[:, r0:r1]).sum(-1)
        if dlse is not None:
            delta = delta - dlse[:, r0:r1]
        sel = np.nonzero((dq_rows >= r0) & (dq_rows < r1))[0]
        if sel.size:
            local = torch.as_tensor(dq_rows[sel] - r0)
            dp = torch.matmul(dout[:, r0:r1][:, local], vc.T)
            ds = p[:, local] * (dp - delta[:, local, None])
            dq[:, torch.as_tensor(sel)] = torch.matmul(ds, kc) * scale
        for (k0, k1), (dk_r, dv_r) in zip(key_ranges, dkv):
            off = 0
            for lo, hi in windows:
                a, b = max(k0, lo), min(k1, hi)
                if a < b:
                    pt = p[:, :, off + a - lo:off + b - lo]
                    dv_r[a - k0:b - k0] += torch.einsum("gqk,gqd->kd", pt, dout[:, r0:r1])
                    dp = torch.matmul(dout[:, r0:r1], v[a:b].T)
                    ds = pt * (dp - delta[..., None])
                    dk_r[a - k0:b - k0] += torch.einsum("gqk,gqd->kd", ds, q[:, r0:r1]) * scale
                off += hi - lo
    return {"out": out, "lse": lse, "dq": dq, "dkv": dkv}
