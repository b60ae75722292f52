"""One-layer DSpark draft step oracle in float64 (CPU torch / numpy). TEST INFRASTRUCTURE ONLY --
see oracle/__init__.py.

  rms_norm      `_dflash_rms_norm` (aspec/models/draft/dflash.py:282-293), residual add first
  swiglu        `DFlashMLP.forward` (dflash.py:967-980): silu(gate) * up
  adamw_steps   `BF16Optimizer.step` (aspec/training/optimizer.py:90-140) with torch's AdamW:
                global-norm clip, non-finite skip, decoupled weight decay, bias correction
  layer_forward the draft layer of `DFlashDecoderLayer.forward` (dflash.py:1015-1062) between
                `extract_context_feature` (dflash.py:1258-1284) and `final_norm` (dflash.py:1471),
                with the Q/K preparation of `_prepare_dflash_qk` (dflash.py:296-327) and masked
                softmax attention over the DSpark visibility (oracle/attention.py).
  layer_forward_rows  the same layer for a subset of query rows: keys and values of every token,
                everything else for the chosen rows only (the layer is row-local except for its
                attention), so a full-size geometry stays affordable on the CPU.
Pinned by tests/test_oracle_layer.py: constant rows normalise to +-w, finite-difference gradients
of RMSNorm and SwiGLU, silu's value at 0 and its limits, AdamW's closed-form first step
(p - lr * g / (|g| + eps) for a fresh state) and its clipping and skip rules, and against
torch.optim.AdamW (float64, clip_grad_norm_) over parameters that miss gradients in some steps;
layer_forward by
zeroed sublayers, single-key routing, gate/up order and a hand-computed residual case;
layer_forward_rows by equality with layer_forward's rows, values and parameter gradients.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import attention as oattn


def rms_norm(x, w, eps, residual=None):
    """(y, out) with y = x + residual (x when residual is None), out = y * rstd * w."""
    x = np.asarray(x, np.float64)
    y = x if residual is None else x + np.asarray(residual, np.float64)
    rstd = 1.0 / np.sqrt((y * y).mean(axis=-1, keepdims=True) + eps)
    return y, y * rstd * np.asarray(w, np.float64)


def rms_norm_grad(y, w, eps, dout, dy_extra=None):
    """(dy, dw) of out = y * rstd(y) * w for upstream dout (plus dy_extra reaching y directly)."""
    y = np.asarray(y, np.float64)
    w = np.asarray(w, np.float64)
    dout = np.asarray(dout, np.float64)
    rstd = 1.0 / np.sqrt((y * y).mean(axis=-1, keepdims=True) + eps)
    n = y * rstd
    g = dout * w
    dy = rstd * (g - n * (g * n).mean(axis=-1, keepdims=True))
    if dy_extra is not None:
        dy = dy + np.asarray(dy_extra, np.float64)
    dw = (dout * n).reshape(-1, y.shape[-1]).sum(axis=0)
    return dy, dw


def _silu(x):
    return x / (1.0 + np.exp(-x))


def swiglu(gu):
    gu = np.asarray(gu, np.float64)
    f = gu.shape[-1] // 2
    return _silu(gu[..., :f]) * gu[..., f:]


def swiglu_grad(gu, dout):
    gu = np.asarray(gu, np.float64)
    dout = np.asarray(dout, np.float64)
    f = gu.shape[-1] // 2
    g, u = gu[..., :f], gu[..., f:]
    s = 1.0 / (1.0 + np.exp(-g))
    return np.concatenate([dout * u * s * (1.0 + g * (1.0 - s)), dout * g * s], axis=-1)


def adamw_steps(p, grads, *, lrs, weight_decay=0.0, betas=(0.9, 0.999), eps=1e-8, max_grad_norm=0.5,
                active=None):
    """Runs BF16Optimizer steps on a flat fp64 parameter vector for a list of gradients (one per
    step) and learning rates; returns (params after each step, norms, steps taken).
    `active` (optional, one boolean vector per step) marks the elements whose parameter has a
    gradient in that step (optimizer.py:99-109): the others add nothing to the norm and are left
    unchanged, and each element counts its own steps for the bias corrections (torch's AdamW keeps
    a step count per parameter)."""
    p = np.asarray(p, np.float64).copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    te = np.zeros(p.shape, np.int64)  # steps in which the element had a gradient
    t = 0
    out, norms = [], []
    for k, (g, lr) in enumerate(zip(grads, lrs)):
        on = np.ones(p.shape, bool) if active is None else np.asarray(active[k], bool)
        g = np.where(on, np.asarray(g, np.float64), 0.0)
        norm = math.sqrt(float((g * g).sum()))
        norms.append(norm)
        if not math.isfinite(norm):
            out.append(p.copy())
            continue
        coef = min(max_grad_norm / (norm + 1e-6), 1.0) if max_grad_norm > 0 else 1.0
        g = g * coef
        t += 1
        te = te + on
        bc1 = 1.0 - betas[0] ** te
        bc2 = 1.0 - betas[1] ** te
        p_new = p * (1.0 - lr * weight_decay)
        m_new = m + (1.0 - betas[0]) * (g - m)
        v_new = betas[1] * v + (1.0 - betas[1]) * g * g
        with np.errstate(divide="ignore", invalid="ignore"):
            p_new = p_new - (lr / bc1) * m_new / (np.sqrt(v_new) / np.sqrt(bc2) + eps)
        p = np.where(on, p_new, p)
        m = np.where(on, m_new, m)
        v = np.where(on, v_new, v)
        out.append(p.copy())
    return out, norms, t


def _t(a):
    return a if isinstance(a, torch.Tensor) else torch.as_tensor(np.asarray(a), dtype=torch.float64)


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def _norm_rope(x, w, cos, sin, pos, eps):
    """x [L, heads, D]: RMSNorm per head row, then RoPE at positions pos (dflash.py:314-327)."""
    a = _rms(x, w, eps)
    c, s = cos[pos][:, None, :], sin[pos][:, None, :]
    return a * c + _rotate_half(a) * s


def layer_forward(params, target_hidden, draft_ids, context_positions, draft_positions, visible,
                  cos, sin, eps):
    """Draft layer in fp64 torch (autograd-capable): params is a dict of fp64 tensors named as
    `aspec_amd.draft_layer.DSparkDraftLayerModel`'s parameters; visible [Nq, T + Nq] bool.
    Returns the final-normed hidden states [Nq, H]."""
    P = {k: _t(v) for k, v in params.items()}
    th = _t(target_hidden).reshape(-1, P["context_proj"].shape[1])
    ctx = _rms(th @ P["context_proj"].T, P["context_norm"], eps)
    draft = P["embed_tokens"][torch.as_tensor(np.asarray(draft_ids)).reshape(-1)]
    x = _rms(draft, P["input_layernorm"], eps)
    hq = P["q_proj"].shape[0] // P["q_norm"].shape[0]
    D = P["q_norm"].shape[0]
    hkv = P["k_proj"].shape[0] // D
    nq, T = x.shape[0], ctx.shape[0]
    q = (x @ P["q_proj"].T).view(nq, hq, D)
    k = torch.cat([ctx @ P["k_proj"].T, x @ P["k_proj"].T], 0).view(T + nq, hkv, D)
    v = torch.cat([ctx @ P["v_proj"].T, x @ P["v_proj"].T], 0).view(T + nq, hkv, D)
    cos2, sin2 = _t(cos).reshape(-1, D), _t(sin).reshape(-1, D)
    pos_q = torch.as_tensor(np.asarray(draft_positions)).reshape(-1)
    pos_k = torch.cat([torch.as_tensor(np.asarray(context_positions)).reshape(-1), pos_q])
    q = _norm_rope(q, P["q_norm"], cos2, sin2, pos_q, eps)
    k = _norm_rope(k, P["k_norm"], cos2, sin2, pos_k, eps)
    vis = torch.as_tensor(np.asarray(visible), dtype=torch.bool)
    group = hq // hkv
    heads = [oattn._group_forward(q[:, h * group:(h + 1) * group].permute(1, 0, 2), k[:, h], v[:, h], vis,
                                  D ** -0.5, torch.float64)[0] for h in range(hkv)]
    attn = torch.cat(heads, 0).permute(1, 0, 2).reshape(nq, hq * D)
    h = draft + attn @ P["o_proj"].T
    x2 = _rms(h, P["post_attention_layernorm"], eps)
    gu = x2 @ P["gate_up_proj"].T
    f = gu.shape[-1] // 2
    h = h + (torch.nn.functional.silu(gu[:, :f]) * gu[:, f:]) @ P["down_proj"].T
    return _rms(h, P["final_norm"], eps)


def layer_forward_rows(params, target_hidden, draft_ids, context_positions, draft_positions,
                       visible_rows, rows, cos, sin, eps, dtype=torch.float64):
    """`layer_forward` restricted to query rows `rows` (int array): keys and values of every context
    and draft token, queries, attention, o_proj, MLP and final norm of the chosen rows only.
    visible_rows [len(rows), T + Nq] bool is the visibility of those rows. Computed in `dtype`;
    params may be tensors that require gradients (autograd flows into every parameter the chosen
    rows depend on). Returns [len(rows), H]."""
    P = {k: (v if isinstance(v, torch.Tensor) else torch.as_tensor(np.asarray(v))).to(dtype)
         for k, v in params.items()}
    th = torch.as_tensor(np.asarray(target_hidden)).to(dtype).reshape(-1, P["context_proj"].shape[1])
    ctx = _rms(th @ P["context_proj"].T, P["context_norm"], eps)
    ids = torch.as_tensor(np.asarray(draft_ids)).reshape(-1)
    draft = P["embed_tokens"][ids]
    x = _rms(draft, P["input_layernorm"], eps)
    D = P["q_norm"].shape[0]
    hq = P["q_proj"].shape[0] // D
    hkv = P["k_proj"].shape[0] // D
    nq, T = x.shape[0], ctx.shape[0]
    rows = torch.as_tensor(np.asarray(rows, dtype=np.int64))
    cos2 = torch.as_tensor(np.asarray(cos)).to(dtype).reshape(-1, D)
    sin2 = torch.as_tensor(np.asarray(sin)).to(dtype).reshape(-1, D)
    pos_q = torch.as_tensor(np.asarray(draft_positions)).reshape(-1)
    pos_k = torch.cat([torch.as_tensor(np.asarray(context_positions)).reshape(-1), pos_q])
    k = torch.cat([ctx @ P["k_proj"].T, x @ P["k_proj"].T], 0).view(T + nq, hkv, D)
    v = torch.cat([ctx @ P["v_proj"].T, x @ P["v_proj"].T], 0).view(T + nq, hkv, D)
    k = _norm_rope(k, P["k_norm"], cos2, sin2, pos_k, eps)
    xr = x[rows]
    q = _norm_rope((xr @ P["q_proj"].T).view(len(rows), hq, D), P["q_norm"], cos2, sin2, pos_q[rows], eps)
    vis = torch.as_tensor(np.asarray(visible_rows), dtype=torch.bool)
    group = hq // hkv
    heads = [oattn._group_forward(q[:, h * group:(h + 1) * group].permute(1, 0, 2), k[:, h], v[:, h], vis,
                                  D ** -0.5, dtype)[0] for h in range(hkv)]
    attn = torch.cat(heads, 0).permute(1, 0, 2).reshape(len(rows), hq * D)
    h = draft[rows] + attn @ P["o_proj"].T
    x2 = _rms(h, P["post_attention_layernorm"], eps)
    gu = x2 @ P["gate_up_proj"].T
    f = gu.shape[-1] // 2
    h = h + (torch.nn.functional.silu(gu[:, :f]) * gu[:, f:]) @ P["down_proj"].T
    return _rms(h, P["final_norm"], eps)
