"""Tiled FP32 softmax-L1 loss on MI355X (aspec/models/ops/tiled_l1.py).

Same contract as `tiled_l1_from_logits` (tiled_l1.py:176-209): per-row
sum_v |softmax(x)_v - softmax(y)_v| in fp32 from bf16 logits, a frozen teacher (optionally an
int64-indexed teacher table), eight fp32 statistics per row kept for the backward (and for an
optional checkpoint replay cache), backward p * (sign - E_p[sign]) in the cancellation-free form.
The HIP forward reads each logit row once; the backward reads x and y once and writes dx once.
Out-of-range teacher indices fail closed: the forward writes NaN rows and a device flag, and the
backward (or, when no backward follows, the forward itself) raises ValueError.
"""

from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from aspec_amd import _lib
from aspec_amd.loss import IndexCheck

STATS = 8


def _forward_stats(logits, target, indices, rows, vocab):
    stats = torch.empty((rows, STATS), dtype=torch.float32, device=logits.device)
    loss = torch.empty(logits.shape[:-1], dtype=torch.float32, device=logits.device)
    flags = torch.zeros(1, dtype=torch.int32, device=logits.device)
    _lib.call("aspec_ce_l1_fwd", _lib.ptr(logits), _lib.ptr(target), _lib.ptr(indices),
              target.shape[0] if indices is not None else rows, None, -100, rows, vocab,
              _lib.ptr(loss), None, _lib.ptr(stats), _lib.ptr(flags),
              _lib.stream_handle(logits.device))
    return stats, loss, flags


class _TiledL1(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, target, indices, replay_cache):
        vocab = logits.shape[-1]
        rows = logits.numel() // vocab
        if replay_cache:
            stats, loss = replay_cache["statistics"]
            if (loss.shape != logits.shape[:-1] or stats.device != logits.device
                    or replay_cache["vocab"] != vocab):
                raise ValueError("L1 checkpoint statistics belong to a different head chunk")
        else:
            stats, loss, flags = _forward_stats(logits, target, indices, rows, vocab)
            ctx.index_check = IndexCheck(flags)
            if not ctx.needs_input_grad[0]:
                ctx.index_check.raise_if_bad()
            if replay_cache is not None:
                replay_cache["statistics"] = stats, loss.detach()
                replay_cache["vocab"] = vocab
        ctx.save_for_backward(logits, target, stats, indices)
        return loss.view_as(loss)

    @staticmethod
    @once_differentiable
    def backward(ctx, gradient):
        logits, target, stats, indices = ctx.saved_tensors
        vocab = logits.shape[-1]
        rows = logits.numel() // vocab
        grad_logits = torch.empty_like(logits)
        g = gradient.to(torch.float32).contiguous()
        _lib.call("aspec_ce_l1_bwd", _lib.ptr(logits), _lib.ptr(target), _lib.ptr(indices),
                  target.shape[0] if indices is not None else rows, None, -100, rows, vocab,
                  _lib.ptr(stats), _lib.ptr(g), None, _lib.ptr(grad_logits),
                  _lib.stream_handle(logits.device))
        # the forward's index flag, read with this backward's kernel already queued
        check = getattr(ctx, "index_check", None)
        if check is not None:
            check.raise_if_bad()
        return grad_logits, None, None, None


def tiled_l1_from_logits(logits: torch.Tensor, target: torch.Tensor, *,
                         target_indices: torch.Tensor | None = None,
                         _replay_cache: dict | None = None) -> torch.Tensor:
    """First-order L1 from compact logits and a frozen teacher (tiled_l1.py:176-209)."""
    if not logits.is_cuda or target.device != logits.device:
        raise ValueError("tiled L1 requires CUDA logits on one device")
    if logits.dtype != torch.bfloat16:
        raise ValueError("tiled L1 requires BF16 logits")
    if logits.ndim < 1 or logits.numel() == 0:
        raise ValueError("tiled L1 requires nonempty logits with a vocabulary dimension")
    if target.requires_grad:
        raise ValueError("tiled L1 requires frozen teacher logits")
    if logits.dtype != target.dtype or (target_indices is None and logits.shape != target.shape):
        raise ValueError("draft and teacher logits must share shape and dtype")
    if not logits.is_contiguous() or not target.is_contiguous():
        raise ValueError("tiled L1 requires contiguous logits")
    if target_indices is not None:
        if (target.ndim != 2 or target.shape[-1] != logits.shape[-1] or target.shape[0] == 0
                or target_indices.device != logits.device or target_indices.dtype != torch.int64
                or target_indices.ndim != 1 or not target_indices.is_contiguous()
                or target_indices.numel() != logits.numel() // logits.shape[-1]):
            raise ValueError("indexed teacher requires a nonempty 2D table and one contiguous CUDA "
                             "int64 index per Draft row")
    return _TiledL1.apply(logits, target, target_indices, _replay_cache)
