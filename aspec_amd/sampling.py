"""Sampled L1 and the sampling-filtered logits, on the HIP kernels of csrc/sampling.hip.

Drop-ins for `aspec.models.ops.loss.sampling_logits` and `compiled_l1_from_logits`
(aspec/models/ops/loss.py:57-89), the L1 of the DSpark head when `l1_target_sampling` /
`l1_draft_sampling` are set (aspec/models/dspark.py:606-609). A sampling is a
(temperature, top_p, top_k) triple; (1.0, 1.0, -1) leaves a distribution as it is:

  scaled = (x - max x) / temperature        (only when temperature != 1)
  keep   = the top_k highest tokens (0 < top_k < V) and the tokens whose preceding probability
           mass, in descending order with ties by token index, is <= top_p (top_p < 1)
  p      = softmax(scaled) renormalised over the kept tokens, 0 elsewhere.

The support is discrete and carries no gradient. bf16 logits (the head GEMM's output); the
teacher is frozen. No CPU path: the HIP library runs or the call raises.
"""

from __future__ import annotations

import math

import torch
from torch.autograd.function import once_differentiable

from aspec_amd import _lib, _timing
from aspec_amd.loss import IndexCheck

DEFAULT_SAMPLING = (1.0, 1.0, -1)


def _params(sampling, name: str) -> tuple[float, float, int]:
    """(temperature, top_p, top_k) validated as the reference's plan does (aspec/planning.py
    rejects a temperature that is not finite and > 0, top_p outside (0, 1], top_k 0 or < -1)."""
    try:
        temperature, top_p, top_k = sampling
    except (TypeError, ValueError):
        raise ValueError(f"{name} must be a (temperature, top_p, top_k) triple") from None
    temperature, top_p = float(temperature), float(top_p)
    if not (math.isfinite(temperature) and temperature > 0.0):
        raise ValueError(f"{name}: temperature must be finite and > 0, got {temperature}")
    if not (0.0 < top_p <= 1.0):
        raise ValueError(f"{name}: top_p must lie in (0, 1], got {top_p}")
    if int(top_k) != top_k or top_k == 0 or top_k < -1:
        raise ValueError(f"{name}: top_k must be -1 or >= 1, got {top_k}")
    return temperature, top_p, int(top_k)


def _rows(logits: torch.Tensor, what: str) -> torch.Tensor:
    if not logits.is_cuda:
        raise ValueError(f"{what} requires CUDA logits")
    if logits.dtype != torch.bfloat16:
        raise NotImplementedError(f"{what} takes bf16 logits (the head GEMM's output), got {logits.dtype}")
    if logits.ndim < 1 or logits.numel() == 0:
        raise ValueError(f"{what} requires nonempty logits with a vocabulary dimension")
    return logits.reshape(-1, logits.shape[-1]).contiguous()


class _SamplingLogits(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, temperature, top_p, top_k):
        flat = _rows(logits, "sampling_logits")
        rows, vocab = flat.shape
        out = torch.empty((rows, vocab), dtype=torch.float32, device=flat.device)
        stats = torch.empty((rows, _lib.load().aspec_sampling_stats_floats()), dtype=torch.float32,
                            device=flat.device)
        with _timing.region("sampling_logits"):
            _lib.call("aspec_sampling_logits_fwd", flat.data_ptr(), rows, vocab, temperature, top_p,
                      top_k, out.data_ptr(), stats.data_ptr(), _lib.stream_handle(flat.device))
        ctx.save_for_backward(flat, stats)
        ctx.shape = logits.shape
        return out.view(*logits.shape[:-1], vocab)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        flat, stats = ctx.saved_tensors
        rows, vocab = flat.shape
        g = grad_out.reshape(rows, vocab).to(torch.float32).contiguous()
        dx = torch.empty_like(flat)
        _lib.call("aspec_sampling_logits_bwd", flat.data_ptr(), g.data_ptr(), stats.data_ptr(), rows,
                  vocab, dx.data_ptr(), _lib.stream_handle(flat.device))
        return dx.view(ctx.shape), None, None, None


def sampling_logits(logits: torch.Tensor, sampling=DEFAULT_SAMPLING) -> torch.Tensor:
    """Differentiable fp32 logits on the joint top-k / top-p support (-inf elsewhere); ties use
    token-ID order (aspec/models/ops/loss.py:57-80). The default sampling returns `logits` itself;
    a temperature of 1 without an active filter returns `logits.float()`."""
    temperature, top_p, top_k = _params(sampling, "sampling")
    if (temperature, top_p, top_k) == DEFAULT_SAMPLING:
        return logits
    vocab = logits.shape[-1]
    if temperature == 1.0 and top_p == 1.0 and (top_k == -1 or top_k >= vocab):
        return logits.float()
    return _SamplingLogits.apply(logits, temperature, top_p, top_k)


class _SampledL1(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, teacher, indices, target_params, draft_params):
        flat = _rows(logits, "sampled L1")
        rows, vocab = flat.shape
        table = teacher.reshape(-1, vocab).contiguous()
        dev = flat.device
        l1 = torch.empty(rows, dtype=torch.float32, device=dev)
        stats = torch.empty((rows, _lib.load().aspec_sampled_l1_stats_floats()), dtype=torch.float32,
                            device=dev)
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        dt, dp, dk = draft_params
        tt, tp, tk = target_params
        with _timing.region("sampled_l1_fwd"):
            _lib.call("aspec_sampled_l1_fwd", flat.data_ptr(), table.data_ptr(), _lib.ptr(indices),
                      table.shape[0], rows, vocab, dt, dp, dk, tt, tp, tk, l1.data_ptr(),
                      stats.data_ptr(), flags.data_ptr(), _lib.stream_handle(dev))
        check = IndexCheck(flags)
        if not ctx.needs_input_grad[0]:
            check.raise_if_bad()
            ctx.check = None
        else:
            ctx.check = check
        ctx.save_for_backward(flat, table, indices, stats)
        ctx.shape = logits.shape
        return l1.view(logits.shape[:-1])

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_l1):
        flat, table, indices, stats = ctx.saved_tensors
        rows, vocab = flat.shape
        g = grad_l1.reshape(rows).to(torch.float32).contiguous()
        dx = torch.empty_like(flat)
        with _timing.region("sampled_l1_bwd"):
            _lib.call("aspec_sampled_l1_bwd", flat.data_ptr(), table.data_ptr(), _lib.ptr(indices),
                      table.shape[0], rows, vocab, stats.data_ptr(), g.data_ptr(), dx.data_ptr(),
                      _lib.stream_handle(flat.device))
        # the forward's index flag, read with this backward's kernel already queued
        if ctx.check is not None:
            ctx.check.raise_if_bad()
        return dx.view(ctx.shape), None, None, None, None


def compiled_l1_from_logits(logits: torch.Tensor, target_logits: torch.Tensor,
                            target_sampling=DEFAULT_SAMPLING, draft_sampling=DEFAULT_SAMPLING, *,
                            teacher_indices: torch.Tensor | None = None) -> torch.Tensor:
    """Per-token L1 between the sampling-filtered fp32 distributions of the draft logits and the
    teacher logits (aspec/models/ops/loss.py:83-89), differentiable in `logits`. With
    `teacher_indices` [rows] the teacher is a [T, V] table addressed per draft row. Both samplings
    at their default run the unsampled tiled-L1 kernels."""
    tparams = _params(target_sampling, "target_sampling")
    dparams = _params(draft_sampling, "draft_sampling")
    if target_logits.requires_grad:
        raise NotImplementedError("the teacher logits are frozen here (DSpark's teacher is); "
                                  "detach them or use a differentiable composition")
    if target_logits.device != logits.device or target_logits.dtype != logits.dtype:
        raise ValueError("draft and teacher logits must share device and dtype")
    vocab = logits.shape[-1]
    if teacher_indices is not None:
        if (target_logits.ndim != 2 or target_logits.shape[-1] != vocab or target_logits.shape[0] == 0
                or teacher_indices.dtype != torch.int64 or teacher_indices.device != logits.device
                or teacher_indices.numel() != logits.numel() // max(vocab, 1)):
            raise ValueError("indexed teacher requires a nonempty 2D table and one int64 index per "
                             "draft row on the logits device")
        teacher_indices = teacher_indices.reshape(-1).contiguous()
    elif target_logits.shape != logits.shape:
        raise ValueError("draft and teacher logits must share shape")
    if tparams == DEFAULT_SAMPLING and dparams == DEFAULT_SAMPLING:
        from aspec_amd.tiled_l1 import tiled_l1_from_logits

        return tiled_l1_from_logits(logits.contiguous(), target_logits.contiguous(),
                                    target_indices=teacher_indices)
    return _SampledL1.apply(logits, target_logits, teacher_indices, tparams, dparams)
