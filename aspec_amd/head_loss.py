"""The selective-head objective as one operator: vocab GEMM + CE + softmax-L1, logits through HBM once.

The DSpark head (`_prediction_terms`, aspec/models/dspark.py:553-612) projects the draft hidden
states onto the vocabulary, takes CE against the labels and the tiled L1 against the frozen
teacher, and the model combines them into `ce_alpha * ce_num + l1_alpha * l1_num`
(dspark.py:485-491) with per-row eval-mask x decay weights. With those weights known before the
forward, `selective_head_objective` computes logits = hidden W^T with the library GEMM, then one
loss pass (`aspec_ce_l1_fused_fwd_bwd`) writes CE, L1 and the objective's dlogits over the logits
in place; the backward is dh = g * dlogits W (g scales dh in place on the device, a no-op pass when
g == 1). Against the unfused composition (GEMM, loss forward,
loss backward, dgrad GEMM) this drops the backward's second read of the logits and teacher rows and
one kernel launch. Vocabularies the fused pass does not cover (V % 8 != 0 or V > 32768) run that
composition instead, with the same results.
"""

from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from aspec_amd import _lib, _timing
from aspec_amd.loss import _ce_l1_fused, ce_l1_from_logits, fused_grad_vocab


class _SelectiveHeadObjective(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, weight_t, targets, teacher, indices, ce_weights, l1_weights,
                ignore_index, want_argmax, teacher_ready):
        with _timing.region("head_gemm_fwd"):
            logits = torch.matmul(hidden, weight.t())
        if teacher_ready is not None:
            torch.cuda.current_stream(hidden.device).wait_event(teacher_ready)
        ce, l1, dlogits, amax, check = _ce_l1_fused(logits, targets, teacher, ce_weights, l1_weights,
                                                    indices, ignore_index, want_argmax, True)
        if not ctx.needs_input_grad[0]:
            check.raise_if_bad()
            ctx.check = None
        else:
            ctx.check = check
        objective = torch.dot(ce_weights.reshape(-1).float(), ce.reshape(-1)) + torch.dot(
            l1_weights.reshape(-1).float(), l1.reshape(-1))
        ctx.save_for_backward(dlogits, weight_t)
        ctx.mark_non_differentiable(ce, l1)
        if want_argmax:
            ctx.mark_non_differentiable(amax)
            return objective, ce, l1, amax
        return objective, ce, l1

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_objective, *unused):
        dlogits, weight_t = ctx.saved_tensors
        with _timing.region("head_gemm_dgrad"):
            dh = torch.matmul(dlogits, weight_t.t())
        if grad_objective is not None:
            # dh *= g on the device; g is exactly 1 for loss.backward(), and then nothing is written
            g = grad_objective.detach().reshape(()).to(device=dh.device, dtype=torch.float32)
            _lib.call("aspec_scale_bf16_by_device_scalar", dh.data_ptr(), dh.numel(), g.data_ptr(),
                      _lib.stream_handle(dh.device))
        # The forward's index flag is read only now, with the dgrad GEMM already queued behind the
        # loss pass: the host waits for the loss kernel while the GPU has the GEMM to run, and a bad
        # index still raises before dh reaches the caller.
        if ctx.check is not None:
            ctx.check.raise_if_bad()
        return dh, None, None, None, None, None, None, None, None, None, None


def selective_head_objective(hidden, weight, targets, teacher, *, ce_weights, l1_weights,
                             teacher_indices=None, weight_t=None, ignore_index=-100,
                             return_argmax=False, teacher_ready=None):
    """objective = sum_r (ce_weights[r] ce[r] + l1_weights[r] l1[r]) for the logits hidden W^T.

    hidden [rows, H] (bf16, differentiable), weight W [V, H] (frozen), targets [rows] int64,
    teacher [rows, V] or, with `teacher_indices` [rows] int64, a [T, V] table (frozen), ce_weights /
    l1_weights [rows]. `weight_t` is W^T made contiguous once by the caller (the dgrad GEMM's TN
    operand); it is derived here if omitted. `teacher_ready`, a CUDA event, is waited for after the
    vocabulary GEMM and before the loss (the teacher logits' producer may still run on another
    stream). Returns (objective, ce, l1[, argmax]); only the objective carries gradient (to
    `hidden`)."""
    if hidden.ndim != 2 or weight.ndim != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("hidden [rows, H] and weight [V, H] must share H")
    if weight.requires_grad:
        raise ValueError("the selective head's vocabulary projection is frozen")
    if weight_t is None:
        weight_t = weight.t().contiguous()
    if fused_grad_vocab(weight.shape[0]):
        return _SelectiveHeadObjective.apply(hidden, weight, weight_t, targets.reshape(-1), teacher,
                                             teacher_indices, ce_weights.reshape(-1),
                                             l1_weights.reshape(-1), ignore_index, return_argmax,
                                             teacher_ready)
    with _timing.region("head_gemm_fwd"):
        logits = torch.matmul(hidden, weight.t())
    if teacher_ready is not None:
        torch.cuda.current_stream(hidden.device).wait_event(teacher_ready)
    out = ce_l1_from_logits(logits, targets.reshape(-1), teacher, teacher_indices=teacher_indices,
                            ignore_index=ignore_index, return_argmax=return_argmax)
    ce, l1 = out[0], out[1]
    objective = torch.dot(ce_weights.reshape(-1).float(), ce) + torch.dot(l1_weights.reshape(-1).float(), l1)
    if return_argmax:
        return objective, ce.detach(), l1.detach(), out[2]
    return objective, ce.detach(), l1.detach()
