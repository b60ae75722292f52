"""Selective-head loss kernels: cross-entropy and the fused CE + softmax-L1 (HIP).

`cross_entropy` matches `F.cross_entropy(logits, targets, reduction="none")` as called at
aspec/models/dspark.py:568-570 (ignore_index -100), computed in fp32 from bf16 logits.
`ce_l1_from_logits` returns (ce, l1) per row from ONE read of the draft and teacher logits -- the
two reductions share max / sum(exp) of the draft row -- and its backward writes dlogits once for
both terms. It is what the DSpark head (`_prediction_terms`, dspark.py:553-636) needs per chunk.
"""

from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from aspec_amd import _lib, _timing

STATS = 8


class IndexCheck:
    """Fail-closed check of the indices a loss forward consumed (the reference device-asserts on an
    out-of-range teacher index, tiled_l1.py:41-42, and torch's cross-entropy on a bad target).

    The forward ORs bit 1 (teacher index) / bit 2 (target) into a device flag and writes NaN rows.
    The flag is copied into pinned host memory behind an event on the launch stream, so reading it
    later costs no stall: the backward reads it after its own kernels are queued (the GPU keeps
    working while the host waits for the forward's flag), and a forward that no backward will
    follow reads it at once. Either raises ValueError before a result reaches the caller."""

    def __init__(self, flags: torch.Tensor):
        self.host = torch.empty(1, dtype=torch.int32, pin_memory=True)
        self.host.copy_(flags, non_blocking=True)
        self.event = torch.cuda.Event()
        self.event.record(torch.cuda.current_stream(flags.device))

    def raise_if_bad(self) -> None:
        self.event.synchronize()
        bad = int(self.host[0])
        if bad & 1:
            raise ValueError("teacher index out of range: every target index must address a row "
                             "of the teacher table")
        if bad & 2:
            raise ValueError("cross-entropy target out of range: targets must lie in [0, vocab) "
                             "or equal ignore_index")


def _check_logits(logits):
    if not logits.is_cuda:
        raise ValueError("loss kernels require CUDA logits")
    if logits.dtype != torch.bfloat16:
        raise ValueError("loss kernels require BF16 logits")
    if logits.ndim < 1 or logits.numel() == 0:
        raise ValueError("loss kernels require nonempty logits with a vocabulary dimension")
    if not logits.is_contiguous():
        raise ValueError("loss kernels require contiguous logits")


class _CeL1(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, targets, teacher, indices, ignore_index, want_argmax=False, replay_cache=None):
        vocab = logits.shape[-1]
        rows = logits.numel() // vocab
        dev = logits.device
        trows = teacher.shape[0] if (teacher is not None and indices is not None) else rows
        ctx.index_check = None
        if replay_cache:
            # Checkpoint replay of the same head chunk (the logits are recomputed bit for bit): the
            # first forward's statistics and per-row results are reused and no forward kernel runs
            # (the role of tiled_l1.py:134-139 for L1, here for CE, L1 and argmax together).
            stats, ce, l1, amax = replay_cache["statistics"]
            if (ce.shape != logits.shape[:-1] or stats.device != dev or replay_cache["vocab"] != vocab
                    or (l1 is None) != (teacher is None) or (want_argmax and amax is None)):
                raise ValueError("L1 checkpoint statistics belong to a different head chunk")
        else:
            stats = torch.empty((rows, STATS), dtype=torch.float32, device=dev)
            ce = torch.empty(logits.shape[:-1], dtype=torch.float32, device=dev)
            l1 = torch.empty(logits.shape[:-1], dtype=torch.float32, device=dev) if teacher is not None else None
            flags = torch.zeros(1, dtype=torch.int32, device=dev)
            amax = torch.empty(logits.shape[:-1], dtype=torch.int64, device=dev) if want_argmax else None
            with _timing.region("loss_fwd"):
                _lib.call("aspec_ce_l1_argmax_fwd", _lib.ptr(logits), _lib.ptr(teacher), _lib.ptr(indices),
                          trows, _lib.ptr(targets), ignore_index, rows, vocab, _lib.ptr(l1), _lib.ptr(ce),
                          _lib.ptr(amax), _lib.ptr(stats), _lib.ptr(flags), _lib.stream_handle(dev))
            ctx.index_check = IndexCheck(flags)
            if not ctx.needs_input_grad[0]:
                ctx.index_check.raise_if_bad()
            if replay_cache is not None:
                replay_cache["statistics"] = (stats, ce.detach(), None if l1 is None else l1.detach(),
                                              amax)
                replay_cache["vocab"] = vocab
        ctx.save_for_backward(logits, targets, teacher, indices, stats)
        ctx.ignore_index = ignore_index
        ctx.trows = trows
        ctx.set_materialize_grads(False)
        # new views keep the cached tensors free of this call's grad_fn
        ce = ce.view_as(ce)
        l1 = torch.zeros_like(ce) if l1 is None else l1.view_as(l1)
        if not want_argmax:
            return ce, l1
        amax = amax.view_as(amax)
        ctx.mark_non_differentiable(amax)
        return ce, l1, amax

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_ce, grad_l1, grad_argmax=None):
        logits, targets, teacher, indices, stats = ctx.saved_tensors
        vocab = logits.shape[-1]
        rows = logits.numel() // vocab
        gce = None if grad_ce is None else grad_ce.to(torch.float32).contiguous()
        gl1 = None if (grad_l1 is None or teacher is None) else grad_l1.to(torch.float32).contiguous()
        grad_logits = torch.empty_like(logits)
        if gce is None and gl1 is None:
            grad_logits.zero_()
        else:
            with _timing.region("loss_bwd"):
                _lib.call("aspec_ce_l1_bwd", _lib.ptr(logits), _lib.ptr(teacher), _lib.ptr(indices),
                          ctx.trows, _lib.ptr(targets), ctx.ignore_index, rows, vocab, _lib.ptr(stats),
                          _lib.ptr(gl1), _lib.ptr(gce), _lib.ptr(grad_logits),
                          _lib.stream_handle(logits.device))
        # the forward's index flag, read after this backward's launch is queued (no GPU idle time);
        # a bad index raises before the gradient reaches the caller
        if ctx.index_check is not None:
            ctx.index_check.raise_if_bad()
        return grad_logits, None, None, None, None, None, None


def ce_l1_from_logits(logits, targets, teacher=None, *, teacher_indices=None, ignore_index=-100,
                      return_argmax=False, _replay_cache=None):
    """Per-row (cross-entropy, softmax-L1) from bf16 logits in one pass (HIP). With
    `return_argmax`, also the row argmax (torch.argmax semantics: the first NaN, else the first
    maximum) from the same pass, for the head's accuracy metric (dspark.py:625).

    `_replay_cache` is the head chunk's checkpoint-replay dict (`loss_cache`, dspark.py:473,602):
    an empty dict receives this forward's statistics and results; a filled one is replayed
    without a forward kernel (the recomputed logits of a checkpoint replay are bitwise the same)."""
    _check_logits(logits)
    rows = logits.numel() // logits.shape[-1]
    if targets.dtype != torch.int64 or targets.numel() != rows or targets.device != logits.device:
        raise ValueError("targets must be one int64 class index per logit row on the logits device")
    targets = targets.reshape(-1).contiguous()
    if teacher is not None:
        _check_teacher(logits, teacher, teacher_indices, rows)
        if teacher_indices is not None:
            teacher_indices = teacher_indices.reshape(-1).contiguous()
    return _CeL1.apply(logits, targets, teacher, teacher_indices, ignore_index, return_argmax,
                       _replay_cache)


def _check_teacher(logits, teacher, teacher_indices, rows):
    if teacher.requires_grad:
        raise ValueError("tiled L1 requires frozen teacher logits")
    if teacher.dtype != logits.dtype or not teacher.is_contiguous() or teacher.device != logits.device:
        raise ValueError("draft and teacher logits must share shape and dtype")
    if teacher_indices is None and teacher.shape != logits.shape:
        raise ValueError("draft and teacher logits must share shape and dtype")
    if teacher_indices is not None and (
            teacher.ndim != 2 or teacher.shape[-1] != logits.shape[-1] or teacher.shape[0] == 0
            or teacher_indices.dtype != torch.int64 or teacher_indices.numel() != rows
            or teacher_indices.device != logits.device):
        raise ValueError("indexed teacher requires a nonempty 2D table and one contiguous CUDA "
                         "int64 index per Draft row")


def fused_grad_vocab(vocab: int) -> bool:
    """Whether `ce_l1_fused_grad` covers this vocabulary size (V % 8 == 0, V <= 32768)."""
    return vocab % 8 == 0 and vocab <= 32768


def fused_grad_supported(logits) -> bool:
    """Whether `ce_l1_fused_grad` runs as one kernel for these logits (a covered vocabulary and
    16-byte aligned rows)."""
    return fused_grad_vocab(logits.shape[-1]) and logits.data_ptr() % 16 == 0


def ce_l1_fused_grad(logits, targets, teacher, *, ce_weights, l1_weights, teacher_indices=None,
                     ignore_index=-100, return_argmax=False, in_place=False):
    """Per-row (ce, l1[, argmax]) and dlogits of sum_r (ce_weights[r] ce[r] + l1_weights[r] l1[r])
    from one pass over the logits (no autograd). The DSpark loss numerator
    ce_alpha * ce_num + l1_alpha * l1_num (dspark.py:485-491) has this form with the weights
    alpha * eval mask * decay, so its backward needs no second read of the logits and teacher.
    With `in_place` the dlogits overwrite `logits` (which the caller must no longer need).
    Out-of-range teacher indices / targets raise ValueError. Returns (ce, l1, dlogits[, argmax]);
    raises NotImplementedError where `fused_grad_supported` is False."""
    ce, l1, dlogits, amax, check = _ce_l1_fused(logits, targets, teacher, ce_weights, l1_weights,
                                                teacher_indices, ignore_index, return_argmax, in_place)
    check.raise_if_bad()
    if return_argmax:
        return ce, l1, dlogits, amax
    return ce, l1, dlogits


def _ce_l1_fused(logits, targets, teacher, ce_weights, l1_weights, teacher_indices, ignore_index,
                 return_argmax, in_place):
    """The launch behind `ce_l1_fused_grad`; returns (ce, l1, dlogits, argmax, IndexCheck) with the
    index check still to be read."""
    _check_logits(logits)
    vocab = logits.shape[-1]
    rows = logits.numel() // vocab
    if targets.dtype != torch.int64 or targets.numel() != rows or targets.device != logits.device:
        raise ValueError("targets must be one int64 class index per logit row on the logits device")
    _check_teacher(logits, teacher, teacher_indices, rows)
    for w in (ce_weights, l1_weights):
        if w.numel() != rows or w.device != logits.device:
            raise ValueError("objective weights must hold one value per logit row on the logits device")
    targets = targets.reshape(-1).contiguous()
    indices = None if teacher_indices is None else teacher_indices.reshape(-1).contiguous()
    gce = ce_weights.reshape(-1).to(torch.float32).contiguous()
    gl1 = l1_weights.reshape(-1).to(torch.float32).contiguous()
    dev = logits.device
    trows = teacher.shape[0] if indices is not None else rows
    stats = torch.empty((rows, STATS), dtype=torch.float32, device=dev)
    ce = torch.empty(logits.shape[:-1], dtype=torch.float32, device=dev)
    l1 = torch.empty(logits.shape[:-1], dtype=torch.float32, device=dev)
    amax = torch.empty(logits.shape[:-1], dtype=torch.int64, device=dev) if return_argmax else None
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    dlogits = logits if in_place else torch.empty_like(logits)
    with _timing.region("loss_fused"):
        _lib.call("aspec_ce_l1_fused_fwd_bwd", _lib.ptr(logits), _lib.ptr(teacher), _lib.ptr(indices),
                  trows, _lib.ptr(targets), ignore_index, rows, vocab, _lib.ptr(gce), _lib.ptr(gl1),
                  _lib.ptr(l1), _lib.ptr(ce), _lib.ptr(amax), _lib.ptr(stats), _lib.ptr(dlogits),
                  _lib.ptr(flags), _lib.stream_handle(dev))
    return ce, l1, dlogits, amax, IndexCheck(flags)


def cross_entropy(logits, targets, ignore_index=-100):
    """Per-row cross-entropy of bf16 logits [..., V] against int64 targets (fp32 result)."""
    ce, _ = ce_l1_from_logits(logits, targets, None, ignore_index=ignore_index)
    return ce
