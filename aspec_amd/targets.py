"""DSpark targets: labels, eval mask and decay weights (aspec/models/dspark.py:163-172, 240-272,
311-315, 325) in one HIP launch.

`dspark_targets` returns the tensors `DSparkModel.forward` derives from the anchors before the
head: the (keep-zeroed) label indices, target and previous token ids, the teacher row index
(label - 1), the eval mask and the decay-weighted mask. The decay table itself is the
reference's torch expression (`decay_weights`), so the weighted mask is bit-identical.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib, _timing


def decay_weights(block_size: int, loss_decay_gamma: Optional[float], prediction_start: int = 0,
                  device: torch.device | None = None) -> torch.Tensor:
    """`DSparkModel._decay_weights` (dspark.py:163-172), shape [1, 1, block_size]."""
    k = torch.arange(block_size, device=device).view(1, 1, -1)
    if loss_decay_gamma is not None and loss_decay_gamma > 0:
        return torch.exp(-(k - prediction_start).clamp_min(0).float() / loss_decay_gamma)
    return torch.ones_like(k, dtype=torch.float32)


_decay_tables: dict = {}


def _decay_table(block_size: int, loss_decay_gamma: Optional[float], prediction_start: int,
                 device: torch.device) -> torch.Tensor:
    """The flattened `decay_weights` table, built once per (block size, gamma, start, device): the
    same torch expression, so the same values, without its half-dozen launches on every call."""
    key = (block_size, loss_decay_gamma, prediction_start, str(device))
    table = _decay_tables.get(key)
    if table is None:
        table = decay_weights(block_size, loss_decay_gamma, prediction_start, device).reshape(-1).contiguous()
        _decay_tables[key] = table
    return table


@dataclass
class DSparkTargets:
    label_index: torch.Tensor    # [B, nb, bs] int64, min(a + 1 + k, S - 1), 0 for dropped blocks
    target_ids: torch.Tensor     # [B, nb, bs] int64
    prev_ids: torch.Tensor       # [B, nb, bs] int64 (anchor token, then target_ids[..., :-1])
    teacher_index: torch.Tensor  # [B, nb, bs] int64, max(label_index - 1, 0)
    eval_mask: torch.Tensor      # [B, nb, bs] float32
    weights: torch.Tensor        # [B, nb, bs] float32 = eval_mask * decay


def dspark_targets(anchor_positions: torch.Tensor, block_keep_mask: torch.Tensor,
                   input_ids: torch.Tensor, loss_mask: torch.Tensor, block_size: int,
                   loss_decay_gamma: Optional[float] = None, prediction_start: int = 0,
                   ctx_doc_ids: Optional[torch.Tensor] = None) -> DSparkTargets:
    """Labels and eval mask (DeepSpec convention) of dspark.py:240-272 plus the gathers of
    311-315 and 325, for anchors [B, nb] (in [0, S)) over rows [B, S]."""
    bsz, seq_len = input_ids.shape
    if anchor_positions.shape != block_keep_mask.shape or anchor_positions.shape[0] != bsz:
        raise ValueError("anchor positions and block keep mask must both be [batch, blocks]")
    if loss_mask.shape != input_ids.shape or (ctx_doc_ids is not None and ctx_doc_ids.shape != input_ids.shape):
        raise ValueError("input_ids, loss_mask and ctx_doc_ids must have identical shapes")
    device = input_ids.device
    if device.type != "cuda":
        raise ValueError("DSpark targets (HIP) need their tensors on the GPU")
    n_blocks = anchor_positions.shape[1]
    decay = _decay_table(block_size, loss_decay_gamma, prediction_start, device)
    anchors = anchor_positions.to(torch.long).contiguous()
    keep = block_keep_mask.contiguous()
    if keep.dtype != torch.bool:
        keep = keep != 0
    ids = input_ids.to(torch.long).contiguous()
    mask = loss_mask.contiguous()
    docs = ctx_doc_ids.to(torch.long).contiguous() if ctx_doc_ids is not None else None
    shape = (bsz, n_blocks, block_size)
    with _timing.region("dspark_targets"):
        out = DSparkTargets(*(torch.empty(shape, dtype=torch.long, device=device) for _ in range(4)),
                            torch.empty(shape, dtype=torch.float32, device=device),
                            torch.empty(shape, dtype=torch.float32, device=device))
        _lib.call("aspec_dspark_targets", anchors.data_ptr(), keep.data_ptr(), ids.data_ptr(),
                  mask.data_ptr(), _lib.mask_dtype_code(mask), _lib.ptr(docs), bsz, seq_len,
                  n_blocks, block_size, prediction_start, decay.data_ptr(),
                  out.label_index.data_ptr(), out.target_ids.data_ptr(), out.prev_ids.data_ptr(),
                  out.teacher_index.data_ptr(), out.eval_mask.data_ptr(), out.weights.data_ptr(),
                  _lib.stream_handle(device))
    return out
