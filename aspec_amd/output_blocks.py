"""Output-only block selection (aspec/models/ops/output_blocks.py:19-112) on the GPU.

The stable "kept first" orders, per-owner kept widths and per-chunk kept counts come from one
HIP launch pair (`aspec_output_block_layout`); each public function then makes the same single
device-to-host transfer the reference makes. Gathers and scatters of activations
(`select_blocks`, `restore_blocks`) are the reference's torch indexing.
"""

from __future__ import annotations

import torch

from . import _lib, _timing


def _layout(keep_mask: torch.Tensor, owners: int, chunk_begin: int, chunk_end: int,
            chunk_size: int, with_order: bool):
    if keep_mask.device.type != "cuda":
        raise ValueError("output-block layout (HIP) needs the keep mask on the GPU")
    keep = keep_mask.contiguous()
    if keep.dtype != torch.bool:
        keep = keep != 0
    batch, slots = keep.shape
    chunks = (chunk_end - chunk_begin + chunk_size - 1) // chunk_size if chunk_end > chunk_begin else 0
    with _timing.region("output_block_layout"):
        summary = torch.empty(1 + chunks, dtype=torch.int32, device=keep.device)
        order = torch.empty(batch, slots, dtype=torch.long, device=keep.device) if with_order else None
        _lib.call("aspec_output_block_layout", keep.data_ptr(), batch, slots, owners, chunk_begin,
                  chunk_end, chunk_size, _lib.ptr(order), summary.data_ptr(),
                  _lib.stream_handle(keep.device))
    return order, summary


def _output_block_counts(keep_mask: torch.Tensor, chunk_size: int) -> torch.Tensor:
    """Per-chunk kept counts, max over rows (output_blocks.py:19-25), as a device tensor."""
    _, summary = _layout(keep_mask, 1, 0, keep_mask.shape[1], chunk_size, False)
    return summary[1:].to(torch.long)


def output_block_counts(keep_mask: torch.Tensor, chunk_size: int) -> list[int]:
    """One host transfer for all original head chunks (output_blocks.py:28-30)."""
    _, summary = _layout(keep_mask, 1, 0, keep_mask.shape[1], chunk_size, False)
    return summary[1:].tolist()


def output_block_indices(keep_mask: torch.Tensor, count: int | None = None) -> torch.Tensor | None:
    """Valid blocks in original order, masked padding retained across rows (output_blocks.py:33-48)."""
    order, summary = _layout(keep_mask, 1, 0, keep_mask.shape[1], keep_mask.shape[1] or 1, True)
    if count is None:
        count = int(summary[0].item())
    if count == keep_mask.shape[1]:
        return None
    if count == 0:
        return torch.empty((keep_mask.shape[0], 0), dtype=torch.long, device=keep_mask.device)
    return order[:, :count]


def select_blocks(value: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """output_blocks.py:51-53."""
    index = indices.reshape(*indices.shape, *([1] * (value.ndim - 2)))
    return value.gather(1, index.expand(*indices.shape, *value.shape[2:]))


def owner_block_indices(keep_mask: torch.Tensor, owners: int, *,
                        retained: int | None = None) -> torch.Tensor | None:
    """Stable selection inside each contiguous owner, equal widths (output_blocks.py:56-75)."""
    if owners < 1 or keep_mask.shape[1] % owners:
        raise ValueError("Query slots must divide evenly across CP owners")
    width = keep_mask.shape[1] // owners
    order, summary = _layout(keep_mask, owners, 0, width, width or 1, True)
    if retained is None:
        retained = max(1, int(summary[0].item()))
    return _owner_indices(order, keep_mask.shape[0], owners, width, retained)


def _owner_indices(order, batch, owners, width, retained):
    if not 1 <= retained <= width:
        raise ValueError("Retained owner width must be within the original query slots")
    if retained == width:
        return None
    return order.view(batch, owners, width)[..., :retained].flatten(1)


def prepare_block_layout(keep_mask: torch.Tensor, owners: int, rank: int, chunk_size: int):
    """One pre-backbone transfer for owner width and this rank's head chunks (output_blocks.py:78-91)."""
    if owners < 1 or not 0 <= rank < owners or keep_mask.shape[1] % owners:
        raise ValueError("Query slots and rank must match contiguous CP owners")
    width = keep_mask.shape[1] // owners
    order, summary = _layout(keep_mask, owners, rank * width, (rank + 1) * width, chunk_size, True)
    values = summary.tolist()
    return _owner_indices(order, keep_mask.shape[0], owners, width, max(1, values[0])), values[1:]


def restore_blocks(value: torch.Tensor, indices: torch.Tensor, original_width: int) -> torch.Tensor:
    """Restore the original query slots (output_blocks.py:94-98)."""
    index = indices.reshape(*indices.shape, *([1] * (value.ndim - 2)))
    return value.new_zeros(value.shape[0], original_width, *value.shape[2:]).scatter(
        1, index.expand_as(value), value
    )

