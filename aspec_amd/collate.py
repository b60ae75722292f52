"""Packed-row collation: `DFlashPackingCollator` (aspec/data/utils.py:199-356) on the GPU.

Same constructor arguments, validation and error messages as the reference, and the same output
dict, plus `cu_seqlens` (int32 [ndoc + 1] = [0, cumsum(lengths)]) for the THD kernels. The
features are device tensors (the live data path loads them onto the training device before
collation); every field of the row is written by the HIP library in two launches: one copy
launch for input_ids, loss_mask and the hidden-state fields (document rows plus the zero
padding), one launch for ctx_doc_ids, base_position_ids and attention_mask.
"""

from __future__ import annotations

from typing import Any, Dict, List

import numpy as np
import torch

from . import _lib, _timing

# Copy spans are split into pieces of at most this many bytes so that one large field spreads
# over many workgroups (one workgroup per span).
_SPAN_BYTES = 256 * 1024


def context_shard_bounds(sequence_length: int, rank: int, world_size: int, *,
                         alignment: int = 1) -> tuple[int, int]:
    """Contiguous CP ownership of one document (aspec/inference/context.py:30-55)."""
    if sequence_length < 0:
        raise ValueError("sequence_length must be non-negative")
    if world_size <= 0 or not 0 <= rank < world_size:
        raise ValueError("invalid context-parallel rank or world size")
    if isinstance(alignment, bool) or not isinstance(alignment, int) or alignment <= 0:
        raise ValueError("context shard alignment must be a positive integer")
    complete_groups = sequence_length // alignment
    start = complete_groups * rank // world_size * alignment
    end = complete_groups * (rank + 1) // world_size * alignment
    if rank == world_size - 1:
        end = sequence_length
    return start, end


def _packing_tensor(item: Dict[str, Any], name: str, sample_len: int) -> torch.Tensor:
    """Field validation of aspec/data/utils.py:182-196."""
    value = item.get(name)
    if not isinstance(value, torch.Tensor):
        raise KeyError(f"DFlashPackingCollator: {name} tensor not found")
    expected_dim = 2 if name in {"input_ids", "loss_mask"} else 3
    if value.dim() != expected_dim or value.shape[0] != 1:
        raise ValueError(f"DFlashPackingCollator: invalid {name} shape {tuple(value.shape)}")
    if value.shape[1] < sample_len:
        raise ValueError(
            f"DFlashPackingCollator: {name} length {value.shape[1]} "
            f"is shorter than input_ids length {sample_len}"
        )
    return value[:, :sample_len]


class _SpanTable:
    """Host-side list of copy spans, shipped to the device as one int64 [n, 3] array."""

    def __init__(self):
        self.rows: list[np.ndarray] = []

    def add(self, src: int, dst: int, nbytes: int) -> None:
        if nbytes <= 0:
            return
        offs = np.arange(0, nbytes, _SPAN_BYTES, dtype=np.int64)
        sizes = np.minimum(_SPAN_BYTES, nbytes - offs)
        srcs = np.zeros_like(offs) if src == 0 else src + offs
        self.rows.append(np.stack([srcs, dst + offs, sizes], axis=1))

    def copy_rows(self, src: torch.Tensor, dst: torch.Tensor, dst_row: int) -> None:
        """Rows of `src` [1, n, ...] into `dst` [1, T, ...] from row `dst_row` (row-contiguous)."""
        n = src.shape[1]
        if n == 0:
            return
        if src.dim() > 2 and src.stride(-1) != 1:
            src = src.contiguous()
        row_bytes = dst[0, 0].numel() * dst.element_size()
        base = dst.data_ptr() + dst_row * row_bytes
        if src[0].is_contiguous():
            self.add(src.data_ptr(), base, n * row_bytes)
        else:
            stride = src.stride(1) * src.element_size()
            for r in range(n):
                self.add(src.data_ptr() + r * stride, base + r * row_bytes, row_bytes)

    def zero_rows(self, dst: torch.Tensor, first: int, count: int) -> None:
        if count > 0:
            row_bytes = dst[0, 0].numel() * dst.element_size()
            self.add(0, dst.data_ptr() + first * row_bytes, count * row_bytes)

    def run(self, device) -> None:
        """One copy launch. The table's memory is stream-ordered: a later allocation that reuses
        it is written by work queued after this launch."""
        if not self.rows:
            return
        table = torch.from_numpy(np.concatenate(self.rows)).to(device)
        with _timing.region("pack_copy"):
            _lib.call("aspec_pack_copy", table.data_ptr(), table.shape[0], _lib.stream_handle(device))


class DFlashPackingCollator:
    """Concatenate complete documents into one fixed, document-aware row (utils.py:199-356)."""

    def __init__(
        self, max_seq_length: int, *, pad_to_max_length: bool = True,
        context_parallel_rank: int = 0, context_parallel_size: int = 1,
        context_shard_alignment: int = 1,
    ):
        if max_seq_length <= 0:
            raise ValueError("DFlashPackingCollator requires max_seq_length > 0")
        self.max_seq_length = int(max_seq_length)
        self.pad_to_max_length = bool(pad_to_max_length)
        self.cp_rank = int(context_parallel_rank)
        self.cp_size = int(context_parallel_size)
        self.cp_alignment = int(context_shard_alignment)
        if self.cp_size <= 0 or not 0 <= self.cp_rank < self.cp_size:
            raise ValueError("Invalid packed context-parallel ownership")
        if self.cp_alignment <= 0:
            raise ValueError("Packed context shard alignment must be positive")
        if self.cp_size > 1 and self.pad_to_max_length:
            raise ValueError("Context-sharded packing requires unpadded THD rows")

    def __call__(self, features: List[Dict[str, Any]]) -> Dict[str, Any]:
        if not features:
            raise ValueError("DFlashPackingCollator received an empty row")
        lengths = [int(item["input_ids"].shape[1]) for item in features]
        used = sum(lengths)
        if used <= 0 or used > self.max_seq_length:
            raise ValueError(f"Packed row has {used} tokens; expected 1..{self.max_seq_length}")
        have_hidden = [item.get("hidden_states") is not None for item in features]
        have_last_hidden = [item.get("last_hidden_states") is not None for item in features]
        if any(have_hidden) and not all(have_hidden):
            raise ValueError("hidden_states must be present for every packed document")
        if any(have_last_hidden) and not all(have_last_hidden):
            raise ValueError("last_hidden_states must be present for every packed document")
        ids = [_packing_tensor(item, "input_ids", n) for item, n in zip(features, lengths)]
        masks = [_packing_tensor(item, "loss_mask", n) for item, n in zip(features, lengths)]
        device = ids[0].device
        pad = self.max_seq_length - used if self.pad_to_max_length else 0
        row = used + pad
        hidden: Dict[str, list] = {}
        for name, presence in (("hidden_states", have_hidden),
                               ("last_hidden_states", have_last_hidden)):
            if not all(presence):
                continue
            bounds = [context_shard_bounds(n, self.cp_rank, self.cp_size,
                                           alignment=self.cp_alignment) for n in lengths]
            parts = [_packing_tensor(item, name, end - start)
                     for item, (start, end) in zip(features, bounds, strict=True)]
            if self.cp_size > 1:
                expected = [end - start for start, end in bounds]
                if any(item[name].shape[1] != count for item, count in zip(features, expected)):
                    raise ValueError(f"Packed {name} does not match per-document CP ownership")
            hidden[name] = parts
        work = [item.get("_aspec_work") for item in features]
        if not all(isinstance(item, dict) and isinstance(item.get("execution_id"), str)
                   and item["execution_id"] for item in work):
            raise ValueError("Packed row contains incomplete ASpec work identity")
        for parts in (ids, masks, *hidden.values()):
            if any(p.device != device for p in parts) or device.type != "cuda":
                raise ValueError("DFlashPackingCollator (HIP) needs every feature on one GPU")
            if any(p.dtype != parts[0].dtype or p.shape[2:] != parts[0].shape[2:] for p in parts):
                raise ValueError("DFlashPackingCollator: packed documents disagree in dtype or width")

        with _timing.region("pack_row"):
            spans = _SpanTable()
            batch: Dict[str, Any] = {"packed_document_lengths": tuple(lengths)}
            for name, parts in (("input_ids", ids), ("loss_mask", masks)):
                out = torch.empty((1, row), dtype=parts[0].dtype, device=device)
                offset = 0
                for part in parts:
                    spans.copy_rows(part.unsqueeze(-1), out.unsqueeze(-1), offset)
                    offset += part.shape[1]
                spans.zero_rows(out.unsqueeze(-1), used, pad)
                batch[name] = out
            cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
            cu_dev = torch.from_numpy(cu).to(device)
            docs = torch.empty((1, row), dtype=torch.long, device=device)
            positions = torch.empty((1, row), dtype=torch.long, device=device)
            attention = torch.empty((1, row), dtype=torch.long, device=device)
            _lib.call("aspec_pack_row_metadata", cu_dev.data_ptr(), len(lengths), row,
                      docs.data_ptr(), positions.data_ptr(), attention.data_ptr(),
                      _lib.stream_handle(device))
            batch["attention_mask"] = attention
            batch["ctx_doc_ids"] = docs
            batch["base_position_ids"] = positions
            batch["cu_seqlens"] = cu_dev
            batch["hidden_states"] = None
            batch["target"] = None
            batch["last_hidden_states"] = None
            for name, parts in hidden.items():
                owned = sum(p.shape[1] for p in parts)
                out = torch.empty((1, owned + pad, *parts[0].shape[2:]), dtype=parts[0].dtype,
                                  device=device)
                offset = 0
                for part in parts:
                    spans.copy_rows(part, out, offset)
                    offset += part.shape[1]
                spans.zero_rows(out, owned, pad)
                batch[name] = out
            spans.run(device)
        batch["_aspec_work"] = work
        if self.cp_size > 1:
            offset, owned_positions = 0, []
            for n in lengths:
                start, end = context_shard_bounds(n, self.cp_rank, self.cp_size,
                                                  alignment=self.cp_alignment)
                owned_positions.append(torch.arange(offset + start, offset + end, dtype=torch.long,
                                                    device=device))
                offset += n
            batch["packed_context_positions"] = torch.cat(owned_positions).unsqueeze(0)
        return batch
