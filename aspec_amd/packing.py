"""Work-aware row packing for the live training path: the reference's `aspec/controller/packing.py`
interface (`PackingResult`, `count_eligible_anchor_starts`, `pack_work_aware_rows`), computed by the
native library (`aspec_count_eligible_anchor_starts`, `aspec_pack_work_aware_rows`).

The policy decides which pooled samples form the next dispatch: one packed row per data-parallel
rank, seeded with the oldest samples so that no awkward old sample starves, then filled best-fit by
useful-anchor density. The packed rows then go through `DFlashPackingCollator` and the THD metadata.
Validation and its messages follow the reference (packing.py:43-67, 110-130), so a controller
catches the same `ValueError`s.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import _lib


@dataclass(frozen=True)
class PackingResult:
    """One dispatch (packing.py:30-40): rank_rows[k] lists the pool indices packed for rank k."""

    rank_rows: list[list[int]]
    selected_indices: tuple[int, ...]
    packed_tokens: int
    capacity_tokens: int
    useful_anchor_starts: int

    @property
    def fill_ratio(self) -> float:
        return self.packed_tokens / self.capacity_tokens if self.capacity_tokens else 0.0


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data) if a.size else None


def _runs(packed_loss_mask: str | Sequence[int]) -> list[int]:
    if isinstance(packed_loss_mask, str):
        try:
            return [int(v) for v in packed_loss_mask.split(",") if v]
        except ValueError as exc:
            raise ValueError("packed_loss_mask contains a non-integer run length") from exc
    return [int(v) for v in packed_loss_mask]


def count_eligible_anchor_starts_batch(packed_loss_masks: Sequence[str | Sequence[int]],
                                       sample_lengths: Sequence[int], block_size: int) -> list[int]:
    """`count_eligible_anchor_starts` over a whole pool in one native call."""
    if len(packed_loss_masks) != len(sample_lengths):
        raise ValueError("packed_loss_masks and sample_lengths must have the same size")
    runs = [_runs(m) for m in packed_loss_masks]
    flat = np.ascontiguousarray(np.fromiter((v for r in runs for v in r), np.int64))
    offsets = np.zeros(len(runs) + 1, np.int64)
    np.cumsum([len(r) for r in runs], out=offsets[1:])
    lengths = np.ascontiguousarray(np.asarray(sample_lengths, np.int64).reshape(-1))
    out = np.zeros(len(runs), np.int64)
    if not len(runs):
        return []
    _lib.call("aspec_count_eligible_anchor_starts", _ptr(flat), _ptr(offsets), _ptr(lengths), len(runs),
              int(block_size), _ptr(out))
    return out.tolist()


def count_eligible_anchor_starts(packed_loss_mask: str | list[int], sample_length: int, block_size: int) -> int:
    """Supervised anchor starts whose complete block stays inside the sample (packing.py:43-67)."""
    if sample_length <= 0 or block_size <= 0:
        return 0
    return count_eligible_anchor_starts_batch([packed_loss_mask], [sample_length], block_size)[0]


def pack_work_aware_rows(lengths: list[int], useful_work: list[int], *, dp_size: int, max_seq_length: int,
                         max_selected: int | None = None) -> PackingResult | None:
    """One row per DP rank, oldest-work seeded, best-fit by useful-anchor density (packing.py:87-167).
    Returns None when the pool holds fewer samples than ranks."""
    if len(lengths) != len(useful_work):
        raise ValueError("lengths and useful_work must have the same size")
    if dp_size <= 0 or max_seq_length <= 0:
        raise ValueError("dp_size and max_seq_length must be positive")
    if max_selected is not None and max_selected < dp_size:
        raise ValueError("max_selected must be at least dp_size")
    invalid = [(i, n) for i, n in enumerate(lengths) if n <= 0 or n > max_seq_length]
    if invalid:
        preview = ", ".join(f"{i}:{n}" for i, n in invalid[:5])
        raise ValueError(f"Packing received work that can never fit a row: {preview}; max_seq_length={max_seq_length}")
    if len(lengths) < dp_size:
        return None
    n = np.ascontiguousarray(np.asarray(lengths, np.int64).reshape(-1))
    w = np.ascontiguousarray(np.asarray(useful_work, np.int64).reshape(-1))
    offsets = np.zeros(dp_size + 1, np.int64)
    samples = np.zeros(len(n), np.int64)
    tokens = np.zeros(dp_size, np.int64)
    _lib.call("aspec_pack_work_aware_rows", _ptr(n), _ptr(w), len(n), int(dp_size), int(max_seq_length),
              -1 if max_selected is None else int(max_selected), _ptr(offsets), _ptr(samples), _ptr(tokens))
    rank_rows = [samples[offsets[k]:offsets[k + 1]].tolist() for k in range(dp_size)]
    selected = tuple(sorted(samples[: offsets[-1]].tolist()))
    return PackingResult(
        rank_rows=rank_rows,
        selected_indices=selected,
        packed_tokens=int(tokens.sum()),
        capacity_tokens=dp_size * max_seq_length,
        useful_anchor_starts=int(w[list(selected)].sum()),
    )
