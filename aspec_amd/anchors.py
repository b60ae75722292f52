"""Anchor layout (aspec/models/ops/anchors.py) on the GPU.

Same function names, arguments, error messages and outputs as the reference. The random draws
stay torch's: each sampler calls `torch.rand` with the caller's generator exactly as the
reference does (same shape, device and order), and the HIP kernel turns the draws into anchors
with the reference's arithmetic, so a given generator state selects the same anchors.
"""

from __future__ import annotations

import hashlib
import logging
from typing import Optional, Tuple

import torch

from . import _lib, _timing

logger = logging.getLogger(__name__)


def _empty(bsz: int, num_anchors: int, seq_len: int, block_size: int, device: torch.device):
    """anchors.py:56-65."""
    logger.warning(
        f"Sequence too short for anchor sampling (seq_len={seq_len}, "
        f"block_size={block_size}). Returning dummy anchors so loss is zero."
    )
    return (
        torch.zeros(bsz, num_anchors, dtype=torch.long, device=device),
        torch.zeros(bsz, num_anchors, dtype=torch.bool, device=device),
    )


def anchor_sampling_seed(seed: int, step: int, microbatch: int, replica: int) -> int:
    """Stateless debug RNG key (anchors.py:68-74)."""
    key = f"{seed}:{step}:{microbatch}:{replica}".encode("ascii")
    return int.from_bytes(hashlib.blake2b(key, digest_size=8).digest(), "little") % (2**63)


def _require_gpu(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError("anchor layout (HIP) needs its tensors on the GPU")


def validate_injected_anchors(
    anchors: torch.Tensor,
    keep_mask: torch.Tensor,
    *,
    loss_mask: torch.Tensor,
    num_anchors: int,
    block_size: int,
    ctx_doc_ids: Optional[torch.Tensor] = None,
    allow_partial_last_target: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Validate replay inputs before they reach indexing or CP collectives (anchors.py:77-116).

    One kernel checks every kept slot; one flags read (a single device-to-host transfer) decides
    which of the reference's errors, if any, to raise, in the reference's order."""
    expected = (loss_mask.shape[0], num_anchors)
    if anchors.shape != expected or keep_mask.shape != expected:
        raise ValueError(f"Injected anchors and keep mask must both have shape {expected}")
    if anchors.dtype not in (torch.int32, torch.int64) or keep_mask.dtype != torch.bool:
        raise ValueError("Injected anchors must be integer and keep mask must be boolean")
    if ctx_doc_ids is not None and ctx_doc_ids.shape != loss_mask.shape:
        # the reference checks this after the anchor checks; it can only fire when they pass
        doc_shape_error = True
    else:
        doc_shape_error = False
    device = loss_mask.device
    _require_gpu(loss_mask)
    anchors = anchors.to(device=device, dtype=torch.long).contiguous()
    keep_mask = keep_mask.to(device=device).contiguous()
    loss_mask_c = loss_mask.contiguous()
    docs = None
    if ctx_doc_ids is not None and not doc_shape_error:
        docs = ctx_doc_ids.to(device=device, dtype=torch.long).contiguous()
    with _timing.region("anchor_validate"):
        out = torch.empty_like(anchors)
        flags = torch.zeros(1, dtype=torch.int32, device=device)
        _lib.call("aspec_validate_injected_anchors", anchors.data_ptr(), keep_mask.data_ptr(),
                  loss_mask_c.data_ptr(), _lib.mask_dtype_code(loss_mask_c), _lib.ptr(docs),
                  expected[0], loss_mask.shape[1], num_anchors, block_size,
                  int(bool(allow_partial_last_target)), out.data_ptr(), flags.data_ptr(),
                  _lib.stream_handle(device))
    f = int(flags.item())
    if f & 1:
        raise ValueError("Kept injected anchors must have an in-bounds first prediction target")
    if not f & 8:
        return out, keep_mask
    if f & 2:
        raise ValueError("Kept injected anchors and their first targets must be supervised")
    if doc_shape_error:
        raise ValueError("ctx_doc_ids and loss_mask must have identical shapes")
    if f & 4:
        raise ValueError("Kept injected anchor blocks must not cross document boundaries")
    return out, keep_mask


def document_anchor_slots(document_lengths, num_anchors, block_size, alignment=1):
    """CPU-known structural bounds, padded only for CP anchor ownership (anchors.py:119-127)."""
    if min(num_anchors, block_size, alignment) < 1:
        raise ValueError("Anchor budget, block size and alignment must be positive")
    slots = tuple(min(num_anchors, max(length - block_size + 1, 0))
                  if length > block_size else 0 for length in document_lengths)
    total = sum(slots)
    padded = max(alignment, ((total + alignment - 1) // alignment) * alignment)
    return slots, total, padded


def sample_document_anchor_positions(
    loss_mask: torch.Tensor,
    ctx_doc_ids: torch.Tensor,
    document_lengths: tuple[int, ...],
    num_anchors: int,
    block_size: int,
    generator: Optional[torch.Generator] = None,
    alignment: int = 1,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """The native sampler applied independently to contiguous packed documents
    (anchors.py:130-194): one torch.rand draw per document, then one HIP kernel."""
    if (loss_mask.ndim != 2 or loss_mask.shape[0] != 1
            or ctx_doc_ids.shape != loss_mask.shape):
        raise ValueError("Document anchor sampling requires one packed row and aligned document IDs")
    if not document_lengths or any(length <= 0 for length in document_lengths):
        raise ValueError("Packed document lengths must be nonempty and positive")
    seq_len = loss_mask.shape[1]
    if sum(document_lengths) > seq_len:
        raise ValueError("Packed document lengths exceed the row")
    device = loss_mask.device
    n_docs = len(document_lengths)
    slot_counts, total_slots, padded_slots = document_anchor_slots(
        document_lengths, num_anchors, block_size, alignment
    )
    if total_slots == 0:
        return _empty(1, padded_slots, seq_len, block_size, device)
    _require_gpu(loss_mask, ctx_doc_ids)
    lengths = torch.tensor(document_lengths, device=device, dtype=torch.long)
    uniform = torch.rand(n_docs, device=device, generator=generator)
    mask = loss_mask.contiguous()
    docs = ctx_doc_ids.to(torch.long).contiguous()
    with _timing.region("anchor_sample"):
        workspace = torch.empty(seq_len, dtype=torch.int32, device=device)
        anchors = torch.empty(padded_slots, dtype=torch.long, device=device)
        keep = torch.empty(padded_slots, dtype=torch.bool, device=device)
        _lib.call("aspec_sample_document_anchors", mask.data_ptr(), _lib.mask_dtype_code(mask),
                  docs.data_ptr(), seq_len, lengths.data_ptr(), n_docs, num_anchors, block_size,
                  total_slots, padded_slots, uniform.data_ptr(), workspace.data_ptr(),
                  anchors.data_ptr(), keep.data_ptr(), _lib.stream_handle(device))
    return anchors.reshape(1, -1), keep.reshape(1, -1)


def sample_anchor_positions(
    seq_len: int,
    loss_mask: torch.Tensor,
    num_anchors: int,
    block_size: int,
    device: torch.device,
    max_gap: Optional[int] = None,
    generator: Optional[torch.Generator] = None,
    attention_mask: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sample anchor positions per sample; returns (anchors, keep_mask) (anchors.py:197-266)."""
    bsz = loss_mask.shape[0]
    if max(seq_len - block_size, 0) == 0:
        return _empty(bsz, num_anchors, seq_len, block_size, device)
    if max_gap is None:
        max_gap = block_size
    if attention_mask is not None and attention_mask.shape != loss_mask.shape:
        raise ValueError("Anchor attention_mask and loss_mask must have identical shapes")
    _require_gpu(loss_mask, attention_mask)
    uniform = torch.rand(bsz, 1, device=device, generator=generator)
    mask = loss_mask.contiguous()
    attn = attention_mask.contiguous() if attention_mask is not None else None
    with _timing.region("anchor_sample"):
        workspace = torch.empty(bsz, seq_len, dtype=torch.int32, device=mask.device)
        anchors = torch.empty(bsz, num_anchors, dtype=torch.long, device=mask.device)
        keep = torch.empty(bsz, num_anchors, dtype=torch.bool, device=mask.device)
        _lib.call("aspec_sample_anchors", mask.data_ptr(), _lib.mask_dtype_code(mask),
                  _lib.ptr(attn), _lib.mask_dtype_code(attn) if attn is not None else 0, bsz,
                  seq_len, num_anchors, block_size, max_gap, uniform.data_ptr(),
                  workspace.data_ptr(), anchors.data_ptr(), keep.data_ptr(),
                  _lib.stream_handle(mask.device))
    return anchors, keep
