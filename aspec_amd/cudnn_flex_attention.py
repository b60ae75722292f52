"""cuDNN FlexAttention drop-in on MI355X (aspec/models/ops/cudnn_flex_attention.py).

`build_dspark_mla_mask`, `CudnnFlexMask`, `cudnn_flex_attention` and `resolve_cudnn_gqa_mode` keep
the reference's names, arguments and exceptions; the Draft model's call sites
(aspec/models/dflash.py:732-745 builds the mask, aspec/models/draft/dflash.py:932-942 attends)
work unchanged.

- The interval-union mask (`mask_func`, int32 [1, E, rows]) is built by a HIP kernel
  (`aspec_dspark_mla_mask`). Once per mask and Q/K/V geometry, `CudnnFlexMask.plan_for` turns it
  into the attention kernels' two-interval endpoints (`aspec_flex_mask_intervals`) and tile plan
  (`aspec_dspark_plan_build`), cached on the mask as the reference caches its cuDNN plans.
- BSHD [B, L, H, D] and THD [T, H, D] (with cu_seqlens) inputs run as ONE flattened key space:
  the rows of sequence b see only b's keys, so one forward and one backward launch serve the whole
  batch without per-sequence copies.
- GQA: the kernels reduce the query heads of each KV group inside the workgroup (joint GQA), so
  every `gqa_mode` and `physical_gqa` runs the same kernels; the reference's query-head folding is
  a cuDNN layout choice with no counterpart here and does not change the result.
- Computed in bf16 or fp16 (fp32 accumulation) with head_dim 128. The materialised-MLA
  (Dqk, Dv) = (192, 128) shape raises NotImplementedError. Rows without a visible key return O = 0
  and LSE = -1e30, the convention of the Direct-CP path (direct_cp.py:470-477).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Any

import torch

from aspec_amd import _lib, _timing
from aspec_amd.direct_cp import _DSparkAttention

_SUPPORTED_HEAD_DIMS = {(128, 128), (192, 128)}

__all__ = ["CudnnFlexMask", "build_dspark_mla_mask", "cudnn_flex_attention", "resolve_cudnn_gqa_mode"]


def build_dspark_mla_mask(*, anchor_positions: torch.Tensor, block_keep_mask: torch.Tensor,
                          context_length: int, block_size: int, is_causal: bool = False,
                          sliding_window: int | None = None, context_window: int | None = None,
                          ctx_doc_ids: torch.Tensor | None = None) -> "CudnnFlexMask":
    """Exact interval endpoints of the DSpark context + draft mask (cudnn_flex_attention.py:53-170):
    three per row, [0, anchor) U [draft_begin, draft_end), without documents and windows; five,
    [0, 0) U [context_begin, anchor) U [draft_begin, draft_end), otherwise; zeros for dropped
    blocks. Built on the GPU; one host read of the validation flags, as the reference's checks."""
    if anchor_positions.ndim != 2 or block_keep_mask.shape != anchor_positions.shape:
        raise ValueError("anchor_positions and block_keep_mask must have identical [batch, anchors] shapes")
    if anchor_positions.device != block_keep_mask.device:
        raise ValueError("anchor_positions and block_keep_mask must be on the same device")
    if context_length <= 0:
        raise ValueError(f"context_length must be positive, got {context_length}")
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError(f"sliding_window must be positive, got {sliding_window}")
    if ctx_doc_ids is not None:
        expected = (anchor_positions.shape[0], context_length)
        if ctx_doc_ids.shape != expected:
            raise ValueError(f"ctx_doc_ids must have shape {expected}, got {ctx_doc_ids.shape}")
        if ctx_doc_ids.device != anchor_positions.device:
            raise ValueError("ctx_doc_ids and anchor_positions must be on the same device")
    device = anchor_positions.device
    if device.type != "cuda":
        raise ValueError("aspec_amd builds DSpark masks on the GPU; got CPU anchors")
    window_error = context_window is not None and (
        isinstance(context_window, bool) or not isinstance(context_window, int) or context_window <= 0)
    batch, num_anchors = anchor_positions.shape
    anchors = anchor_positions.to(torch.int64).contiguous()
    keep = block_keep_mask.to(torch.bool).contiguous()
    docs = None if ctx_doc_ids is None else ctx_doc_ids.to(torch.int64).contiguous()
    ends = 3 if (ctx_doc_ids is None and sliding_window is None and context_window is None) else 5
    mask_func = torch.empty((1, ends, batch * num_anchors * block_size), dtype=torch.int32, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    workspace = None
    if docs is not None:
        size = ctypes.c_size_t()
        _lib.call("aspec_dspark_mla_mask_workspace_bytes", batch, context_length, ctypes.byref(size))
        workspace = torch.empty(size.value, dtype=torch.uint8, device=device)
    with _timing.region("dspark_mla_mask"):
        _lib.call("aspec_dspark_mla_mask", _lib.ptr(anchors), _lib.ptr(keep), _lib.ptr(docs), batch,
                  num_anchors, block_size, context_length, int(bool(is_causal)), sliding_window or 0,
                  0 if (window_error or context_window is None) else context_window,
                  _lib.ptr(mask_func), _lib.ptr(workspace), _lib.ptr(flags), _lib.stream_handle(device))
    bad = int(flags.item())
    if bad & 1:
        raise ValueError("anchor_positions must lie inside the context sequence")
    if bad & 2:
        raise ValueError("ctx_doc_ids must contain each document in one contiguous run")
    if window_error:
        raise ValueError("context_window must be a positive integer or null")
    return CudnnFlexMask(mask_func=mask_func)


@dataclass
class _FlexPlan:
    """The attention kernels' view of one mask at one Q/K/V geometry."""

    endpoints: torch.Tensor  # int32 [5, rows] in the flattened key space
    plan: torch.Tensor       # opaque tile plan (aspec_dspark_plan_build)
    num_queries: int
    num_keys: int


@dataclass
class CudnnFlexMask:
    """Per-step endpoints plus per-geometry reusable kernel plans (cudnn_flex_attention.py:173-321)."""

    mask_func: torch.Tensor
    pack_gqa: bool | None = None
    fwd_variant: str | None = None
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int | None = None
    max_seqlen_k: int | None = None
    # Constructor-visible so that dataclasses.replace() keeps sharing the caches, excluded from
    # repr and equality (the reference's graph / FSDP plumbing relies on both).
    _plans: dict[tuple[Any, ...], Any] = field(default_factory=dict, repr=False, compare=False)
    _physical_gqa_masks: dict[tuple[Any, ...], "CudnnFlexMask"] = field(
        default_factory=dict, repr=False, compare=False)
    _joint_backward_plans: dict[tuple[Any, ...], Any] = field(default_factory=dict, repr=False, compare=False)

    def __post_init__(self) -> None:
        varlen = (self.cu_seqlens_q, self.cu_seqlens_k, self.max_seqlen_q, self.max_seqlen_k)
        if any(v is not None for v in varlen) and not all(v is not None for v in varlen):
            raise ValueError("cuDNN THD masks require both cumulative lengths and both maxima")

    def for_physical_gqa(self, ratio: int) -> "CudnnFlexMask":
        """The mask of the query-head-folded layout (each query row repeated `ratio` times), as the
        reference derives it for cuDNN's physical GQA. The HIP kernels never need it: they reduce
        the GQA group themselves."""
        if ratio < 1:
            raise ValueError("physical GQA ratio must be positive")
        if ratio == 1:
            return self
        if self.mask_func.shape[0] != 1:
            raise ValueError("physical GQA folding requires a head-independent mask")
        key = (ratio, self.mask_func.data_ptr(), self.mask_func._version, tuple(self.mask_func.shape),
               tuple(self.mask_func.stride()), self.fwd_variant,
               _tensor_identity(self.cu_seqlens_q), _tensor_identity(self.cu_seqlens_k),
               self.max_seqlen_q, self.max_seqlen_k)
        physical = self._physical_gqa_masks.get(key)
        if physical is None:
            physical = CudnnFlexMask(
                mask_func=self.mask_func.repeat_interleave(ratio, dim=-1).contiguous(),
                pack_gqa=False, fwd_variant=self.fwd_variant,
                cu_seqlens_q=None if self.cu_seqlens_q is None else self.cu_seqlens_q * ratio,
                cu_seqlens_k=self.cu_seqlens_k,
                max_seqlen_q=None if self.max_seqlen_q is None else self.max_seqlen_q * ratio,
                max_seqlen_k=self.max_seqlen_k)
            self._physical_gqa_masks[key] = physical
        return physical

    def _plan_key(self, q, k, v, pack_gqa) -> tuple[Any, ...]:
        m = self.mask_func
        return (m.device, m.dtype, tuple(m.shape), tuple(m.stride()), m.data_ptr(), m._version,
                q.device, q.dtype, tuple(q.shape), tuple(k.shape), tuple(v.shape), tuple(q.stride()),
                tuple(k.stride()), tuple(v.stride()), pack_gqa, self.fwd_variant,
                _tensor_identity(self.cu_seqlens_q), _tensor_identity(self.cu_seqlens_k),
                self.max_seqlen_q, self.max_seqlen_k)

    def plan_for(self, q, k, v, *, pack_gqa: bool | None = None, build_backward: bool = True) -> _FlexPlan:
        """Endpoints and tile plan of this mask for Q/K/V of these shapes, built once (two integer
        kernels, one host read of their validation flags) and reused while the mask is unchanged."""
        effective_pack_gqa = self.pack_gqa if pack_gqa is None else pack_gqa
        key = self._plan_key(q, k, v, effective_pack_gqa) + (build_backward,)
        plan = self._plans.get(key)
        if plan is not None:
            return plan
        plan = _build_plan(self, q, k)
        self._plans[key] = plan
        return plan


def _tensor_identity(t):
    return None if t is None else (t.data_ptr(), t._version)


def _build_plan(mask: CudnnFlexMask, q, k) -> _FlexPlan:
    device = q.device
    m = mask.mask_func
    if m.ndim != 3:
        raise ValueError("mask_func must be [heads, endpoints, query rows]")
    if m.shape[0] != 1:
        raise NotImplementedError("per-head interval masks are not supported by the DSpark kernels")
    rows = m.shape[2]
    if q.ndim == 4:
        batch, lq = q.shape[0], q.shape[1]
        nq, nk, lk = batch * lq, batch * k.shape[1], k.shape[1]
        cu_q = cu_k = None
        segments = 0
    else:
        nq, nk = q.shape[0], k.shape[0]
        lq = lk = 0
        cu_q = mask.cu_seqlens_q.to(device=device, dtype=torch.int32).contiguous()
        cu_k = mask.cu_seqlens_k.to(device=device, dtype=torch.int32).contiguous()
        if cu_q.ndim != 1 or cu_q.shape != cu_k.shape or cu_q.numel() < 2:
            raise ValueError("cu_seqlens_q and cu_seqlens_k must be [segments + 1] vectors")
        segments = cu_q.numel() - 1
    if rows != nq:
        raise ValueError(f"the mask has {rows} query rows but the queries have {nq}")
    endpoints = torch.empty((5, nq), dtype=torch.int32, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    stream = _lib.stream_handle(device)
    rows_i32 = m[0].to(torch.int32).contiguous()
    with _timing.region("flex_mask_intervals"):
        _lib.call("aspec_flex_mask_intervals", _lib.ptr(rows_i32), m.shape[1], nq, _lib.ptr(cu_q),
                  _lib.ptr(cu_k), segments, lq, lk, _lib.ptr(endpoints), _lib.ptr(flags), stream)
    if cu_q is not None:
        bad, q_total, k_total = torch.cat((flags, cu_q[-1:], cu_k[-1:])).tolist()
        if q_total != nq or k_total != nk:
            raise ValueError("cu_seqlens must end at the THD query and key token counts")
    else:
        bad = int(flags.item())
    if bad & 1:
        raise ValueError("interval mask endpoints must lie inside their sequence's keys")
    if bad & 4:
        raise ValueError("every THD query row must lie inside cu_seqlens_q")
    if bad & 2:
        raise NotImplementedError(
            "a query row sees more than two disjoint key intervals; the DSpark kernels take two")
    size = ctypes.c_size_t()
    _lib.call("aspec_dspark_plan_bytes", nq, nk, ctypes.byref(size))
    plan = torch.empty(size.value, dtype=torch.uint8, device=device)
    with _timing.region("attn_plan_build"):
        _lib.call("aspec_dspark_plan_build", _lib.ptr(endpoints), nq, nk, _lib.ptr(plan), stream)
    return _FlexPlan(endpoints, plan, nq, nk)


def resolve_cudnn_gqa_mode(mode: str, *, physical_gqa: bool = False) -> str:
    """The execution policy name (cudnn_flex_attention.py:324-328); all of them run the same
    joint-GQA HIP kernels here."""
    if mode not in {"auto", "native", "external", "internal"}:
        raise ValueError(f"Unsupported cuDNN GQA mode: {mode!r}")
    return ("external" if physical_gqa else "native") if mode == "auto" else mode


def cudnn_flex_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *,
                         mask: CudnnFlexMask, scale: float, pack_gqa: bool | None = None,
                         physical_gqa: bool = False, gqa_mode: str = "auto", return_lse: bool = False):
    """Masked attention over BSHD [B, L, H, D] or THD [T, H, D] Q/K/V with an interval-union mask
    (cudnn_flex_attention.py:331-440): output in the query's layout and, with return_lse, the
    natural-log LSE ([B, Hq, Lq] for BSHD, [Hq, T] for THD). Autograd to Q, K and V (and through
    the LSE)."""
    if not isinstance(mask, CudnnFlexMask):
        raise TypeError("cudnn_flex_attention requires a CudnnFlexMask")
    if not (query.is_cuda and key.is_cuda and value.is_cuda):
        raise ValueError("cudnn_flex_attention requires CUDA Q/K/V tensors")
    if query.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("cudnn_flex_attention requires FP16 or BF16 Q/K/V tensors")
    if query.dtype != key.dtype or query.dtype != value.dtype:
        raise TypeError("Q/K/V must have the same dtype")
    if query.ndim not in (3, 4) or key.ndim != query.ndim or value.ndim != query.ndim:
        raise ValueError("Q/K/V must all be rank-4 BSHD or rank-3 THD tensors")
    if query.ndim == 4:
        if query.shape[0] != key.shape[0] or key.shape[:3] != value.shape[:3]:
            raise ValueError("Q/K/V batch, KV sequence, and KV head shapes must agree")
        query_heads, key_heads = query.shape[2], key.shape[2]
    else:
        if mask.cu_seqlens_q is None:
            raise ValueError("rank-3 THD Q/K/V require cumulative sequence lengths")
        if key.shape[:2] != value.shape[:2]:
            raise ValueError("THD K/V token and head shapes must agree")
        query_heads, key_heads = query.shape[1], key.shape[1]
    if query_heads % key_heads:
        raise ValueError("the number of query heads must be divisible by KV heads")
    if query.shape[-1] != key.shape[-1]:
        raise ValueError("Q and K must have the same head dimension")
    dims = (query.shape[-1], value.shape[-1])
    if dims not in _SUPPORTED_HEAD_DIMS:
        raise ValueError("the ASpec cuDNN path currently supports (Dqk,Dv)=(128,128) "
                         f"for GQA and (192,128) for materialized MLA; got {dims}")
    if dims == (192, 128) and query_heads != key_heads:
        raise ValueError("materialized MLA currently requires Hq=Hkv")
    resolve_cudnn_gqa_mode(gqa_mode, physical_gqa=physical_gqa)
    if dims != (128, 128):
        raise NotImplementedError("materialized MLA (Dqk=192) is outside the DSpark GQA kernels of this build")
    plan = mask.plan_for(query, key, value, pack_gqa=pack_gqa)
    if query.ndim == 4:
        batch, lq = query.shape[:2]
        flat = [t.reshape(t.shape[0] * t.shape[1], t.shape[2], t.shape[3]) for t in (query, key, value)]
    else:
        flat = [query, key, value]
    q4, k4, v4 = (t[None].transpose(1, 2) for t in flat)  # [1, H, tokens, D] views
    out4, lse3 = _DSparkAttention.apply(q4, k4, v4, plan.endpoints, plan.plan, float(scale))
    out = out4.transpose(1, 2)[0]  # [rows, Hq, D], token-major storage
    lse = lse3[0]                  # [Hq, rows]
    if query.ndim == 4:
        out = out.view(batch, lq, query_heads, value.shape[-1])
        lse = lse.view(query_heads, batch, lq).permute(1, 0, 2).contiguous()
    return (out, lse) if return_lse else out
