"""Fused Q/K RMSNorm, split-K join and indexed RoPE for DSpark training (HIP).

Drop-in for `aspec.models.ops.dspark_qk_norm_rope` (aspec/models/ops/dspark_qk_norm_rope.py):
same function names, arguments, validation messages, outputs and saved state. The arithmetic is
`_prepare_dflash_qk` (aspec/models/draft/dflash.py:280-327) in fp32, rounded once to the
activation dtype, as the reference's fused kernel does; the weight gradients are fp32 and
deterministic. A position outside the cos/sin table gives NaN rows (the reference's eager path
would raise on the indexing) and is reported by `last_position_error()` after a synchronization.
"""

from __future__ import annotations

import ctypes
import os

import torch
from torch.autograd.function import once_differentiable

from . import _lib, _timing

_HEAD_DIM = 128


def dspark_qk_norm_rope_available() -> bool:
    """Whether the HIP library can serve the DSpark specialization (dspark_qk_norm_rope.py:43-50)."""
    if os.getenv("ASPEC_DISABLE_DSPARK_QK_KERNEL") == "1":
        return False
    try:
        _lib.load()
    except RuntimeError:
        return False
    return True


def _require_compact(name: str, tensor: torch.Tensor) -> None:
    if not tensor.is_contiguous():
        raise ValueError(
            f"{name} must be contiguous for the DSpark fused Q/K kernel, "
            f"got stride {tensor.stride()}"
        )


def _table(t: torch.Tensor) -> torch.Tensor:
    table = t.squeeze(0).squeeze(0)
    if table.ndim != 2 or table.shape[-1] < _HEAD_DIM:
        raise ValueError("cos/sin must be [1, 1, positions, head_dim] (or squeezable to 2D)")
    if table.stride(-1) != 1 or table.stride(0) % 4 != 0:
        raise ValueError("cos/sin rows must be contiguous and 8-byte aligned")
    return table


class _DSparkQkNormRope(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, context_key, draft_key, query_norm_weight, key_norm_weight, cos, sin,
                query_position_ids, context_position_ids, draft_position_ids, variance_epsilon,
                num_heads, num_kv_heads, head_dim):
        for name, tensor in (
            ("query", query),
            ("context_key", context_key),
            ("draft_key", draft_key),
            ("query_position_ids", query_position_ids),
            ("context_position_ids", context_position_ids),
            ("draft_position_ids", draft_position_ids),
        ):
            _require_compact(name, tensor)
        if query.device.type != "cuda":
            raise ValueError("the DSpark fused Q/K kernel requires CUDA tensors")
        if query.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"the DSpark fused Q/K kernel serves bf16/f16, got {query.dtype}")
        if context_key.dtype != query.dtype or draft_key.dtype != query.dtype:
            raise ValueError("query, context_key, and draft_key must share one dtype")
        if query_norm_weight.dtype != query.dtype or key_norm_weight.dtype != query.dtype:
            raise ValueError("Q/K norm weights must share the activation dtype")
        if head_dim != _HEAD_DIM:
            raise NotImplementedError(f"the HIP Q/K kernel serves head_dim {_HEAD_DIM}, got {head_dim}")

        batch, draft_len, query_width = query.shape
        context_len = int(context_key.shape[1])
        if tuple(draft_key.shape[:2]) != (batch, draft_len):
            raise ValueError("draft_key must share query batch and draft length")
        if int(context_key.shape[0]) != batch:
            raise ValueError("context_key must share the query batch")
        if query_width != num_heads * head_dim:
            raise ValueError("query width does not match num_heads * head_dim")
        if (
            int(context_key.shape[2]) != num_kv_heads * head_dim
            or int(draft_key.shape[2]) != num_kv_heads * head_dim
        ):
            raise ValueError("K width does not match num_kv_heads * head_dim")
        for name, ids, length in (("query_position_ids", query_position_ids, draft_len),
                                  ("context_position_ids", context_position_ids, context_len),
                                  ("draft_position_ids", draft_position_ids, draft_len)):
            if ids.dtype != torch.int64 or ids.numel() != batch * length or ids.device != query.device:
                raise ValueError(f"{name} must be int64 [batch, length] on the query device")
        cos_2d, sin_2d = _table(cos), _table(sin)
        if cos_2d.shape != sin_2d.shape or cos_2d.dtype != query.dtype or sin_2d.dtype != query.dtype:
            raise ValueError("cos and sin must share one shape and the activation dtype")
        for w in (query_norm_weight, key_norm_weight):
            if w.numel() != head_dim or not w.is_contiguous() or w.device != query.device:
                raise ValueError("Q/K norm weights must be contiguous [head_dim] on the query device")

        dev = query.device
        query_out = torch.empty(batch * draft_len, num_heads, head_dim, device=dev, dtype=query.dtype)
        key_out = torch.empty(batch * (context_len + draft_len), num_kv_heads, head_dim, device=dev,
                              dtype=query.dtype)
        rstd_q = torch.empty(batch * draft_len, num_heads, device=dev, dtype=torch.float32)
        rstd_k = torch.empty(batch * (context_len + draft_len), num_kv_heads, device=dev,
                             dtype=torch.float32)
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        with _timing.region("qk_norm_rope_fwd"):
            _lib.call("aspec_qk_norm_rope_fwd", query.data_ptr(), context_key.data_ptr(),
                      draft_key.data_ptr(), query_norm_weight.data_ptr(), key_norm_weight.data_ptr(),
                      cos_2d.data_ptr(), sin_2d.data_ptr(), cos_2d.shape[0], cos_2d.stride(0),
                      query_position_ids.data_ptr(), context_position_ids.data_ptr(),
                      draft_position_ids.data_ptr(), batch, context_len, draft_len, num_heads,
                      num_kv_heads, head_dim, float(variance_epsilon), _lib.mask_dtype_code(query),
                      query_out.data_ptr(), key_out.data_ptr(), rstd_q.data_ptr(), rstd_k.data_ptr(),
                      flags.data_ptr(), _lib.stream_handle(dev))
        global _last_flags
        _last_flags = flags
        ctx.save_for_backward(query, context_key, draft_key, query_norm_weight, key_norm_weight,
                              cos_2d, sin_2d, query_position_ids, context_position_ids,
                              draft_position_ids, rstd_q, rstd_k)
        ctx.sizes = (batch, context_len, draft_len, num_heads, num_kv_heads, head_dim)
        ctx.variance_epsilon = float(variance_epsilon)
        return (query_out.view(batch, draft_len, num_heads, head_dim),
                key_out.view(batch, context_len + draft_len, num_kv_heads, head_dim))

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_query, grad_key):
        (query, context_key, draft_key, query_norm_weight, key_norm_weight, cos, sin, position_q,
         position_context, position_draft, rstd_q, rstd_k) = ctx.saved_tensors
        batch, context_len, draft_len, num_heads, num_kv_heads, head_dim = ctx.sizes
        dev = query.device
        if grad_query is None:
            grad_query = torch.zeros(batch, draft_len, num_heads, head_dim, device=dev, dtype=query.dtype)
        if grad_key is None:
            grad_key = torch.zeros(batch, context_len + draft_len, num_kv_heads, head_dim, device=dev,
                                   dtype=query.dtype)
        grad_query = grad_query.to(query.dtype).contiguous()
        grad_key = grad_key.to(query.dtype).contiguous()
        out_query = torch.empty_like(query)
        out_context_key = torch.empty_like(context_key)
        out_draft_key = torch.empty_like(draft_key)
        dw_q = torch.empty(head_dim, device=dev, dtype=torch.float32)
        dw_k = torch.empty_like(dw_q)
        size = ctypes.c_size_t()
        _lib.call("aspec_qk_norm_rope_bwd_workspace_bytes", batch, context_len, draft_len, num_heads,
                  num_kv_heads, ctypes.byref(size))
        workspace = torch.empty(size.value, dtype=torch.uint8, device=dev)
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        with _timing.region("qk_norm_rope_bwd"):
            _lib.call("aspec_qk_norm_rope_bwd", grad_query.data_ptr(), grad_key.data_ptr(),
                      query.data_ptr(), context_key.data_ptr(), draft_key.data_ptr(),
                      rstd_q.data_ptr(), rstd_k.data_ptr(), query_norm_weight.data_ptr(),
                      key_norm_weight.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
                      cos.stride(0), position_q.data_ptr(), position_context.data_ptr(),
                      position_draft.data_ptr(), batch, context_len, draft_len, num_heads,
                      num_kv_heads, head_dim, ctx.variance_epsilon, _lib.mask_dtype_code(query),
                      out_query.data_ptr(),
                      out_context_key.data_ptr(), out_draft_key.data_ptr(), dw_q.data_ptr(),
                      dw_k.data_ptr(), workspace.data_ptr(), flags.data_ptr(),
                      _lib.stream_handle(dev))
        return (out_query, out_context_key, out_draft_key, dw_q, dw_k, None, None, None, None, None,
                None, None, None, None)


_last_flags = None


def last_position_error() -> bool:
    """True when the last forward met a position outside the cos/sin table (synchronizes)."""
    return bool(_last_flags is not None and int(_last_flags.item()) != 0)


def dspark_qk_norm_rope(query, context_key, draft_key, query_norm_weight, key_norm_weight,
                        variance_epsilon, cos, sin, query_position_ids, context_position_ids,
                        draft_position_ids, num_heads, num_kv_heads, head_dim):
    """Fused Q/K RMSNorm, split-K join and indexed RoPE for DSpark training
    (dspark_qk_norm_rope.py:401-434): returns q [B, Ld, Hq, D] and k [B, Lc + Ld, Hkv, D]."""
    return _DSparkQkNormRope.apply(query, context_key, draft_key, query_norm_weight,
                                   key_norm_weight, cos, sin, query_position_ids,
                                   context_position_ids, draft_position_ids, variance_epsilon,
                                   num_heads, num_kv_heads, head_dim)
