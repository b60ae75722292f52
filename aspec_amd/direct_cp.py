"""Direct-CP / THD DSpark attention on MI355X (context-parallel degree 1 end to end).

Mirrors the operator surface of aspec/models/ops/direct_cp.py: `DirectCPMetadata` (147-262),
`direct_cp_attention_from_kv` (1047-1100), `direct_cp_attention` (1027-1044),
`build_context_positions` (23-53), `merge_attention_partials` (362-367) and
`direct_cp_attention_observation` (265-284). Every GPU backend name the reference accepts ("auto",
"fa4", "cudnn_flex_attention") and "hip" run the same HIP kernels; the reference's CPU "math"
backend is not part of this product. With cp_size > 1 one rank's share of the work (all gathered
queries against its context shard and its own draft blocks) runs through
`direct_cp_partial_attention`; the collectives around it need several GPUs.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch
from torch import Tensor

from aspec_amd import _lib, _timing

MASK_VALUE = -1.0e30  # direct_cp.py:20

_GPU_BACKENDS = {"auto", "hip", "fa4", "cudnn_flex_attention"}
_GQA_MODES = {"auto", "native", "external", "internal"}


def build_context_positions(total_positions: int, cp_rank: int, cp_size: int, *,
                            layout: str = "contiguous", alignment: int = 1) -> Tensor:
    """Positions owned by one CP rank (direct_cp.py:23-53): a contiguous shard
    (`context_shard_bounds`, aligned groups), or for "zigzag" the chunks cp_rank and
    2*cp_size - 1 - cp_rank of 2*cp_size equal chunks."""
    if total_positions < 0 or cp_size <= 0 or not 0 <= cp_rank < cp_size:
        raise ValueError("invalid context-parallel position layout")
    if layout not in {"contiguous", "zigzag"}:
        raise ValueError(f"unsupported context-parallel layout: {layout}")
    if layout == "contiguous" or cp_size == 1:
        from aspec_amd.collate import context_shard_bounds

        start, end = context_shard_bounds(total_positions, cp_rank, cp_size, alignment=alignment)
        return torch.arange(start, end, dtype=torch.long)
    if alignment != 1:
        raise ValueError("zigzag context ownership does not support aligned groups")
    chunks = 2 * cp_size
    owned = []
    for chunk_rank in (cp_rank, chunks - 1 - cp_rank):
        start = total_positions * chunk_rank // chunks
        end = total_positions * (chunk_rank + 1) // chunks
        owned.append(torch.arange(start, end, dtype=torch.long))
    return torch.cat(owned)


class _ForwardSparseCache:
    """Per-forward integer metadata shared by all layers (direct_cp.py:124-145): row metadata,
    endpoints and the attention plan live here, never across forwards."""

    def __init__(self):
        self._entries = {}
        self.thd_inputs = {}

    def get(self, key):
        return self._entries.get(key)

    def __setitem__(self, key, value):
        self._entries[key] = value

    def values(self):
        return self._entries.values()


@dataclass
class DirectCPMetadata:
    """Replicated mask metadata plus this rank's context and query ownership (direct_cp.py:147-245)."""

    anchor_positions: Tensor
    block_keep_mask: Tensor
    context_position_ids: Tensor
    block_size: int
    cp_rank: int
    cp_size: int
    group: Optional[object]
    context_doc_ids: Optional[Tensor] = None
    anchor_doc_ids: Optional[Tensor] = None
    context_rope_position_ids: Optional[Tensor] = None
    sequence_length: Optional[int] = None
    backend: str = "fa4"
    layout: str = "contiguous"
    fa4_sparse: bool = True
    context_window: Optional[int] = None
    query_window: Optional[int] = None
    draft_is_causal: bool = False
    _fa4_cache: _ForwardSparseCache = field(default_factory=_ForwardSparseCache, repr=False)
    attention_observation: dict = field(default_factory=dict, repr=False)

    def __post_init__(self) -> None:
        if self.anchor_positions.ndim != 2 or self.block_keep_mask.ndim != 2:
            raise ValueError("anchor_positions and block_keep_mask must be [batch, blocks]")
        if self.anchor_positions.shape != self.block_keep_mask.shape:
            raise ValueError("anchor_positions and block_keep_mask shapes must match")
        if self.context_position_ids.ndim != 2:
            raise ValueError("context_position_ids must be [batch, local_context]")
        if self.context_position_ids.shape[0] != self.anchor_positions.shape[0]:
            raise ValueError("context and anchor batches must match")
        if (self.context_doc_ids is None) != (self.anchor_doc_ids is None):
            raise ValueError("context_doc_ids and anchor_doc_ids must be provided together")
        if self.context_doc_ids is not None:
            if self.context_doc_ids.shape != self.context_position_ids.shape:
                raise ValueError("context_doc_ids must match context_position_ids")
            if self.anchor_doc_ids.shape != self.anchor_positions.shape:
                raise ValueError("anchor_doc_ids must match anchor_positions")
        if (self.context_rope_position_ids is not None
                and self.context_rope_position_ids.shape != self.context_position_ids.shape):
            raise ValueError("context_rope_position_ids must match context_position_ids")
        for name in ("context_window", "query_window"):
            value = getattr(self, name)
            if value is not None and (isinstance(value, bool) or not isinstance(value, int) or value <= 0):
                raise ValueError(f"{name} must be a positive integer or null")
        if not isinstance(self.draft_is_causal, bool):
            raise ValueError("draft_is_causal must be boolean")
        if self.block_size <= 0 or self.cp_size <= 0:
            raise ValueError("block_size and cp_size must be positive")
        if self.sequence_length is not None and self.sequence_length <= 0:
            raise ValueError("sequence_length must be positive")
        if not 0 <= self.cp_rank < self.cp_size:
            raise ValueError("invalid CP rank")
        if self.layout not in {"contiguous", "zigzag"}:
            raise ValueError(f"unsupported context-parallel layout: {self.layout}")
        divisor = 1 if self.cp_size == 1 else (self.cp_size if self.layout == "contiguous" else 2 * self.cp_size)
        if self.num_blocks % divisor != 0:
            raise ValueError(f"direct CP requires num_blocks divisible by {divisor} for {self.layout}")
        if self.backend not in _GPU_BACKENDS | {"math"}:
            raise ValueError(f"unsupported direct CP backend: {self.backend}")
        if self.cp_size > 1 and self.group is None:
            raise ValueError("a process group is required when cp_size > 1")

    @property
    def num_blocks(self) -> int:
        return self.anchor_positions.shape[1]

    @property
    def blocks_per_rank(self) -> int:
        return self.num_blocks // self.cp_size

    @property
    def queries_per_rank(self) -> int:
        return self.blocks_per_rank * self.block_size

    @property
    def context_length(self) -> int:
        return self.context_position_ids.shape[1]

    @property
    def local_block_ids(self) -> Tensor:
        """The blocks whose draft keys this rank holds (direct_cp.py:248-252)."""
        return build_context_positions(self.num_blocks, self.cp_rank, self.cp_size, layout=self.layout)

    @property
    def collective_block_ids(self) -> Tensor:
        """Every rank's local blocks in rank order: the order of the gathered queries
        (direct_cp.py:255-262)."""
        return torch.cat([build_context_positions(self.num_blocks, rank, self.cp_size, layout=self.layout)
                          for rank in range(self.cp_size)])


def direct_cp_attention_observation(metadata: DirectCPMetadata) -> dict:
    """Forward-scoped observation shared across metadata copies (direct_cp.py:265-284)."""
    key = ("attention_observation", metadata.backend, metadata.context_window,
           metadata.query_window, metadata.draft_is_causal)
    observation = metadata._fa4_cache.get(key)
    if observation is None:
        observation = metadata.attention_observation
        metadata._fa4_cache[key] = observation
    return observation


# ---------------------------------------------------------------------------------------------
# Integer metadata (HIP): THD mask tensors, interval endpoints and the attention plan.
# ---------------------------------------------------------------------------------------------
class ThdRows:
    """Device-resident row metadata of one forward: query_aux [4, B*Nq], key_aux [4, B*K] (int32),
    endpoints [5, B*Nq] (int32, flattened key space: batch row b owns keys b*K .. b*K + K - 1) and
    the layout status flags. num_queries / num_keys count all batch rows."""

    def __init__(self, query_aux, key_aux, endpoints, flags, num_queries, num_keys, batch=1):
        self.query_aux = query_aux
        self.key_aux = key_aux
        self.endpoints = endpoints
        self.flags = flags
        self.num_queries = num_queries
        self.num_keys = num_keys
        self.batch = batch
        self._checked = False

    def check_layout(self) -> None:
        """Fail closed on layouts the interval form cannot represent (one host sync per forward,
        as the reference's monotonic check at direct_cp.py:776-780)."""
        if self._checked:
            return
        bad = int(self.flags.item())
        if bad & 1:
            raise ValueError("THD attention requires monotonically ordered context positions")
        if bad & 2:
            raise ValueError("THD attention requires contiguous ascending documents (padding last)")
        self._checked = True


def thd_row_metadata(metadata: DirectCPMetadata, device) -> ThdRows:
    """HIP `aspec_thd_batch_row_metadata`: `_query_metadata` / `_key_metadata`
    (thd_attention.py:25-56) and `_build_cudnn_thd_mask` (direct_cp.py:750-900) for every batch
    row at once, cached per forward. Batch > 1 is served for unpacked rows on every backend and
    for packed rows on the cuDNN / HIP backends; packed rows on the FA4 path keep the reference's
    one-row rule (thd_attention.py:141-142)."""
    device = torch.device(device)
    key = ("hip_thd_rows", device)
    rows = metadata._fa4_cache.thd_inputs.get(key)
    if rows is not None:
        return rows
    batch = metadata.anchor_positions.shape[0]
    if batch != 1 and metadata.context_doc_ids is not None and metadata.backend in {"fa4", "auto"}:
        raise ValueError("THD packing requires one controller-owned row per microbatch")
    if metadata.cp_size != 1:
        raise NotImplementedError("context parallelism > 1 needs several GPUs; this build is CP=1")
    n, block, T = metadata.num_blocks, metadata.block_size, metadata.context_length
    nq, nk = n * block, T + n * block
    anchors = metadata.anchor_positions.to(device=device, dtype=torch.int64).contiguous()
    keep = metadata.block_keep_mask.to(device=device, dtype=torch.bool).contiguous()
    positions = metadata.context_position_ids.to(device=device, dtype=torch.int64).contiguous()
    if metadata.context_doc_ids is None:
        # Unpacked rows: one document each (the reference's packed=False mask, direct_cp.py:540-545).
        anchor_docs = torch.zeros((batch, n), dtype=torch.int64, device=device)
        context_docs = torch.zeros((batch, T), dtype=torch.int64, device=device)
    else:
        anchor_docs = metadata.anchor_doc_ids.to(device=device, dtype=torch.int64).contiguous()
        context_docs = metadata.context_doc_ids.to(device=device, dtype=torch.int64).contiguous()
    query_aux = torch.empty((4, batch * nq), dtype=torch.int32, device=device)
    key_aux = torch.empty((4, batch * nk), dtype=torch.int32, device=device)
    endpoints = torch.empty((5, batch * nq), dtype=torch.int32, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    seq = metadata.sequence_length if metadata.sequence_length is not None else 0
    with _timing.region("thd_row_metadata"):
        _lib.call(
            "aspec_thd_batch_row_metadata", _lib.ptr(anchors), _lib.ptr(keep), _lib.ptr(anchor_docs),
            _lib.ptr(positions), _lib.ptr(context_docs), batch, n, block, T, seq,
            metadata.context_window or 0, metadata.query_window or 0, int(metadata.draft_is_causal),
            _lib.ptr(query_aux), _lib.ptr(key_aux), _lib.ptr(endpoints), _lib.ptr(flags),
            _lib.stream_handle(device),
        )
    rows = ThdRows(query_aux, key_aux, endpoints, flags, batch * nq, batch * nk, batch)
    metadata._fa4_cache.thd_inputs[key] = rows
    return rows


def attention_plan(metadata: DirectCPMetadata, rows: ThdRows, device) -> Tensor:
    """HIP `aspec_dspark_plan_build`: the tile lists of the attention kernels, once per forward."""
    key = ("hip_attention_plan", torch.device(device))
    plan = metadata._fa4_cache.get(key)
    if plan is not None:
        return plan
    import ctypes

    size = ctypes.c_size_t()
    _lib.call("aspec_dspark_plan_bytes", rows.num_queries, rows.num_keys, ctypes.byref(size))
    plan = torch.empty(size.value, dtype=torch.uint8, device=device)
    with _timing.region("attn_plan_build"):
        _lib.call("aspec_dspark_plan_build", _lib.ptr(rows.endpoints), rows.num_queries,
                  rows.num_keys, _lib.ptr(plan), _lib.stream_handle(device))
    metadata._fa4_cache[key] = plan
    return plan


# ---------------------------------------------------------------------------------------------
# Attention (HIP forward / backward behind autograd)
# ---------------------------------------------------------------------------------------------
def _thd_view(x: Tensor) -> Tensor:
    """A [1, H, L, D] tensor whose rows the kernels can address: unit stride on D, 16-byte aligned
    rows. Token-major ([1, L, H, D] storage) and head-major views both qualify as is."""
    ok = (x.stride(3) == 1 and x.data_ptr() % 16 == 0
          and x.stride(1) % 8 == 0 and x.stride(2) % 8 == 0)
    return x if ok else x.transpose(1, 2).contiguous().transpose(1, 2)


class _DSparkAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, key, value, endpoints, plan, scale):
        q, k, v = _thd_view(query), _thd_view(key), _thd_view(value)
        _, hq, nq, d = q.shape
        hkv, nk = k.shape[1], k.shape[2]
        out = torch.empty((1, nq, hq, v.shape[-1]), dtype=q.dtype, device=q.device)
        lse = torch.empty((1, hq, nq), dtype=torch.float32, device=q.device)
        with _timing.region("attn_fwd"):
            _lib.call(
                "aspec_dspark_attn_fwd",
                _lib.ptr(q), q.stride(2), q.stride(1), _lib.ptr(k), k.stride(2), k.stride(1),
                _lib.ptr(v), v.stride(2), v.stride(1), _lib.ptr(endpoints), _lib.ptr(plan),
                nq, nk, hq, hkv, d, float(scale), _lib.ptr(out), out.stride(1), out.stride(2),
                _lib.ptr(lse), _lib.mask_dtype_code(q), _lib.stream_handle(q.device),
            )
        ctx.save_for_backward(q, k, v, out, lse, endpoints, plan)
        ctx.scale = float(scale)
        ctx.set_materialize_grads(False)
        return out.transpose(1, 2), lse

    @staticmethod
    def backward(ctx, dout, dlse):
        import ctypes

        q, k, v, out, lse, endpoints, plan = ctx.saved_tensors
        _, hq, nq, d = q.shape
        hkv, nk = k.shape[1], k.shape[2]
        if dout is None:
            dout = torch.zeros((1, hq, nq, d), dtype=q.dtype, device=q.device)
        dout = _thd_view(dout.to(q.dtype))
        dlse_c = None if dlse is None else dlse.to(torch.float32).contiguous()
        dq = torch.empty((1, nq, hq, d), dtype=q.dtype, device=q.device)
        dk = torch.empty((1, nk, hkv, d), dtype=k.dtype, device=k.device)
        dv = torch.empty((1, nk, hkv, v.shape[-1]), dtype=v.dtype, device=v.device)
        size = ctypes.c_size_t()
        _lib.call("aspec_dspark_attn_bwd_workspace_bytes", nq, nk, hq, hkv, ctypes.byref(size))
        workspace = torch.empty(size.value, dtype=torch.uint8, device=q.device)
        outv = out.transpose(1, 2)
        args = (
            _lib.ptr(q), q.stride(2), q.stride(1), _lib.ptr(k), k.stride(2), k.stride(1),
            _lib.ptr(v), v.stride(2), v.stride(1), _lib.ptr(out), outv.stride(2), outv.stride(1),
            _lib.ptr(dout), dout.stride(2), dout.stride(1), _lib.ptr(lse), _lib.ptr(dlse_c),
            _lib.ptr(endpoints), _lib.ptr(plan), nq, nk, hq, hkv, d, ctx.scale,
            _lib.ptr(dq), dq.stride(1), dq.stride(2), _lib.ptr(dk), dk.stride(1), dk.stride(2),
            _lib.ptr(dv), dv.stride(1), dv.stride(2), _lib.ptr(workspace), _lib.mask_dtype_code(q),
            _lib.stream_handle(q.device),
        )
        # dQ and dK/dV depend only on the prepare stage: dQ runs on a second stream (default
        # priority) beside dK/dV, so each fills the other's tail of partly occupied CUs.
        main = torch.cuda.current_stream(q.device)
        side = _backward_side_stream(q.device) if _overlap_backward else None
        with _timing.region("attn_bwd_prepare"):
            _lib.call("aspec_dspark_attn_bwd_stages", 1, *args)
        if side is not None:
            side.wait_stream(main)
            with torch.cuda.stream(side), _timing.region("attn_bwd_dq"):
                _lib.call("aspec_dspark_attn_bwd_stages", 2, *args[:-1], side.cuda_stream)
        else:
            with _timing.region("attn_bwd_dq"):
                _lib.call("aspec_dspark_attn_bwd_stages", 2, *args)
        with _timing.region("attn_bwd_dkdv"):
            _lib.call("aspec_dspark_attn_bwd_stages", 4, *args)
        with _timing.region("attn_bwd_finalize"):
            _lib.call("aspec_dspark_attn_bwd_stages", 8, *args)
        if side is not None:
            main.wait_stream(side)
        return dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2), None, None, None


_overlap_backward = True
_side_streams: dict = {}


def backward_overlap() -> bool:
    """Whether the attention backward runs dQ beside dK/dV (see set_backward_overlap)."""
    return _overlap_backward


def set_backward_overlap(enabled: bool) -> None:
    """Run the attention backward's dQ kernel beside dK/dV on a second stream (the default) or
    after it on the caller's stream. Both do the same work; the serial order gives each kernel the
    whole GPU, for per-kernel timing and hardware counters."""
    global _overlap_backward
    _overlap_backward = bool(enabled)


def _backward_side_stream(device) -> torch.cuda.Stream:
    """One extra stream per device for the attention backward (created once, default priority)."""
    key = torch.device(device).index
    stream = _side_streams.get(key)
    if stream is None:
        stream = torch.cuda.Stream(device=device)
        _side_streams[key] = stream
    return stream


def _join_batch(x: Tensor) -> Tensor:
    """[B, H, L, D] -> [1, H, B*L, D] with batch row b's tokens at b*L .. b*L + L - 1 (a view when
    the storage is token-major [B, L, H, D], a copy otherwise)."""
    b, h, n, d = x.shape
    return x.transpose(1, 2).reshape(1, b * n, h, d).transpose(1, 2)


def _check_dtypes(query: Tensor, key: Tensor, value: Tensor) -> None:
    """bf16 or fp16 Q/K/V of one dtype (the reference's GPU paths take both: FA4 for either,
    direct_cp.py:1063-1068; cuDNN, cudnn_flex_attention.py:353-356); fp32 accumulation."""
    if query.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError("aspec_amd DSpark attention computes in bf16 or fp16 (fp32 accumulation)")
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise TypeError("Q/K/V must have the same dtype")


def dspark_attention(query: Tensor, key: Tensor, value: Tensor, metadata: DirectCPMetadata,
                     scale: float) -> tuple[Tensor, Tensor]:
    """HIP block-sparse DSpark attention over the metadata's rows: (out [B,Hq,Nq,D], lse [B,Hq,Nq])."""
    if not query.is_cuda:
        raise ValueError("aspec_amd attention runs on the GPU; got a CPU tensor")
    _check_dtypes(query, key, value)
    batch = query.shape[0]
    if batch != metadata.anchor_positions.shape[0]:
        raise ValueError("query batch must match the metadata batch")
    if query.shape[1] % key.shape[1]:
        raise ValueError("THD query heads must be divisible by KV heads")
    if query.shape[2] != metadata.num_blocks * metadata.block_size:
        raise ValueError("query rows must equal num_blocks * block_size")
    rows = thd_row_metadata(metadata, query.device)
    rows.check_layout()
    plan = attention_plan(metadata, rows, query.device)
    if batch == 1:
        output, lse = _DSparkAttention.apply(query, key, value, rows.endpoints, plan, scale)
    else:
        # Every batch row in one launch: rows are concatenated into one token axis (a view of
        # token-major [B, L, H, D] storage), and the endpoints already address the flattened keys.
        output, lse = _DSparkAttention.apply(_join_batch(query), _join_batch(key), _join_batch(value),
                                             rows.endpoints, plan, scale)
        nq, hq = query.shape[2], query.shape[1]
        output = output.transpose(1, 2).reshape(batch, nq, hq, output.shape[-1]).transpose(1, 2)
        lse = lse[0].view(hq, batch, nq).permute(1, 0, 2)
    observation = direct_cp_attention_observation(metadata)
    observation.update(
        qkv_format="thd", kernel_backend="hip", kernel_mode="block_sparse_interval",
        backward_strategy="hip_joint_gqa", gqa_layout="internal_joint", backward_observed=False,
        context_parallel_size=metadata.cp_size, context_parallel_rank=metadata.cp_rank,
        empty_local_partition=False, query_tokens=query.shape[2], key_tokens=key.shape[2],
        context_tokens=metadata.context_length, context_window=metadata.context_window,
        query_window=metadata.query_window, draft_is_causal=metadata.draft_is_causal,
    )

    def observe_backward(gradient):
        observation["backward_observed"] = True
        return gradient

    for tensor in (output, lse):
        if tensor.requires_grad:
            tensor.register_hook(observe_backward)
    return output, lse


def cp_shard_endpoints(metadata: DirectCPMetadata, device) -> Tensor:
    """HIP `aspec_thd_cp_shard_endpoints`: the interval endpoints of this rank's partial
    (`_build_cudnn_thd_mask` at cp_size > 1, direct_cp.py:750-878): every gathered query row (the
    collective block order) against this rank's context shard and the draft keys of its own
    blocks. Cached per forward; one host read of the layout flags, as the reference's monotonic
    check (direct_cp.py:776-780)."""
    device = torch.device(device)
    key = ("hip_cp_shard_endpoints", device)
    ends = metadata._fa4_cache.get(key)
    if ends is not None:
        return ends
    batch, n, block, T = (metadata.anchor_positions.shape[0], metadata.num_blocks,
                          metadata.block_size, metadata.context_length)
    anchors = metadata.anchor_positions.to(device=device, dtype=torch.int64).contiguous()
    keep = metadata.block_keep_mask.to(device=device, dtype=torch.bool).contiguous()
    positions = metadata.context_position_ids.to(device=device, dtype=torch.int64).contiguous()
    if metadata.context_doc_ids is None:
        anchor_docs = torch.zeros((batch, n), dtype=torch.int64, device=device)
        context_docs = torch.zeros((batch, T), dtype=torch.int64, device=device)
    else:
        anchor_docs = metadata.anchor_doc_ids.to(device=device, dtype=torch.int64).contiguous()
        context_docs = metadata.context_doc_ids.to(device=device, dtype=torch.int64).contiguous()
    query_blocks = metadata.collective_block_ids.to(device)
    local_blocks = metadata.local_block_ids.to(device)
    nq = query_blocks.numel() * block
    ends = torch.empty((5, batch * nq), dtype=torch.int32, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    seq = metadata.sequence_length if metadata.sequence_length is not None else 0
    with _timing.region("thd_row_metadata"):
        _lib.call("aspec_thd_cp_shard_endpoints", _lib.ptr(anchors), _lib.ptr(keep), _lib.ptr(anchor_docs),
                  _lib.ptr(positions), _lib.ptr(context_docs), batch, n, block, T, _lib.ptr(query_blocks),
                  query_blocks.numel(), _lib.ptr(local_blocks), local_blocks.numel(), seq,
                  metadata.context_window or 0, metadata.query_window or 0, int(metadata.draft_is_causal),
                  _lib.ptr(ends), _lib.ptr(flags), _lib.stream_handle(device))
    bad = int(flags.item())
    if bad & 1:
        raise ValueError("cuDNN THD requires monotonically ordered context positions")
    if bad & 2:
        raise ValueError("THD attention requires contiguous ascending documents (padding last)")
    if bad & 4:
        raise ValueError("CP block ownership out of range or not ascending")
    metadata._fa4_cache[key] = ends
    return ends


def direct_cp_partial_attention(query_full: Tensor, key: Tensor, value: Tensor,
                                metadata: DirectCPMetadata, scale: Optional[float] = None
                                ) -> tuple[Tensor, Tensor]:
    """One CP rank's partial attention, the step of direct_cp_attention_from_kv between the query
    all-gather and the all-to-all of the partials (direct_cp.py:1077-1093): every gathered query
    ([B, Hq, num_blocks * block_size, D] in the collective block order) against this rank's keys
    ([B, Hkv, context_length + queries_per_rank, D]: its context shard, then its own blocks' draft
    keys). Returns the partial (out, lse), each row normalised over this rank's keys only (rows
    without a visible key here: O = 0, LSE = -1e30); `merge_attention_partials` combines the ranks'
    partials exactly. Differentiable in query, key and value. The collectives around it need
    several GPUs and are not part of this single-GPU build."""
    length = metadata.context_length + metadata.queries_per_rank
    if (key.ndim != 4 or value.ndim != 4 or key.shape[:3] != value.shape[:3]
            or key.shape[0] != query_full.shape[0] or key.shape[2] != length):
        raise ValueError("Combined KV must match local context and draft ownership")
    if query_full.ndim != 4 or query_full.shape[2] != metadata.num_blocks * metadata.block_size:
        raise ValueError(f"expected {metadata.num_blocks * metadata.block_size} gathered queries")
    if not query_full.is_cuda:
        raise ValueError("aspec_amd attention runs on the GPU; got a CPU tensor")
    _check_dtypes(query_full, key, value)
    if query_full.shape[1] % key.shape[1]:
        raise ValueError("query heads must be divisible by the matching KV head count")
    if metadata.backend == "math":
        raise NotImplementedError(
            "the math backend is the reference's CPU path; aspec_amd runs the HIP kernels only")
    scale = scale if scale is not None else query_full.shape[-1] ** -0.5
    ends = cp_shard_endpoints(metadata, query_full.device)
    batch = query_full.shape[0]
    rows = ThdRows(None, None, ends, None, batch * query_full.shape[2], batch * key.shape[2], batch)
    plan = attention_plan(metadata, rows, query_full.device)
    if batch == 1:
        return _DSparkAttention.apply(query_full, key, value, ends, plan, scale)
    output, lse = _DSparkAttention.apply(_join_batch(query_full), _join_batch(key), _join_batch(value),
                                         ends, plan, scale)
    nq, hq = query_full.shape[2], query_full.shape[1]
    output = output.transpose(1, 2).reshape(batch, nq, hq, output.shape[-1]).transpose(1, 2)
    return output, lse[0].view(hq, batch, nq).permute(1, 0, 2)


def merge_attention_partials(outputs: Tensor, lse_parts: Tensor) -> tuple[Tensor, Tensor]:
    """Merge independently normalised attention partials exactly (`merge_attention_partials` /
    `_merge_partials`, direct_cp.py:362-367,460-467): outputs [P, ..., D] and lse_parts [P, ...]
    stacked over the P partials. lse = logsumexp over the partials, each partial weighted by
    exp(lse_p - lse); a row none of whose partials is finite keeps LSE = -1e30. Differentiable."""
    has_keys = torch.isfinite(lse_parts).any(dim=0)
    safe_parts = torch.where(has_keys.unsqueeze(0), lse_parts, torch.zeros_like(lse_parts))
    safe_lse = torch.logsumexp(safe_parts, dim=0)
    lse = torch.where(has_keys, safe_lse, torch.full_like(safe_lse, MASK_VALUE))
    weights = torch.exp(lse_parts - safe_lse.unsqueeze(0))
    weights = torch.where(has_keys.unsqueeze(0), weights, torch.zeros_like(weights))
    return (weights.unsqueeze(-1) * outputs).sum(dim=0), lse


def direct_cp_attention_from_kv(query_own: Tensor, key: Tensor, value: Tensor,
                                metadata: DirectCPMetadata, scale: Optional[float] = None, *,
                                cudnn_gqa_mode: str = "auto") -> tuple[Tensor, Tensor]:
    """Use already assembled context+draft KV (direct_cp.py:1047-1100)."""
    length = metadata.context_length + metadata.queries_per_rank
    if (key.ndim != 4 or value.ndim != 4 or key.shape[:3] != value.shape[:3]
            or key.shape[0] != query_own.shape[0] or key.shape[2] != length):
        raise ValueError("Combined KV must match local context and draft ownership")
    scale = scale if scale is not None else query_own.shape[-1] ** -0.5
    if cudnn_gqa_mode not in _GQA_MODES:
        raise ValueError(f"unsupported cuDNN GQA mode: {cudnn_gqa_mode}")
    if cudnn_gqa_mode != "auto" and metadata.backend != "cudnn_flex_attention":
        raise ValueError("Explicit cudnn_gqa_mode requires the cuDNN backend")
    if metadata.backend == "math":
        raise NotImplementedError(
            "the math backend is the reference's CPU path; aspec_amd runs the HIP kernels only")
    if metadata.cp_size != 1:
        raise NotImplementedError(
            "context parallelism > 1 gathers queries and exchanges partials between GPUs; this "
            "single-GPU build runs one rank's share with direct_cp_partial_attention and combines "
            "partials with merge_attention_partials")
    output, lse = dspark_attention(query_own, key, value, metadata, scale)
    return output.to(query_own.dtype), lse


def direct_cp_attention(query_own: Tensor, context_key: Tensor, context_value: Tensor,
                        draft_key_own: Tensor, draft_value_own: Tensor, metadata: DirectCPMetadata,
                        scale: Optional[float] = None) -> tuple[Tensor, Tensor]:
    """Concatenate context and draft KV, then attend (direct_cp.py:1027-1044)."""
    return direct_cp_attention_from_kv(
        query_own, torch.cat((context_key, draft_key_own), dim=2),
        torch.cat((context_value, draft_value_own), dim=2), metadata, scale,
    )
