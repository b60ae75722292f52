"""THD block-sparse tile metadata on the GPU (aspec/models/ops/thd_sparse_metadata.py).

`build_thd_sparse_pair` keeps the reference signature (thd_sparse_metadata.py:149-186): from the
eight THD mask tensors it produces forward (per query tile) and backward (per key tile) ordered
lists of partial and full tiles. The HIP path first recovers per-row interval endpoints from the
mask tensors, then classifies tiles exactly (every row, not one representative per block) and
compacts the lists with a wavefront ballot scan.
"""

from __future__ import annotations

import torch

from aspec_amd import _lib
from aspec_amd.fa4_sparse import BlockSparseTensors, FA4SparsePair, sparse_block_sizes


def _check_aux(aux_tensors, query_length, key_length):
    if len(aux_tensors) != 8 or aux_tensors[0].ndim != 2:
        raise ValueError("Expected eight THD fixed mask tensors")
    anchors = aux_tensors[0]
    batch = anchors.shape[0]
    for index, tensor in enumerate(aux_tensors):
        shape = (batch, query_length if index < 4 else key_length)
        if (tuple(tensor.shape) != shape or tensor.dtype != torch.int32
                or tensor.device != anchors.device or not tensor.is_cuda
                or not tensor.is_contiguous()):
            raise ValueError("Expected contiguous int32 THD aux tensors on one CUDA device")
    if batch != 1:
        raise NotImplementedError("THD sparse metadata covers one packed row per microbatch")


def aux_endpoints(aux_tensors, *, block_size, query_length, key_length, context_window=None,
                  query_window=None, draft_is_causal=False):
    """Interval endpoints [5, Nq] from the eight mask tensors (HIP `aspec_thd_aux_endpoints`)."""
    _check_aux(aux_tensors, query_length, key_length)
    if key_length < query_length:
        raise ValueError("Invalid THD fixed sparse geometry")
    device = aux_tensors[0].device
    query_aux = torch.stack([t[0] for t in aux_tensors[:4]]).contiguous()
    key_aux = torch.stack([t[0] for t in aux_tensors[4:]]).contiguous()
    ends = torch.empty((5, query_length), dtype=torch.int32, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    _lib.call("aspec_thd_aux_endpoints", _lib.ptr(query_aux), _lib.ptr(key_aux), query_length,
              key_length, block_size, context_window or 0, query_window or 0,
              int(draft_is_causal), _lib.ptr(ends), _lib.ptr(flags), _lib.stream_handle(device))
    return ends, flags


def tile_metadata(endpoints, *, query_length, key_length, tile_m, tile_n, pad_visible=True,
                  forward=True, backward=True):
    """Classes [nm, nn] plus forward row lists and backward column lists (HIP)."""
    device = endpoints.device
    nm = -(-query_length // tile_m)
    nn = -(-key_length // tile_n)
    i32 = dict(dtype=torch.int32, device=device)
    classes = torch.empty((nm, nn), **i32)
    out = {"classes": classes}
    if forward:
        out.update(fwd_partial_cnt=torch.empty(nm, **i32), fwd_partial_idx=torch.empty((nm, nn), **i32),
                   fwd_full_cnt=torch.empty(nm, **i32), fwd_full_idx=torch.empty((nm, nn), **i32))
    if backward:
        out.update(bwd_partial_cnt=torch.empty(nn, **i32), bwd_partial_idx=torch.empty((nn, nm), **i32),
                   bwd_full_cnt=torch.empty(nn, **i32), bwd_full_idx=torch.empty((nn, nm), **i32))
    names = ["fwd_partial_cnt", "fwd_partial_idx", "fwd_full_cnt", "fwd_full_idx",
             "bwd_partial_cnt", "bwd_partial_idx", "bwd_full_cnt", "bwd_full_idx"]
    _lib.call("aspec_thd_tile_metadata", _lib.ptr(endpoints), query_length, key_length, tile_m,
              tile_n, int(pad_visible), _lib.ptr(classes), *[_lib.ptr(out.get(n)) for n in names],
              _lib.stream_handle(device))
    return out


def _build_sparse_source(*, aux_tensors, block_size, query_length, key_length, tile_m, tile_n,
                         context_window=None, query_window=None, draft_is_causal=False,
                         transposed=False):
    """Ordered lists at one tile geometry (thd_sparse_metadata.py:97-146); `transposed` gives the
    per-key-tile lists that `_transpose_fixed_sparse` (fa4_sparse.py:94-113) would produce."""
    if len(aux_tensors) != 8:
        raise ValueError("Expected eight THD fixed mask tensors")
    if min(block_size, query_length, key_length, tile_m, tile_n) <= 0:
        raise ValueError("Invalid THD fixed sparse geometry")
    ends, flags = aux_endpoints(aux_tensors, block_size=block_size, query_length=query_length,
                                key_length=key_length, context_window=context_window,
                                query_window=query_window, draft_is_causal=draft_is_causal)
    lists = tile_metadata(ends, query_length=query_length, key_length=key_length, tile_m=tile_m,
                          tile_n=tile_n, pad_visible=True, forward=not transposed,
                          backward=transposed)
    bad = int(flags.item())
    if bad:
        raise ValueError(f"THD mask tensors violate the packed layout contract (flags={bad})")
    side = "bwd" if transposed else "fwd"
    return BlockSparseTensors(
        mask_block_cnt=lists[f"{side}_partial_cnt"][None, None],
        mask_block_idx=lists[f"{side}_partial_idx"][None, None],
        full_block_cnt=lists[f"{side}_full_cnt"][None, None],
        full_block_idx=lists[f"{side}_full_idx"][None, None],
        block_size=(tile_m, tile_n),
    )


def build_thd_sparse_pair(*, aux_tensors, block_size, query_length, key_length, query_head_dim,
                          value_head_dim, context_window=None, query_window=None,
                          draft_is_causal=False) -> FA4SparsePair:
    """Forward lists and transposed backward lists (thd_sparse_metadata.py:149-186)."""
    forward_size, backward_size = sparse_block_sizes(aux_tensors[0].device if aux_tensors else None,
                                                     query_head_dim, value_head_dim)
    common = dict(aux_tensors=aux_tensors, block_size=block_size, query_length=query_length,
                  key_length=key_length, context_window=context_window,
                  query_window=query_window, draft_is_causal=draft_is_causal)
    forward = _build_sparse_source(**common, tile_m=forward_size[0], tile_n=forward_size[1])
    backward = _build_sparse_source(**common, tile_m=backward_size[0], tile_n=backward_size[1],
                                    transposed=True)
    return FA4SparsePair(forward=forward, backward=backward)
