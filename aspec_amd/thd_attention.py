"""Unpadded THD packing: one physical row of concatenated documents (thd_attention.py).

`_query_metadata` / `_key_metadata` keep the reference's return contract
(thd_attention.py:25-56) but are produced by the HIP row-metadata kernel; `thd_fa4_attention`
(thd_attention.py:136-220) runs the HIP block-sparse kernels.
"""

from __future__ import annotations

from torch import Tensor

from aspec_amd.direct_cp import dspark_attention, thd_row_metadata


def _query_metadata(metadata, device, blocks=None):
    """(query_docs, query_blocks, anchors, query_keep) per query row, CP=1 (all blocks)."""
    if blocks is not None and blocks.numel() != metadata.num_blocks:
        raise NotImplementedError("block subsets belong to CP>1 ownership")
    rows = thd_row_metadata(metadata, device)
    anchors, keep, qblocks, docs = rows.query_aux
    return docs.long(), qblocks.long(), anchors.long(), keep.bool()


def _key_metadata(metadata, device):
    """(key_docs, key_positions, key_blocks, key_keep); draft offsets o are encoded as -o-1."""
    rows = thd_row_metadata(metadata, device)
    docs, positions, blocks, keep = rows.key_aux
    return docs.long(), positions.long(), blocks.long(), keep.bool()


def thd_fixed_aux(metadata, device):
    """The eight int32 [1, L] mask tensors in `fixed_aux` order (thd_attention.py:149-161)."""
    rows = thd_row_metadata(metadata, device)
    return [t[None] for t in rows.query_aux] + [t[None] for t in rows.key_aux]


def thd_fa4_attention(query: Tensor, key: Tensor, value: Tensor, metadata, scale):
    """(out [1,Hq,Nq,D], lse [1,Hq,Nq]) over one packed row (thd_attention.py:136-220)."""
    if query.shape[0] != 1:
        raise ValueError("THD packing requires one controller-owned row per microbatch")
    if metadata.context_doc_ids is None or metadata.sequence_length is None:
        raise ValueError("THD requires document boundaries and physical ownership")
    if query.shape[1] % key.shape[1]:
        raise ValueError("THD query heads must be divisible by KV heads")
    return dspark_attention(query, key, value, metadata, scale)
