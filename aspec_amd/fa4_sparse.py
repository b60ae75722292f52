"""Block-sparse metadata containers (aspec/models/ops/fa4_sparse.py).

`BlockSparseTensors` carries the field names of FA4's `BlockSparseTensorsTorch` that the
reference reads and writes (mask_block_cnt/idx = partial tiles, full_block_cnt/idx = full tiles,
block_size); `FA4SparsePair` is fa4_sparse.py:38-41. The tile geometry is the reference's SM100
choice (fa4_sparse.py:16-23), kept so the lists are bit-comparable with the reference's.
"""

from __future__ import annotations

from dataclasses import dataclass

from torch import Tensor

SPARSE_FORWARD_BLOCK_SIZE = (256, 128)
SPARSE_BACKWARD_BLOCK_SIZE = (256, 128)


@dataclass(frozen=True)
class BlockSparseTensors:
    mask_block_cnt: Tensor
    mask_block_idx: Tensor
    full_block_cnt: Tensor
    full_block_idx: Tensor
    block_size: tuple


@dataclass(frozen=True)
class FA4SparsePair:
    forward: object
    backward: object


def sparse_block_sizes(device=None, query_head_dim: int = 128, value_head_dim: int = 128):
    """Sparse metadata tiles (fa4_sparse.py:44-72): (forward, backward) (rows, keys)."""
    del device, query_head_dim, value_head_dim
    return SPARSE_FORWARD_BLOCK_SIZE, SPARSE_BACKWARD_BLOCK_SIZE
