"""The context-parallel shard oracle (oracle/metadata.py: `shard_positions`, `cp_blocks`,
`cp_math_visibility`, `cp_endpoints`) pinned on the CPU, and the product's CP ownership helpers
against it.

* Ownership: known answers of `build_context_positions` (direct_cp.py:23-53) for the contiguous
  layout (with aligned groups, the last rank taking the remainder) and the zigzag layout (chunks r and
  2cp-1-r); every layout partitions the positions (each exactly once).
* The rank's visibility is the CP = 1 visibility restricted to its keys: the ranks' visible sets,
  mapped back to global keys, partition the CP = 1 mask exactly (each visible pair on exactly one
  rank), so a wrong shard, a wrong draft slot or a lost document check fails.
* At cp_size 1 the shard visibility equals `math_visibility`.
* The shard endpoints reproduce the shard visibility exactly (blocks the rank does not own: both
  draft endpoints at the key length, an empty interval).
* `aspec_amd.direct_cp.build_context_positions` and `DirectCPMetadata.local_block_ids /
  collective_block_ids` equal the oracle.
"""

import numpy as np
import pytest
import torch

from aspec_amd import workloads as W
from aspec_amd.direct_cp import DirectCPMetadata, build_context_positions
from oracle import metadata as M


def test_shard_positions_known_answers_and_partition():
    assert [M.shard_positions(10, r, 3).tolist() for r in range(3)] == [[0, 1, 2], [3, 4, 5], [6, 7, 8, 9]]
    assert [M.shard_positions(10, r, 3, alignment=4).tolist() for r in range(3)] == [[], [0, 1, 2, 3], [4, 5, 6, 7, 8, 9]]
    assert [M.shard_positions(8, r, 2, "zigzag").tolist() for r in range(2)] == [[0, 1, 6, 7], [2, 3, 4, 5]]
    assert M.shard_positions(12, 1, 3, "zigzag").tolist() == [2, 3, 8, 9]
    for total in (0, 1, 7, 64, 4096, 4099):
        for cp in (1, 2, 3, 4, 8):
            for layout in ("contiguous", "zigzag"):
                parts = [M.shard_positions(total, r, cp, layout) for r in range(cp)]
                joined = np.sort(np.concatenate(parts))
                assert np.array_equal(joined, np.arange(total)), (total, cp, layout)
                assert all(np.all(np.diff(p) > 0) for p in parts)
                mine = [build_context_positions(total, r, cp, layout=layout).numpy() for r in range(cp)]
                assert all(np.array_equal(a, b) for a, b in zip(mine, parts))


def _layouts():
    yield W.config1(0)
    lengths = [100, 37, 250, 64, 180, 90]  # ragged documents, an anchor every 16 tokens
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    anchors = np.concatenate([s + np.arange(0, n - 8, 16) for s, n in zip(starts, lengths)])
    docs = np.concatenate([np.full(len(np.arange(0, n - 8, 16)), d) for d, n in enumerate(lengths)])
    yield W.from_layout("ragged", lengths, anchors, docs, 8)
    w = W.from_layout("dropped", [150, 106, 40], np.array([0, 40, 96, 120, 150, 190, 230, 250]),
                      np.array([0, 0, 0, 0, 1, 1, 1, 2]), 16,
                      keep=[True, False, True, True, True, True, False, True], pad_to=300)
    yield w


def _shard(w, n, rank, cp, layout):
    pos = M.shard_positions(w.context_length, rank, cp, layout)
    collective, local = M.cp_blocks(n, rank, cp, layout)
    return pos, collective, local


@pytest.mark.parametrize("cp", [2, 4])
@pytest.mark.parametrize("layout", ["contiguous", "zigzag"])
@pytest.mark.parametrize("opts", [{}, {"draft_is_causal": True}, {"context_window": 100},
                                  {"query_window": 5}])
def test_shard_visibility_partitions_the_cp1_mask(cp, layout, opts):
    for w in _layouts():
        n = w.num_blocks - w.num_blocks % (2 * cp)  # divisibility, as DirectCPMetadata requires
        anchors, keep, adocs = w.anchors[:n], w.keep[:n], w.anchor_doc_ids[:n]
        full = M.math_visibility(anchors, keep, w.context_positions, w.ctx_doc_ids, adocs, w.block_size,
                                 w.sequence_length, **opts)
        T = w.context_length
        covered = np.zeros(full.shape, np.int64)
        for rank in range(cp):
            pos, collective, local = _shard(w, n, rank, cp, layout)
            vis = M.cp_math_visibility(anchors, keep, adocs, pos, w.ctx_doc_ids[pos], w.block_size,
                                       w.sequence_length, collective, local, **opts)
            qrows = (np.repeat(collective, w.block_size) * w.block_size
                     + np.tile(np.arange(w.block_size), collective.size))
            gkeys = np.concatenate([pos, T + np.repeat(local, w.block_size) * w.block_size
                                    + np.tile(np.arange(w.block_size), local.size)])
            covered[np.ix_(qrows, gkeys)] += vis
            ends = M.cp_endpoints(anchors, keep, adocs, pos, w.ctx_doc_ids[pos], w.block_size,
                                  w.sequence_length, collective, local, **opts)
            assert np.array_equal(M.endpoints_to_dense(ends, vis.shape[1]), vis)
            absent = ~np.isin(np.repeat(collective, w.block_size), local) & (ends[1] + ends[2] > 0)
            assert np.all(ends[3][absent] == vis.shape[1]) and np.all(ends[4][absent] == vis.shape[1])
        assert covered.max() <= 1
        assert np.array_equal(covered.astype(bool), full)


def test_shard_visibility_at_cp1_is_the_math_visibility():
    for w in _layouts():
        collective, local = M.cp_blocks(w.num_blocks, 0, 1)
        a = M.cp_math_visibility(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                                 w.block_size, w.sequence_length, collective, local)
        b = M.math_visibility(w.anchors, w.keep, w.context_positions, w.ctx_doc_ids, w.anchor_doc_ids,
                              w.block_size, w.sequence_length)
        assert np.array_equal(a, b)
        assert np.array_equal(
            M.cp_endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                           w.block_size, w.sequence_length, collective, local),
            M.endpoints(w.anchors, w.keep, w.anchor_doc_ids, w.context_positions, w.ctx_doc_ids,
                        w.block_size, w.sequence_length))


@pytest.mark.parametrize("layout", ["contiguous", "zigzag"])
def test_metadata_block_ownership_matches_oracle(layout):
    n, cp = 16, 4
    anchors = torch.arange(n)[None] * 8
    for rank in range(cp):
        meta = DirectCPMetadata(anchors, torch.ones_like(anchors, dtype=torch.bool),
                                build_context_positions(128, rank, cp, layout=layout)[None], 4, rank, cp,
                                "virtual", layout=layout)
        collective, local = M.cp_blocks(n, rank, cp, layout)
        assert np.array_equal(meta.local_block_ids.numpy(), local)
        assert np.array_equal(meta.collective_block_ids.numpy(), collective)
        assert meta.queries_per_rank == local.size * 4
