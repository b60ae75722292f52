"""Seeded synthetic inputs for the benchmark configurations of the DSpark draft hot path.

Each builder returns a `Workload`: one packed THD row (document lengths, ctx_doc_ids,
context positions) plus an anchor layout (anchors, keep, anchor_doc_ids) with block size B.
All layouts are deterministic given the seed; nothing here reads data from disk.

  config 1: 4 documents, lengths U[256, 1024] (resampled until the sum is <= 4096), an anchor every
            64 doc-local tokens (u <= L - B), B = 16, GQA 32/8 x 128.
  config 2: one 4096-token document, 512 anchors at linspace(0, 4096 - 16, 512).round(), B = 16.
  config 3: 64 log-normal documents (median 600, sigma 1, clipped to [32, 8192]) first-fit packed
            into 32768-token bins (one bin per workload), an anchor every 32 tokens, B = 16.
  config 4: one 32768-token document, 2048 anchors at linspace(0, 32768 - 16, 2048), GQA 40/8.
  config 5: 3 documents of seeded lengths (sum 4096), an anchor every 8 doc-local tokens
            (u <= L - B - 1), B = 16, GQA 32/8 x 128: the full one-layer training step's row.
  reference_b7: the reference's published attention study (10 x 4096 + 40960 + 49152 context
            tokens, 512 captured anchors per document, B = 7, GQA 32/8 x 128), read from
            tests/golden/dspark_b7_workload.json.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np

B7_FIXTURE = Path(__file__).resolve().parent.parent / "tests" / "golden" / "dspark_b7_workload.json"


@dataclass
class Workload:
    name: str
    lengths: list
    ctx_doc_ids: np.ndarray      # [T] int64, -1 on padding
    context_positions: np.ndarray  # [T] int64 (arange at CP=1)
    anchors: np.ndarray          # [N] int64
    keep: np.ndarray             # [N] bool
    anchor_doc_ids: np.ndarray   # [N] int64
    block_size: int
    sequence_length: int
    q_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128

    @property
    def num_blocks(self) -> int:
        return int(self.anchors.size)

    @property
    def num_queries(self) -> int:
        return self.num_blocks * self.block_size

    @property
    def context_length(self) -> int:
        return int(self.ctx_doc_ids.size)

    @property
    def num_keys(self) -> int:
        return self.context_length + self.num_queries


def _row(lengths, pad_to=None):
    used = int(sum(lengths))
    pad = 0 if pad_to is None else pad_to - used
    docs = np.concatenate([np.full(n, i, np.int64) for i, n in enumerate(lengths)]
                          + [np.full(pad, -1, np.int64)])
    return docs, np.arange(docs.size, dtype=np.int64)


def _strided_anchors(lengths, stride, block):
    anchors, docs = [], []
    start = 0
    for d, n in enumerate(lengths):
        for u in range(0, n - block + 1, stride):
            anchors.append(start + u)
            docs.append(d)
        start += n
    return np.asarray(anchors, np.int64), np.asarray(docs, np.int64)


def from_layout(name, lengths, anchors, anchor_docs, block, keep=None, q_heads=32, kv_heads=8,
                pad_to=None):
    docs, pos = _row(lengths, pad_to)
    keep = np.ones(anchors.size, bool) if keep is None else np.asarray(keep, bool)
    return Workload(name, list(map(int, lengths)), docs, pos, np.asarray(anchors, np.int64), keep,
                    np.asarray(anchor_docs, np.int64), block, int(docs.size), q_heads, kv_heads)


def config1(seed: int = 0) -> Workload:
    rng = np.random.default_rng(seed)
    while True:
        lengths = rng.integers(256, 1025, size=4)
        if lengths.sum() <= 4096:
            break
    anchors, docs = _strided_anchors(lengths, 64, 16)
    return from_layout("config1", lengths, anchors, docs, 16)


def config2(seed: int = 0) -> Workload:
    del seed
    T, N, B = 4096, 512, 16
    anchors = np.round(np.linspace(0, T - B, N)).astype(np.int64)
    return from_layout("config2", [T], anchors, np.zeros(N, np.int64), B)


def config3(seed: int = 0, bin_index: int = 0) -> Workload:
    rng = np.random.default_rng(seed)
    lengths = np.clip(np.round(np.exp(np.log(600.0) + rng.standard_normal(64))), 32, 8192).astype(int)
    capacity = 32768
    bins: list[list[int]] = []
    for n in lengths:  # first fit
        for b in bins:
            if sum(b) + n <= capacity:
                b.append(int(n))
                break
        else:
            bins.append([int(n)])
    chosen = bins[bin_index]
    anchors, docs = _strided_anchors(chosen, 32, 16)
    return from_layout(f"config3_bin{bin_index}", chosen, anchors, docs, 16)


def config4(seed: int = 0) -> Workload:
    del seed
    T, N, B = 32768, 2048, 16
    anchors = np.round(np.linspace(0, T - B, N)).astype(np.int64)
    return from_layout("config4", [T], anchors, np.zeros(N, np.int64), B, q_heads=40, kv_heads=8)


def config5(seed: int = 0) -> Workload:
    rng = np.random.default_rng(seed)
    cuts = np.sort(rng.choice(np.arange(512, 4096 - 512), size=2, replace=False))
    lengths = np.diff(np.concatenate([[0], cuts, [4096]]))
    # u <= L - B - 1: every block's last target stays in its document, as injected anchors must
    # (anchors.py:107-116)
    anchors, docs = _strided_anchors([n - 1 for n in lengths], 8, 16)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    anchors = anchors - np.concatenate([[0], np.cumsum(np.asarray(lengths) - 1)[:-1]])[docs] + starts[docs]
    return from_layout("config5", lengths, anchors, docs, 16)


def reference_b7(path=None) -> Workload:
    """The workload of the reference's DSpark B=7 attention study
    (tools/performance/bench_dspark_b7_attention.py; docs/dspark_attn_kernel_optimization.md:49-51):
    twelve documents packed into one 131072-token row, each with its 512 captured document-local
    anchors in the sampler's order, B = 7, so 43008 draft queries and 174080 keys. Per document
    the visible keys are its prefix before the anchor plus the anchor's own block, exactly the
    reference's per-document THD segments laid end to end."""
    data = json.loads(Path(path or B7_FIXTURE).read_text())
    lengths = [int(n) for n in data["lengths"]]
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
    anchors, docs = [], []
    for d, local in enumerate(data["anchor_positions"]):
        anchors.append(starts[d] + np.asarray(local, np.int64))
        docs.append(np.full(len(local), d, np.int64))
    return from_layout("reference_b7", lengths, np.concatenate(anchors), np.concatenate(docs),
                       int(data["block"]))


def reference_b7_published(path=None) -> dict:
    """The study's own figures (SM100): per route, median/min/max ms of fwd, bwd and fb, and its
    timing contract."""
    data = json.loads(Path(path or B7_FIXTURE).read_text())
    return {"architecture": data["architecture"], "timing_contract": data["timing_contract"],
            "ms": data["published_ms"]}


def reference_test_layout(block_size: int, lengths=(257, 263, 19), drop_doc: bool = True) -> Workload:
    """The packed layout of the reference's tile-metadata tests
    (tests/test_thd_sparse_metadata.py:119-139): documents 257/263/19, anchors
    [0, 19, 256, 257, 281, 519, 520, 537], block 2 dropped, block 6 on a missing document."""
    docs, _ = _row(lengths)
    anchors = np.array([0, 19, 256, 257, 281, 519, 520, 537], np.int64)
    anchors = anchors[anchors < docs.size]
    adocs = docs[anchors].copy()
    if drop_doc and adocs.size > 6:
        adocs[6] = -1
    keep = np.array([True, True, False, True, True, True, True, True])[: anchors.size]
    return from_layout(f"reftest_b{block_size}", list(lengths), anchors, adocs, block_size, keep=keep)


def metadata_for(w: Workload, device, **overrides):
    """DirectCPMetadata of a workload on `device` (CP=1)."""
    import torch

    from aspec_amd.direct_cp import DirectCPMetadata

    def t(x, dtype):
        return torch.as_tensor(x, dtype=dtype, device=device)[None]

    kwargs = dict(context_doc_ids=t(w.ctx_doc_ids, torch.long), anchor_doc_ids=t(w.anchor_doc_ids, torch.long),
                  sequence_length=w.sequence_length)
    kwargs.update(overrides)
    return DirectCPMetadata(t(w.anchors, torch.long), t(w.keep, torch.bool),
                            t(w.context_positions, torch.long), w.block_size, 0, 1, None, **kwargs)
