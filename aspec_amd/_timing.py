"""Optional per-region GPU timing with events recorded on the stream the kernels launch on.

Disabled by default (zero cost beyond a flag test). `enable()` makes every `region(name)` record a
start/end event pair on the current stream; `summary()` synchronises and returns per-region
launch counts and mean milliseconds.
"""

from __future__ import annotations

import contextlib
from collections import defaultdict

_enabled = False
_records = defaultdict(list)


def enable(flag: bool = True) -> None:
    global _enabled
    _enabled = flag


def reset() -> None:
    _records.clear()


@contextlib.contextmanager
def region(name: str):
    if not _enabled:
        yield
        return
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    try:
        yield
    finally:
        end.record()
        _records[name].append((start, end))


def summary() -> dict:
    import torch

    torch.cuda.synchronize()
    out = {}
    for name, pairs in _records.items():
        times = [s.elapsed_time(e) for s, e in pairs]
        out[name] = {"launches": len(times), "mean_ms": sum(times) / len(times), "total_ms": sum(times)}
    return out
