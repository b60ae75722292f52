"""Optional per-region GPU timing with events recorded on the stream the kernels launch on.

Disabled by default (zero cost beyond a flag test). `enable()` makes every `region(name)` record a
start/end event pair on the current stream; `summary()` synchronises and returns per-region
launch counts and mean milliseconds.

A start event recorded while the GPU is idle (the host has just waited on it) is timestamped at
once, so the region would also count the host's time to build and launch its kernels. With
`enable(lead_us=...)` each region first queues a GPU spin of about that many microseconds on its
stream and records its start event behind it: the event then fires when the spin ends, by which
time the host has queued the region's own launches, and the region times its kernels only.
"""

from __future__ import annotations

import contextlib
from collections import defaultdict

_enabled = False
_lead_cycles = 0
_cycles_per_us = None
_records = defaultdict(list)


def _spin_rate() -> float:
    """Clock cycles per microsecond of torch's GPU spin kernel, measured once."""
    global _cycles_per_us
    if _cycles_per_us is None:
        import torch

        torch.cuda._sleep(1000)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        cycles = 2_000_000
        start.record()
        torch.cuda._sleep(cycles)
        end.record()
        end.synchronize()
        _cycles_per_us = cycles / max(start.elapsed_time(end) * 1e3, 1.0)
    return _cycles_per_us


def enable(flag: bool = True, lead_us: float = 0.0) -> None:
    global _enabled, _lead_cycles
    _enabled = flag
    _lead_cycles = int(lead_us * _spin_rate()) if (flag and lead_us > 0) else 0


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
    if _lead_cycles:
        torch.cuda._sleep(_lead_cycles)
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
