"""Per-stage GPU timing of the render path (the role of the reference's
per-stage profiler, examples/benchmark_gaussian_splatting.py:88-148).

While a ``StageTimer`` is active, each stage of the fused render records a
pair of events on the stream its kernels are launched on (torch's current
stream), so the measured interval is exactly that stage's device time.
Inactive, the hooks cost one global lookup.
"""

from __future__ import annotations

import contextlib
from collections import defaultdict

import torch

_active: "StageTimer | None" = None


class StageTimer:
    def __init__(self):
        self._pending: list[tuple[str, torch.cuda.Event, torch.cuda.Event]] = []
        self.samples: dict[str, list[float]] = defaultdict(list)
        self.counters: dict[str, list[float]] = defaultdict(list)

    def __enter__(self):
        global _active
        self._prev = _active
        _active = self
        return self

    def __exit__(self, *exc):
        global _active
        _active = self._prev
        self.collect()
        return False

    def collect(self):
        if not self._pending:
            return
        torch.cuda.synchronize()
        for name, a, b in self._pending:
            self.samples[name].append(a.elapsed_time(b))
        self._pending.clear()

    def mean_ms(self, name: str) -> float:
        s = self.samples.get(name, [])
        return sum(s) / len(s) if s else float("nan")

    def median_ms(self, name: str) -> float:
        s = sorted(self.samples.get(name, []))
        if not s:
            return float("nan")
        m = len(s) // 2
        return s[m] if len(s) % 2 else 0.5 * (s[m - 1] + s[m])

    def count(self, name: str, value: float):
        self.counters[name].append(float(value))


@contextlib.contextmanager
def stage(name: str):
    t = _active
    if t is None:
        yield
        return
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    try:
        yield
    finally:
        b.record()
        t._pending.append((name, a, b))


def count(name: str, value: float):
    if _active is not None:
        _active.count(name, value)
