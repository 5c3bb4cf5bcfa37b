"""GPU timing harness (HIP events) and the geomean ranking metric.

Same methodology as the reference (src/qrbench/bench.py:57-91): ``warmup``
untimed calls, then ``iters`` calls each bracketed by a fresh event pair on the
current stream and a device synchronise; report median/min/mean. The input is
not cloned per call (the QR is out of place and must not modify A).
"""

from __future__ import annotations

import math
import statistics
from dataclasses import dataclass, field
from typing import Callable

import torch


@dataclass
class TimingResult:
    times_ms: list[float] = field(default_factory=list)

    @property
    def mean(self) -> float:
        return statistics.fmean(self.times_ms)

    @property
    def median(self) -> float:
        return statistics.median(self.times_ms)

    @property
    def min(self) -> float:
        return min(self.times_ms)

    @property
    def max(self) -> float:
        return max(self.times_ms)

    @property
    def std(self) -> float:
        return statistics.pstdev(self.times_ms) if len(self.times_ms) > 1 else 0.0

    def as_dict(self) -> dict:
        return {
            "runs": len(self.times_ms),
            "times_ms": self.times_ms,
            "mean_ms": self.mean,
            "median_ms": self.median,
            "min_ms": self.min,
            "max_ms": self.max,
            "std_ms": self.std,
        }


def benchmark(fn: Callable[[torch.Tensor], object], A: torch.Tensor, warmup: int = 10,
              iters: int = 10) -> TimingResult:
    torch.cuda.synchronize()
    for _ in range(warmup):
        fn(A)
    torch.cuda.synchronize()
    times: list[float] = []
    for _ in range(iters):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        fn(A)
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end))
    return TimingResult(times_ms=times)


def geomean(values: list[float]) -> float:
    """Geometric mean of positive runtimes; nan for an empty list."""
    if not values:
        return float("nan")
    if any(v <= 0 for v in values):
        raise ValueError("geomean needs positive values")
    return math.exp(sum(math.log(v) for v in values) / len(values))


def qr_flops(batch: int, n: int) -> float:
    """Algorithmic flop count of a square Householder QR batch: 4/3 n^3 per matrix."""
    return 4.0 / 3.0 * n**3 * batch


def qr_bytes(batch: int, n: int) -> float:
    """Algorithmic HBM bytes: read A, write H and tau (fp32)."""
    return (2.0 * n * n + n) * 4.0 * batch
