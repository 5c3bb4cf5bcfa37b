"""Per-call event timing of a QR variant, the geomean ranking metric and the
algorithmic work counts.

The timing convention is the reference's (src/qrbench/bench.py:57-91): the
warm-up calls are not timed; each timed call sits between its own pair of HIP
events on the current stream and completes before the next one starts; the
statistics are taken over the per-call times. The input is reused by every
call (the variants are out of place and must not modify it). The statistics'
key names in ``TimingResult.as_dict`` are the DB record's ``timing`` schema.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Sequence

import numpy as np
import torch


@dataclass(frozen=True)
class TimingResult:
    """Per-call times (ms) of one timed run, with its summary statistics."""

    times_ms: tuple[float, ...]

    def _a(self) -> np.ndarray:
        return np.asarray(self.times_ms, dtype=np.float64)

    @property
    def median(self) -> float:
        return float(np.median(self._a()))

    @property
    def mean(self) -> float:
        return float(self._a().mean())

    @property
    def min(self) -> float:
        return float(self._a().min())

    @property
    def max(self) -> float:
        return float(self._a().max())

    @property
    def std(self) -> float:
        """Population standard deviation (0 for a single call)."""
        return float(self._a().std())

    def as_dict(self) -> dict:
        """The ``timing`` entry of a DB record."""
        return {"runs": len(self.times_ms), "times_ms": list(self.times_ms),
                "mean_ms": self.mean, "median_ms": self.median, "min_ms": self.min,
                "max_ms": self.max, "std_ms": self.std}


def benchmark(fn: Callable[[torch.Tensor], object], A: torch.Tensor, warmup: int = 10,
              iters: int = 10) -> TimingResult:
    """Time ``iters`` calls of ``fn(A)`` after ``warmup`` untimed ones."""
    if iters < 1:
        raise ValueError("iters must be at least 1")
    for _ in range(warmup):
        fn(A)
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(iters)]
    torch.cuda.synchronize()
    for begin, end in marks:
        begin.record()
        fn(A)
        end.record()
        end.synchronize()  # this call is complete before the next is enqueued
    return TimingResult(tuple(begin.elapsed_time(end) for begin, end in marks))


def geomean(values: Sequence[float]) -> float:
    """Geometric mean of positive runtimes (the leaderboard's ranking metric);
    nan for no values."""
    a = np.asarray(list(values), dtype=np.float64)
    if a.size == 0:
        return float("nan")
    if not np.all(a > 0):
        raise ValueError("geomean needs positive values")
    return float(np.exp(np.log(a).mean()))


def qr_flops(batch: int, n: int) -> float:
    """Algorithmic flop count of a square Householder QR batch: 4/3 n^3 per matrix."""
    return 4.0 / 3.0 * n**3 * batch


def qr_bytes(batch: int, n: int) -> float:
    """Algorithmic HBM bytes: read A, write H and tau (fp32)."""
    return (2.0 * n * n + n) * 4.0 * batch
