"""Baseline QR implementation and the run registry.

Mirrors src/qrbench/reference.py:15-25 of the reference: every implementation is
a callable ``fn(A) -> (H, tau)`` in the ``torch.geqrf`` convention, and
``REGISTRY`` maps names to callables. ``torch_geqrf`` (rocSOLVER on the GPU,
LAPACK/MKL on the CPU) is the baseline the GPU path is timed against.
"""

from __future__ import annotations

from typing import Callable

import torch

QRImpl = Callable[[torch.Tensor], tuple[torch.Tensor, torch.Tensor]]


def geqrf_reference(A: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """torch.geqrf (batched): rocSOLVER on ROCm, LAPACK on the CPU."""
    return torch.geqrf(A)


REGISTRY: dict[str, QRImpl] = {
    "torch_geqrf": geqrf_reference,
}
