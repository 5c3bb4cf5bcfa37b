"""Correctness gates of the compact-Householder QR contract (FP64 residuals).

Same gates and reporting as the reference checker (src/qrbench/checker.py:1-158):

- ``Q = householder_product(H, tau)`` is materialised in the factors' precision
  (fp32), then promoted to fp64 together with ``R = triu(H)`` and ``A``.
- factor residual  ``max_b ||R - Q^T A||_1 / ||A||_1 <= 20 n eps32``
- orthogonality    ``max_b ||Q^T Q - I||_1            <= 100 n eps32``
- diagnostics: lower-triangular leakage ``||tril(Q^T A, -1)||_1 / ||A||_1`` and
  reconstruction ``||Q R - A||_1 / ||A||_1``.

``||.||_1`` is the induced matrix 1-norm (max absolute column sum), reduced as a
max over the batch; the batch is chunked so the fp64 temporaries of one slice
stay under 2 GB.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import EPS32


@dataclass
class CheckResult:
    n: int
    batch: int
    factor_residual: float
    factor_threshold: float
    factor_pass: bool
    orth_residual: float
    orth_threshold: float
    orth_pass: bool
    leakage: float
    reconstruction: float

    @property
    def passed(self) -> bool:
        return bool(self.factor_pass and self.orth_pass)

    def as_dict(self) -> dict:
        return {
            "n": self.n,
            "batch": self.batch,
            "factor_residual": self.factor_residual,
            "factor_threshold": self.factor_threshold,
            "factor_pass": self.factor_pass,
            "orth_residual": self.orth_residual,
            "orth_threshold": self.orth_threshold,
            "orth_pass": self.orth_pass,
            "leakage": self.leakage,
            "reconstruction": self.reconstruction,
            "passed": self.passed,
        }


def _l1(x: torch.Tensor) -> torch.Tensor:
    """Induced 1-norm of each matrix of a batch (max absolute column sum)."""
    return torch.linalg.matrix_norm(x, ord=1)


def _chunk(batch: int, n: int, max_bytes: int = 2_000_000_000) -> int:
    per_item = 4 * n * n * 8  # A, Q, Q^T A, R in fp64
    if per_item <= 0:
        return max(batch, 1)
    return max(1, min(batch, max_bytes // per_item))


def thresholds(n: int) -> tuple[float, float]:
    """(factor, orthogonality) gate thresholds for size n."""
    return 20.0 * n * EPS32, 100.0 * n * EPS32


def _residuals(A, H, tau, eye):
    A64 = A.double()
    Q = torch.linalg.householder_product(H, tau).double()
    R = torch.triu(H).double()
    QtA = Q.transpose(-2, -1) @ A64
    a_norm = _l1(A64).clamp_min(torch.finfo(torch.float64).tiny)
    factor = (_l1(R - QtA) / a_norm).max().item()
    orth = _l1(Q.transpose(-2, -1) @ Q - eye).max().item()
    leak = (_l1(torch.tril(QtA, diagonal=-1)) / a_norm).max().item()
    recon = (_l1(Q @ R - A64) / a_norm).max().item()
    return factor, orth, leak, recon


def _worse(cur: float, new: float) -> float:
    """The larger residual, NaN winning: Python's max(0.0, nan) is 0.0, which
    would let a NaN factorisation pass."""
    if cur != cur:
        return cur
    return new if (new != new or new > cur) else cur


def check(A: torch.Tensor, H: torch.Tensor, tau: torch.Tensor) -> CheckResult:
    """Validate a compact (H, tau) factorisation of A; residuals in FP64.
    A NaN or Inf anywhere in (H, tau) gives a NaN or Inf residual and fails."""
    n = A.shape[-1]
    batch = A.shape[0]
    f_thr, o_thr = thresholds(n)
    eye = torch.eye(n, device=A.device, dtype=torch.float64)
    factor = orth = leak = recon = 0.0
    step = _chunk(batch, n)
    for s in range(0, batch, step):
        e = min(s + step, batch)
        f, o, lk, rc = _residuals(A[s:e], H[s:e], tau[s:e], eye)
        factor, orth = _worse(factor, f), _worse(orth, o)
        leak, recon = _worse(leak, lk), _worse(recon, rc)
    return CheckResult(
        n=n,
        batch=batch,
        factor_residual=factor,
        factor_threshold=f_thr,
        factor_pass=factor <= f_thr,
        orth_residual=orth,
        orth_threshold=o_thr,
        orth_pass=orth <= o_thr,
        leakage=leak,
        reconstruction=recon,
    )
