"""Elementwise parity metrics between two compact (H, tau) factorisations.

Stated tolerance, per matrix b of the batch:
    |dV_ij|                      <= tol_b   (strictly lower part of H)
    |dtau_j|                     <= tol_b
    |dR_ij| / ||A[:, j]||_2      <= tol_b   (upper triangle incl. diagonal)
    tol_b = 4 n eps32 * max(1, kappa_2(A_b) / 10)
V entries are bounded by 1 in magnitude and tau lies in {0} U [1, 2], so the
first two are relative errors as well. The kappa factor is first-order QR
perturbation theory (forward error of Q and R grows like kappa_2(A) n eps):
for kappa_2 <= 10 the tolerance is the flat 4 n eps32; beyond that it grows
linearly, ten times tighter than the first-order bound. The divisor 10 is the
smallest round value that admits two correct fp32 implementations against each
other: LAPACK sgeqrf (MKL) against the C oracle on 4000 Gaussian matrices per n
reaches 2.3x the kappa/100 tolerance at n = 4 and stays below 0.5x the kappa/10
one for n = 2..64 (test_parity_tolerance_admits_mkl). kappa_2 is only computed
(fp64 SVD) for matrices that exceed the flat tolerance.
"""

from __future__ import annotations

import numpy as np

EPS32 = 2.0**-23
KAPPA0 = 10.0


def tolerance(n: int, c: float = 4.0) -> float:
    return c * max(n, 1) * EPS32


def _per_matrix_errors(A, H, tau, H_ref, tau_ref):
    A = np.asarray(A, dtype=np.float64)
    H = np.asarray(H, dtype=np.float64)
    Hr = np.asarray(H_ref, dtype=np.float64)
    n = A.shape[-1]
    colnorm = np.sqrt((A * A).sum(axis=-2))  # (batch, n): ||A[:, j]||_2
    colnorm = np.maximum(colnorm, np.finfo(np.float64).tiny)
    upper = np.triu(np.ones((n, n), dtype=bool))
    dH = np.abs(H - Hr)
    r_err = np.where(upper, dH / colnorm[:, None, :], 0.0).max(axis=(1, 2), initial=0.0)
    v_err = np.where(~upper, dH, 0.0).max(axis=(1, 2), initial=0.0)
    t_err = np.abs(np.asarray(tau, np.float64) - np.asarray(tau_ref, np.float64)).max(
        axis=1, initial=0.0)
    return r_err, v_err, t_err


def parity_errors(A, H, tau, H_ref, tau_ref) -> dict:
    """Max errors over the batch of (H, tau) against (H_ref, tau_ref) for A (batch, n, n)."""
    r, v, t = _per_matrix_errors(A, H, tau, H_ref, tau_ref)
    return {"R": float(r.max(initial=0.0)), "V": float(v.max(initial=0.0)),
            "tau": float(t.max(initial=0.0))}


def assert_parity(A, H, tau, H_ref, tau_ref, tol: float | None = None, what: str = "") -> dict:
    A = np.asarray(A)
    if A.ndim == 2:
        A, H, tau = A[None], np.asarray(H)[None], np.asarray(tau)[None]
        H_ref, tau_ref = np.asarray(H_ref)[None], np.asarray(tau_ref)[None]
    n = A.shape[-1]
    base = tolerance(n) if tol is None else tol
    r, v, t = _per_matrix_errors(A, H, tau, H_ref, tau_ref)
    worst = np.maximum(np.maximum(r, v), t)
    for b in np.nonzero(~(worst <= base))[0]:
        s = np.linalg.svd(A[b].astype(np.float64), compute_uv=False)
        kappa = s[0] / s[-1] if s[-1] > 0 else np.inf
        tol_b = base * max(1.0, kappa / KAPPA0)
        assert worst[b] <= tol_b, (
            f"{what} matrix {b}: parity beyond tol {tol_b:.3e} (kappa_2={kappa:.3e}): "
            f"R={r[b]:.3e} V={v[b]:.3e} tau={t[b]:.3e}"
        )
    return {"R": float(r.max(initial=0.0)), "V": float(v.max(initial=0.0)),
            "tau": float(t.max(initial=0.0))}
