"""Elementwise parity metrics between two compact (H, tau) factorisations.

Stated tolerance (applied where the factorisation is well conditioned):
    |dV_ij|                      <= 4 n eps32   (strictly lower part of H)
    |dtau_j|                     <= 4 n eps32
    |dR_ij| / ||A[:, j]||_2      <= 4 n eps32   (upper triangle incl. diagonal)
V entries are bounded by 1 in magnitude and tau lies in {0} U [1, 2], so the
first two are relative errors as well.
"""

from __future__ import annotations

import numpy as np

EPS32 = 2.0**-23


def tolerance(n: int, c: float = 4.0) -> float:
    return c * max(n, 1) * EPS32


def parity_errors(A, H, tau, H_ref, tau_ref) -> dict:
    """Max errors of (H, tau) against (H_ref, tau_ref) for inputs A (batch, n, n)."""
    A = np.asarray(A, dtype=np.float64)
    H = np.asarray(H, dtype=np.float64)
    Hr = np.asarray(H_ref, dtype=np.float64)
    n = A.shape[-1]
    colnorm = np.sqrt((A * A).sum(axis=-2))  # (batch, n): ||A[:, j]||_2
    colnorm = np.maximum(colnorm, np.finfo(np.float64).tiny)
    upper = np.triu(np.ones((n, n), dtype=bool))
    dH = np.abs(H - Hr)
    r_err = np.where(upper, dH / colnorm[:, None, :], 0.0).max(initial=0.0)
    v_err = np.where(~upper, dH, 0.0).max(initial=0.0)
    t_err = np.abs(np.asarray(tau, np.float64) - np.asarray(tau_ref, np.float64)).max(initial=0.0)
    return {"R": float(r_err), "V": float(v_err), "tau": float(t_err)}


def assert_parity(A, H, tau, H_ref, tau_ref, tol: float | None = None, what: str = "") -> dict:
    n = np.asarray(A).shape[-1]
    tol = tolerance(n) if tol is None else tol
    err = parity_errors(A, H, tau, H_ref, tau_ref)
    bad = {k: v for k, v in err.items() if not (v <= tol)}
    assert not bad, f"{what} parity beyond tol {tol:.3e}: {err}"
    return err
