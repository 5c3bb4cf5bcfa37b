"""Elementwise parity metrics between two compact (H, tau) factorisations.

(H, tau) is compared with a reference (H_ref, tau_ref) of the same input A.
For matrix b, row i and column j:
    |dV_ij|                 <= 4 n (eps32 + f_j) g_j     (i > j, below the diagonal)
    |dtau_j|                <= 4 n (eps32 + f_j) g_j
    |dR_ij| / ||A[:, j]||_2 <= 4 n (eps32 + f_j) g_i     (i <= j, R with its diagonal)
V entries are bounded by 1 in magnitude and tau lies in {0} U [1, 2], so these
are relative errors as well.

* 4 n eps32 is the flat bound. For most columns it is the whole tolerance:
  fp32 torch.geqrf against fp64 on Gaussian, cond-1e2 and zeroed/1e4-column
  inputs up to n = 2048 differs by 2e-6 .. 2e-5, well under 4 n eps32
  (4.9e-4 at n = 1024).

* g_j = max(1, S_j / 10) is the sensitivity of column j's reflector. The
  reflector of column j is the direction of x_j, the part of A[:, j] left
  after the reflectors 0..j-1, and ||x_j|| = |R_jj|. Rounding perturbs x_j by
  about n eps32 ||A[:, j]|| (Householder QR is columnwise backward stable), so
  v_j and tau_j move by about n eps32 s_j with s_j = ||A[:, j]||_2 / |R_jj|,
  and a reflector that moved turns every later column with it. S_j is the
  largest s_k over k <= j (s_k = 1 for a zero column), taken from the
  reference's R; R entries of row i depend on the reflectors 0..i only, hence
  g_i for them. The divisor 10 keeps the rule ten times tighter than that
  first-order estimate. Most columns have S_j < 10 (g_j = 1); it grows at a
  small pivot, typically in the last columns of a large Gaussian matrix.
  Two correct fp32 implementations need it: LAPACK sgeqrf from MKL against
  the C oracle exceeds the flat bound by 2.5x on Gaussian 3 x 3 matrices with
  a nearly dependent column pair, and by 1.1x on matrix 63 of the n = 1024
  Gaussian benchmark input (|R_1021,1021| = 0.28 against ||a|| = 32), and
  stays under 0.75x this rule for n = 2 .. 1024 (test_parity_rule.py).

* f_j is fp32's subnormal floor: arithmetic on numbers below 2^-126 rounds
  to an absolute 2^-149, so a column whose entries are that small carries a
  relative error of 2^-149 / rms(a_k) in every operation, passed on to every
  later column. f_j is the largest 2^-149 / rms(A[:, k]) over k <= j (0 for
  zero columns); it is below 1e-14 for any column of rms above 1e-31, so only
  subnormal columns (1e-40) feel it, where MKL and the oracle differ by 1.6x
  the flat bound at n = 300.

assert_parity prints one line with the largest errors and the largest
error-to-tolerance ratio, so a test log shows the margin of every comparison.
"""

from __future__ import annotations

import numpy as np

EPS32 = 2.0**-23
ETA32 = 2.0**-149  # spacing of the fp32 subnormals
S0 = 10.0  # sensitivity at which the tolerance starts to widen

# The one-line margin of every comparison that passed, in order;
# tests/conftest.py prints them in pytest's terminal summary so a quiet (-q)
# run still shows each margin. (A rejected comparison raises with its own
# message instead.)
MARGINS: list[str] = []


def tolerance(n: int, c: float = 4.0) -> float:
    """The flat bound c n eps32."""
    return c * max(n, 1) * EPS32


def _colnorm(A: np.ndarray) -> np.ndarray:
    return np.sqrt((A * A).sum(axis=-2))  # (batch, n): ||A[:, j]||_2


def subnormal_floor(A) -> np.ndarray:
    """f_j of the module docstring for A (batch, n, n): (batch, n)."""
    A = np.asarray(A, dtype=np.float64)
    rms = np.sqrt((A * A).mean(axis=-2))
    f = np.where(rms > 0, ETA32 / np.where(rms > 0, rms, 1.0), 0.0)
    return np.maximum.accumulate(f, axis=-1)


def sensitivity(A, H_ref) -> np.ndarray:
    """S_j of the module docstring: running max over k <= j of
    ||A[:, k]|| / |R_ref[k, k]| (1 for a zero column); (batch, n)."""
    A = np.asarray(A, dtype=np.float64)
    cn = _colnorm(A)
    rkk = np.abs(np.diagonal(np.asarray(H_ref, dtype=np.float64), axis1=-2, axis2=-1))
    s = np.ones_like(cn)
    nz = cn > 0
    s[nz] = cn[nz] / np.maximum(rkk[nz], np.finfo(np.float64).tiny)
    return np.maximum.accumulate(s, axis=-1)


def _entry_ratios(A, H, tau, H_ref, tau_ref, tol):
    """Error-to-tolerance ratios: R (batch, n, n; upper triangle), V (same,
    strictly lower), tau (batch, n); plus the raw max errors. NaN counts as
    +inf."""
    A = np.asarray(A, dtype=np.float64)
    H = np.asarray(H, dtype=np.float64)
    Hr = np.asarray(H_ref, dtype=np.float64)
    n = A.shape[-1]
    upper = np.triu(np.ones((n, n), dtype=bool))
    cn = np.maximum(_colnorm(A), np.finfo(np.float64).tiny)
    dH = np.abs(H - Hr)
    dH = np.where(np.isnan(dH), np.inf, dH)
    dt = np.abs(np.asarray(tau, np.float64) - np.asarray(tau_ref, np.float64))
    dt = np.where(np.isnan(dt), np.inf, dt)
    dR = np.where(upper, dH / cn[:, None, :], 0.0)
    dV = np.where(upper, 0.0, dH)
    if tol is None:
        base = 4.0 * max(n, 1) * (EPS32 + subnormal_floor(A))  # (batch, n), per column
        g = np.maximum(1.0, sensitivity(A, Hr) / S0)  # (batch, n)
        rR = dR / (base[:, None, :] * g[:, :, None])  # row factor g_i
        rV = dV / (base * g)[:, None, :]  # column factor g_j
        rT = dt / (base * g)
    else:
        rR, rV, rT = dR / tol, dV / tol, dt / tol
    errs = {"R": float(dR.max(initial=0.0)), "V": float(dV.max(initial=0.0)),
            "tau": float(dt.max(initial=0.0))}
    return rR, rV, rT, errs


def parity_errors(A, H, tau, H_ref, tau_ref) -> dict:
    """Max errors over the batch of (H, tau) against (H_ref, tau_ref) for A (batch, n, n)."""
    return _entry_ratios(np.asarray(A)[None] if np.ndim(A) == 2 else A, H, tau, H_ref, tau_ref,
                         1.0)[3]


def assert_parity(A, H, tau, H_ref, tau_ref, tol: float | None = None, what: str = "",
                  quiet: bool = False) -> dict:
    """Check the stated tolerance; returns the max errors, the flat bound and
    the largest error-to-tolerance ratio. ``tol`` replaces the whole rule by
    one flat number."""
    A = np.asarray(A)
    if A.ndim == 2:
        A, H, tau = A[None], np.asarray(H)[None], np.asarray(tau)[None]
        H_ref, tau_ref = np.asarray(H_ref)[None], np.asarray(tau_ref)[None]
    n = A.shape[-1]
    rR, rV, rT, errs = _entry_ratios(A, H, tau, H_ref, tau_ref, tol)
    worst = {"R": rR.max(initial=0.0), "V": rV.max(initial=0.0), "tau": rT.max(initial=0.0)}
    ratio = float(max(worst.values()))
    out = {**errs, "tol": tolerance(n) if tol is None else tol, "ratio": ratio}
    line = (f"{what or 'case'}: n={n} batch={A.shape[0]} max|dV|={errs['V']:.2e} "
            f"max|dtau|={errs['tau']:.2e} max|dR|/|a_j|={errs['R']:.2e} "
            f"flat tol={out['tol']:.2e} worst/tol={ratio:.3f}")
    if not quiet:
        print(f"[parity] {line}", flush=True)
    if not ratio <= 1.0:
        part = max(worst, key=lambda k: worst[k])
        arr = {"R": rR, "V": rV, "tau": rT}[part]
        where = np.unravel_index(int(np.argmax(arr)), arr.shape)
        raise AssertionError(
            f"{what}: parity beyond tolerance in {part} at (matrix, ...) {tuple(map(int, where))}: "
            f"error/tolerance = {ratio:.3f}; largest errors R={errs['R']:.3e} V={errs['V']:.3e} "
            f"tau={errs['tau']:.3e}, flat bound {tolerance(n):.3e}")
    MARGINS.append(line)
    return out
