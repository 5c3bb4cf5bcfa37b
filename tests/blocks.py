"""Synthetic 64-column blocks for the CholeskyQR2 route's one-pass bound.

The route skips its second pass when ||R1s^-1||_F^2 <= 144, where R1s is the
Cholesky factor of the column-scaled Gram (unit columns, so its eigenvalues
sigma_i^2 sum to 64). For a given sum of sigma_i^-2 the largest kappa(R1s)
comes from one large eigenvalue, one small one and 62 equal ones; at 144
that is kappa = 34.0 (sigma_max^2 = 22.7, sigma_min^2 = 1/51, the rest 2/3).
"""

from __future__ import annotations

import numpy as np


def near_bound_block(r: int, inv_sum: float, seed: int) -> tuple[np.ndarray, float]:
    """(r x 64 fp32 block with unit columns, kappa(R1s)) whose scaled Gram has
    the spectrum above with sum(sigma^-2) = inv_sum (one large eigenvalue
    22.66, 62 equal ones, one small one)."""
    from scipy.stats import random_correlation

    rng = np.random.default_rng(seed)
    hi = 22.66
    # mid and lo with 62 mid + lo = 64 - hi and 62 / mid + 1 / lo = inv_sum - 1 / hi
    rest = 64.0 - hi
    target = inv_sum - 1.0 / hi
    lo_a, lo_b = 1e-6, rest / 63.0
    for _ in range(200):  # bisection on lo: 62/mid + 1/lo decreases in lo
        lo = 0.5 * (lo_a + lo_b)
        mid = (rest - lo) / 62.0
        if 62.0 / mid + 1.0 / lo > target:
            lo_a = lo
        else:
            lo_b = lo
    eigs = np.array([hi, lo] + [mid] * 62)
    eigs *= 64.0 / eigs.sum()
    C = random_correlation.rvs(eigs, random_state=rng)
    L = np.linalg.cholesky(C)
    Q, _ = np.linalg.qr(rng.standard_normal((r, 64)))
    return (Q @ L.T).astype(np.float32), float(np.sqrt(eigs.max() / eigs.min()))
