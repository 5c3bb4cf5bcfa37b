"""The parity rule of tests/parity.py, pinned from both sides on the CPU.

* It rejects plausible mistakes: a dropped reflector on a 1e-30 column, a
  1e-3 (or uniform 1e-2) error in V and tau at n = 1024, an error of 0.5 on a
  matrix with a zeroed column, a NaN, a 1e-2 error at the most sensitive
  column of a matrix.
* It admits two correct fp32 factorisations of the same input (LAPACK sgeqrf
  from MKL through torch.geqrf, against the C oracle) on every kind of input
  the GPU parity tests feed it: Gaussian up to n = 1024, the benchmark's
  cond-1e2 SVD matrices, zeroed, tiny (1e-30), huge (1e25) and subnormal
  (1e-40) columns; also where the flat bound alone does not (the sensitive
  column 1021 of matrix 63 of the n = 1024 benchmark input).

So a GPU test that passes the rule agrees with the oracle as closely as a
second correct implementation does, and one that makes any of the planted
mistakes fails.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpumode_qr_amd import inputs
from tests.parity import assert_parity, sensitivity, tolerance


def _gauss(batch, n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(batch, n, n, generator=g)


def _extreme(n, cols, scale, seed):
    A = _gauss(2, n, seed)
    A[0, :, cols[0]] *= scale
    A[1, :, cols[1]] *= scale
    A[1, :, cols[2]] *= scale
    return A


def _rejects(*args, **kw):
    with pytest.raises(AssertionError):
        assert_parity(*args, **kw)


def test_rejects_dropped_reflector_on_tiny_column(oracle):
    # The setup of the GPU test of extreme columns: a column scaled by 1e-30
    # in a later panel. Dropping its reflector (tau = 0, V column zero, as a
    # kernel that took the tiny norm for zero would) must fail.
    n, cols = 100, (5, 37, 70)
    A = _extreme(n, cols, 1e-30, seed=n + 7).numpy()
    H, tau = oracle.geqrf(A, nb=16)
    Hb, tb = H.copy(), tau.copy()
    j = cols[1]
    tb[1, j] = 0.0
    Hb[1, j + 1:, j] = 0.0
    assert abs(tau[1, j] - tb[1, j]) > 1.0
    _rejects(A, Hb, tb, H, tau, what="dropped reflector")


@pytest.fixture(scope="module")
def cfg4_first():
    """Matrix 0 of the n = 1024 Gaussian benchmark input, with MKL's factors."""
    A = inputs.config_tensor(inputs.config_spec(4))[:1].contiguous()
    H, tau = torch.geqrf(A)
    return A.numpy(), H.numpy(), tau.numpy()


def test_rejects_small_v_error_at_n1024(cfg4_first):
    A, H, tau = cfg4_first
    Hb = H.copy()
    Hb[0, 700, 300] += 1e-3  # one V entry
    _rejects(A, Hb, tau, H, tau, what="+1e-3 in V")
    Hb = H.copy()
    tb = tau + np.float32(1e-2)
    Hb += np.tril(np.full_like(H[0], 1e-2), -1)[None]
    _rejects(A, Hb, tb, H, tau, what="+1e-2 on all of V and tau")


def test_admits_oracle_against_mkl_at_n1024(oracle, cfg4_first):
    A, H, tau = cfg4_first
    Ho, to = oracle.geqrf(A, nb=16)
    out = assert_parity(A, Ho, to, H, tau, what="oracle vs MKL n=1024")
    assert out["ratio"] < 0.5


@pytest.fixture(scope="module")
def cfg4_m63():
    """Matrix 63 of the n = 1024 Gaussian benchmark input: a small pivot
    (|R_1021,1021| = 0.28, ||a|| = 32) makes column 1021's reflector sensitive."""
    A = inputs.config_tensor(inputs.config_spec(4))[63:64].contiguous()
    H, tau = torch.geqrf(A)
    return A.numpy(), H.numpy(), tau.numpy()


def test_sensitive_column_needs_the_sensitivity_term(oracle, cfg4_m63):
    A, H, tau = cfg4_m63
    Ho, to = oracle.geqrf(A, nb=16)
    with pytest.raises(AssertionError):  # the flat bound alone rejects MKL vs the oracle
        assert_parity(A, H, tau, Ho, to, tol=tolerance(1024), what="flat only")
    out = assert_parity(A, H, tau, Ho, to, what="MKL vs oracle, matrix 63")
    assert out["ratio"] < 0.25
    g = np.maximum(1.0, sensitivity(A, Ho) / 10.0)[0]
    assert g[1021] > 5 and np.mean(g > 1.0) < 0.02  # a few tail columns only


def test_rejects_error_at_the_sensitive_column(cfg4_m63):
    A, H, tau = cfg4_m63
    tb = tau.copy()
    tb[0, 1021] += 1e-2
    _rejects(A, H, tb, H, tau, what="+1e-2 in the sensitive column's tau")
    Hb = H.copy()
    Hb[0, 1023, 1021] += 1e-2
    _rejects(A, Hb, tau, H, tau, what="+1e-2 in the sensitive column's V")


def test_rejects_error_on_zeroed_column_matrix():
    A = _gauss(2, 256, seed=1)
    A[0, :, 85] = 0.0
    H, tau = torch.geqrf(A)
    H, tau = H.numpy(), tau.numpy()
    Hb, tb = H.copy(), tau.copy()
    Hb[0, 200, 120] += 0.5
    tb[0, 120] += 0.5
    _rejects(A.numpy(), Hb, tb, H, tau, what="+0.5 on a singular matrix")
    Hb = H.copy()
    Hb[0, 3, 200] += 1e-3 * np.linalg.norm(A[0, :, 200].numpy())  # an R entry
    _rejects(A.numpy(), Hb, tau, H, tau, what="R error")


def test_rejects_nan():
    A = _gauss(1, 80, seed=2)
    H, tau = torch.geqrf(A)
    H, tau = H.numpy(), tau.numpy()
    Hb = H.copy()
    Hb[0, 50, 10] = np.nan
    _rejects(A.numpy(), Hb, tau, H, tau, what="NaN in V")
    tb = tau.copy()
    tb[0, 3] = np.nan
    _rejects(A.numpy(), H, tb, H, tau, what="NaN in tau")


def test_rejects_subnormal_column_dropped_reflector(oracle):
    # The subnormal floor widens the tolerance for columns at and after a
    # 1e-40 column, yet a dropped reflector there still fails.
    n, cols = 100, (5, 37, 70)
    A = _extreme(n, cols, 1e-40, seed=n + 7).numpy()
    H, tau = oracle.geqrf(A, nb=16)
    Hb, tb = H.copy(), tau.copy()
    tb[1, cols[1]] = 0.0
    Hb[1, cols[1] + 1:, cols[1]] = 0.0
    _rejects(A, Hb, tb, H, tau, what="dropped subnormal reflector")


def test_subnormal_floor_only_from_the_subnormal_column_on():
    # Columns left of the first subnormal column keep the flat bound.
    n, cols = 100, (5, 37, 70)
    A = _extreme(n, cols, 1e-40, seed=n + 7)
    H, tau = torch.geqrf(A)
    H, tau = H.numpy(), tau.numpy()
    Hb = H.copy()
    Hb[1, 60, 20] += 2 * tolerance(n)  # column 20 < 37, matrix 1
    _rejects(A.numpy(), Hb, tau, H, tau, what="before the subnormal column")


KINDS = [
    ("extreme tiny n100", lambda: _extreme(100, (5, 37, 70), 1e-30, 107)),
    ("extreme huge n100", lambda: _extreme(100, (5, 37, 70), 1e25, 107)),
    ("extreme subnormal n100", lambda: _extreme(100, (5, 37, 70), 1e-40, 107)),
    ("extreme tiny n300", lambda: _extreme(300, (20, 150, 290), 1e-30, 307)),
    ("extreme subnormal n300", lambda: _extreme(300, (20, 150, 290), 1e-40, 307)),
    ("gauss n513", lambda: _gauss(2, 513, 5)),
    ("svd cond1e2 n512", lambda: inputs.svd_matrices(2, 512, 2.0,
                                                     torch.Generator().manual_seed(5)).float()),
]


@pytest.mark.parametrize("name,make", KINDS, ids=[k[0] for k in KINDS])
def test_admits_mkl_against_oracle(oracle, name, make):
    A = make().contiguous()
    H, tau = oracle.geqrf(A.numpy(), nb=16)
    Hm, tm = torch.geqrf(A)
    assert_parity(A.numpy(), Hm.numpy(), tm.numpy(), H, tau, what=f"MKL vs oracle {name}")


@pytest.mark.parametrize("kind", ["zero", "tiny", "huge", "subnormal"])
def test_admits_mkl_against_oracle_fallback_inputs(oracle, kind):
    # The inputs of the GPU tests of the CholeskyQR2 route's per-matrix fallback.
    n, cols = 300, (20, 150, 290)
    A = _gauss(3, n, n + 3)
    for b, c in ((0, cols[0]), (1, cols[1]), (1, cols[2])):
        if kind == "zero":
            A[b, :, c] = 0.0
        else:
            A[b, :, c] *= {"tiny": 1e-30, "huge": 1e25, "subnormal": 1e-40}[kind]
    H, tau = oracle.geqrf(A.numpy(), nb=16)
    Hm, tm = torch.geqrf(A)
    assert_parity(A.numpy(), Hm.numpy(), tm.numpy(), H, tau, what=f"MKL vs oracle {kind}")
