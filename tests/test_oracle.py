"""Pins the CPU oracle (oracle/qr_oracle.c) before anything is compared to it.

Independent checks only: LAPACK (MKL sgeqrf) through torch.geqrf live and via
the committed fixtures in tests/golden/, fp64 closed forms, known answers and
fp64 identities. A wrong sign, index or dropped term in the oracle fails at
least one of these.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from gpumode_qr_amd import checker
from tests.parity import assert_parity, tolerance

GOLDEN = Path(__file__).resolve().parent / "golden" / "geqrf_mkl.npz"


def _golden():
    z = np.load(GOLDEN)
    names = sorted({k.split("__")[0] for k in z.files})
    return {nm: (z[nm + "__A"], z[nm + "__H"], z[nm + "__tau"]) for nm in names}


@pytest.mark.parametrize("name", sorted(n for n in _golden() if n != "rank1_n16"))
def test_oracle_matches_mkl_fixtures(oracle, name):
    A, H_ref, tau_ref = _golden()[name]
    for nb in (0, 4):
        H, tau = oracle.geqrf(A, nb=nb)
        assert_parity(A, H, tau, H_ref, tau_ref, what=f"{name} nb={nb}")


def test_oracle_rank1_first_reflector(oracle):
    # After the first reflector a rank-1 matrix's trailing block is rounding
    # noise, so only column 0 and row 0 are well defined.
    A, H_ref, tau_ref = _golden()["rank1_n16"]
    H, tau = oracle.geqrf(A)
    tol = tolerance(16)
    np.testing.assert_allclose(tau[:, 0], tau_ref[:, 0], atol=tol)
    np.testing.assert_allclose(H[:, 1:, 0], H_ref[:, 1:, 0], atol=tol)
    scale = np.abs(A).max()
    np.testing.assert_allclose(H[:, 0, :], H_ref[:, 0, :], atol=tol * scale * 16)


@pytest.mark.parametrize("n,nb", [(7, 0), (31, 8), (64, 16), (100, 16), (130, 32)])
def test_oracle_matches_torch_geqrf_live(oracle, n, nb):
    g = torch.Generator().manual_seed(n * 7 + nb)
    A = torch.randn(4, n, n, generator=g)
    H_ref, tau_ref = torch.geqrf(A)
    H, tau = oracle.geqrf(A.numpy(), nb=nb)
    assert_parity(A.numpy(), H, tau, H_ref.numpy(), tau_ref.numpy(), what=f"n={n} nb={nb}")


def test_oracle_2x2_closed_form(oracle):
    # alpha=3, x=4: beta=-5, tau=(beta-alpha)/beta=1.6, v=4/(3+5)=0.5;
    # second column [1,2] -> [1,2] - tau*(1+0.5*2)*[1,0.5] = [-2.2, 0.4].
    H, tau = oracle.geqrf(np.array([[3.0, 1.0], [4.0, 2.0]], dtype=np.float32))
    np.testing.assert_allclose(H, [[-5.0, -2.2], [0.5, 0.4]], rtol=0, atol=1e-6)
    np.testing.assert_allclose(tau, [1.6, 0.0], rtol=0, atol=1e-7)


def test_oracle_1x1(oracle):
    H, tau = oracle.geqrf(np.array([[[-2.5]]], dtype=np.float32))
    assert H[0, 0, 0] == np.float32(-2.5) and tau[0, 0] == 0.0


def test_oracle_upper_triangular_is_fixed_point(oracle):
    g = torch.Generator().manual_seed(3)
    A = torch.triu(torch.randn(3, 40, 40, generator=g)).numpy()
    H, tau = oracle.geqrf(A, nb=16)
    assert np.array_equal(H, A)
    assert np.all(tau == 0.0)


def test_oracle_zero_column_and_last_tau(oracle):
    g = torch.Generator().manual_seed(4)
    A = torch.randn(2, 30, 30, generator=g)
    A[:, :, 11] = 0.0
    H, tau = oracle.geqrf(A.numpy(), nb=8)
    assert np.all(tau[:, 11] == 0.0)
    assert np.all(H[:, 11, 11] == 0.0)
    assert np.all(H[:, 12:, 11] == 0.0)
    assert np.all(tau[:, -1] == 0.0)


def _slarfg_fp64(alpha: float, x: np.ndarray):
    xn = float(np.sqrt(np.sum(np.asarray(x, np.float64) ** 2)))
    if xn == 0.0:
        return alpha, np.asarray(x, np.float64), 0.0
    beta = -np.copysign(np.hypot(alpha, xn), alpha)
    return beta, np.asarray(x, np.float64) / (alpha - beta), (beta - alpha) / beta


@pytest.mark.parametrize("scale", [1.0, 1e-30, 1e25, 1e-40, 1e-44])
@pytest.mark.parametrize("alpha_kind", ["pos", "neg", "zero"])
def test_oracle_slarfg_closed_form(oracle, scale, alpha_kind):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(9) * scale).astype(np.float32)
    alpha = {"pos": 0.7, "neg": -1.3, "zero": 0.0}[alpha_kind] * scale
    alpha = float(np.float32(alpha))
    beta, v, tau = oracle.slarfg(alpha, x)
    beta_r, v_r, tau_r = _slarfg_fp64(alpha, x.astype(np.float64))
    assert tau == pytest.approx(tau_r, rel=4e-6, abs=4e-7)
    assert beta == pytest.approx(beta_r, rel=4e-6)
    np.testing.assert_allclose(v, v_r, rtol=1e-5, atol=1e-6)


def test_oracle_tau_range(oracle):
    # tau = 1 - alpha / beta with |beta| >= |alpha| and sign(beta) = -sign(alpha),
    # so every tau lies in [1, 2], or is exactly 0 when the column below the
    # diagonal is already zero (here column 5 of matrix 1 and every last column).
    rng = np.random.default_rng(7)
    A = rng.standard_normal((4, 50, 50)).astype(np.float32)
    A[1, :, 5] = 0.0
    _, tau = oracle.geqrf(A, nb=16)
    nz = tau[tau != 0]
    assert np.all(nz >= 1 - 1e-6) and np.all(nz <= 2 + 1e-6)
    assert tau[1, 5] == 0 and np.all(tau[:, -1] == 0)
    assert nz.size == tau.size - 5


def test_oracle_slarfg_degenerate(oracle):
    beta, v, tau = oracle.slarfg(2.0, np.zeros(5, np.float32))
    assert (beta, tau) == (2.0, 0.0) and np.all(v == 0.0)
    beta, v, tau = oracle.slarfg(-3.0, np.zeros(0, np.float32))
    assert (beta, tau) == (-3.0, 0.0)


def test_oracle_snrm2(oracle):
    rng = np.random.default_rng(1)
    for scale in (1.0, 1e-30, 1e30):
        x = (rng.standard_normal(50) * scale).astype(np.float32)
        ref = float(np.sqrt(np.sum(x.astype(np.float64) ** 2)))
        assert oracle.snrm2(x) == pytest.approx(ref, rel=2e-6)


@pytest.mark.parametrize("m,k", [(16, 16), (40, 16), (100, 7), (64, 32)])
def test_oracle_larft_identity(oracle, m, k):
    # I - V T V^T must equal the product of the panel's reflectors (LAPACK
    # orgqr via torch.linalg.householder_product, fp64).
    g = torch.Generator().manual_seed(m + k)
    P = torch.randn(m, k, generator=g).numpy()
    Hp, tau = oracle.geqr2(P)
    T = oracle.larft(Hp, tau)
    V = np.tril(Hp.astype(np.float64), -1)
    V[np.arange(k), np.arange(k)] = 1.0
    Q_wy = np.eye(m) - V @ T.astype(np.float64) @ V.T
    Hfull = np.zeros((m, m), np.float64)
    Hfull[:, :k] = Hp
    taufull = np.zeros(m, np.float64)
    taufull[:k] = tau
    Q_ref = torch.linalg.householder_product(torch.from_numpy(Hfull), torch.from_numpy(taufull)).numpy()
    assert np.abs(Q_wy - Q_ref).max() < 8 * m * 2**-23
    # T is upper triangular with tau on the diagonal.
    assert np.all(np.tril(T, -1) == 0.0)
    np.testing.assert_array_equal(np.diag(T), tau)


@pytest.mark.parametrize("m,c,k", [(32, 20, 16), (77, 5, 16), (64, 64, 8)])
def test_oracle_larfb_matches_fp64(oracle, m, c, k):
    g = torch.Generator().manual_seed(m * c + k)
    P = torch.randn(m, k, generator=g).numpy()
    C = torch.randn(m, c, generator=g).numpy()
    Hp, tau = oracle.geqr2(P)
    T = oracle.larft(Hp, tau)
    out = oracle.larfb_lt(Hp, T, C)
    V = np.tril(Hp.astype(np.float64), -1)
    V[np.arange(k), np.arange(k)] = 1.0
    ref = C - V @ (T.astype(np.float64).T @ (V.T @ C.astype(np.float64)))
    assert np.abs(out - ref).max() <= 16 * m * 2**-23 * max(1.0, np.abs(C).max())


def test_oracle_orgqr_matches_householder_product(oracle):
    g = torch.Generator().manual_seed(11)
    A = torch.randn(1, 37, 37, generator=g).numpy()
    H, tau = oracle.geqrf(A)
    Q = oracle.orgqr(H[0], tau[0])
    Q_ref = torch.linalg.householder_product(torch.from_numpy(H[0]), torch.from_numpy(tau[0])).numpy()
    assert np.abs(Q - Q_ref).max() < 1e-5


@pytest.mark.parametrize("n", [32, 64])
def test_oracle_passes_gates_on_stress_structures(oracle, n):
    from gpumode_qr_amd import inputs

    for prob in inputs.stress_cases(n=n, batch=2, device="cpu"):
        A = prob.tensor
        H, tau = oracle.geqrf(A.numpy(), nb=16)
        res = checker.check(A, torch.from_numpy(H), torch.from_numpy(tau))
        assert res.passed, (prob.name, res.as_dict())


@pytest.mark.parametrize("n", [2, 3, 4, 8, 16, 64])
def test_parity_tolerance_admits_mkl(oracle, n):
    # The stated parity tolerance must accept any correct fp32 factorisation:
    # MKL's sgeqrf against the oracle on the same Gaussian matrices.
    rng = np.random.default_rng(n)
    A = rng.standard_normal((1500 if n <= 16 else 200, n, n)).astype(np.float32)
    H, tau = oracle.geqrf(A, nb=16)
    Hm, tm = torch.geqrf(torch.from_numpy(A))
    assert_parity(A, Hm.numpy(), tm.numpy(), H, tau, what=f"MKL vs oracle n={n}")


def test_gates_catch_a_planted_oracle_mistake(oracle):
    # Plant a plausible bug in the oracle's output (one reflector's tau with the
    # wrong sign, then a transposed R block) and check the FP64 gates reject it.
    g = torch.Generator().manual_seed(5)
    A = torch.randn(2, 24, 24, generator=g)
    H, tau = oracle.geqrf(A.numpy())
    assert checker.check(A, torch.from_numpy(H), torch.from_numpy(tau)).passed
    bad_tau = tau.copy()
    bad_tau[:, 3] = -bad_tau[:, 3]
    assert not checker.check(A, torch.from_numpy(H), torch.from_numpy(bad_tau)).passed
    bad_H = H.copy()
    bad_H[:, 2, 5], bad_H[:, 5, 2] = H[:, 5, 2], H[:, 2, 5]
    assert not checker.check(A, torch.from_numpy(bad_H), torch.from_numpy(tau)).passed
