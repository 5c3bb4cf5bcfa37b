"""CPU model of the CholeskyQR2 block route (gpumode_qr_amd/csrc/qr_cholqr.hip).

The route replaces the Householder column steps of a 64-column outer block by
CholeskyQR2 (two Cholesky-based passes) and the Householder reconstruction of
Ballard, Demmel, Grigori, Jacobsen, Knight and Nguyen (IPDPS 2014): the LU of
Q[0:64] - S without pivoting, S_k = -sign of the k-th pivot candidate. These
tests restate those steps in numpy (fp32 arithmetic, as the kernels compute)
and pin them to LAPACK sgeqrf (scipy) and the C oracle on the same block:

* V, tau and R agree within the GPU parity tolerance (4 r eps32);
* the 16 x 16 diagonal blocks of T = -U S L1^-T equal each panel's larft T
  (the only part of T the trailing update reads);
* the blocked LU (16 x 16 diagonal blocks) gives the unblocked LU's factors
  and signs;
* planting the opposite sign rule flips R's first diagonal sign and fails
  parity.

The model is test code only; the product path is the HIP kernels.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.linalg as sl
from scipy.linalg import lapack

from tests.blocks import near_bound_block
from tests.parity import tolerance

F32 = np.float32


def _chol_upper(G):
    """Upper Cholesky G = R^T R in fp32 (row-by-row, as the blocked kernel's
    16 x 16 steps compute it)."""
    n = G.shape[0]
    A = G.astype(F32).copy()
    R = np.zeros_like(A)
    for k in range(n):
        piv = A[k, k]
        assert piv > 0
        rs = np.sqrt(piv, dtype=F32)
        R[k, k] = rs
        R[k, k + 1:] = A[k, k + 1:] / rs
        A[k + 1:, k + 1:] -= np.outer(R[k, k + 1:], R[k, k + 1:])
    return R


def _inv_upper(R):
    return sl.solve_triangular(R.astype(F32), np.eye(R.shape[0], dtype=F32)).astype(F32)


def _signed_lu(Q, flip=False):
    """LU of Q - S without pivoting, S_k = -sign(candidate) (sign(0) = +)."""
    b = Q.shape[0]
    A = Q.astype(F32).copy()
    S = np.zeros(b, F32)
    L = np.eye(b, dtype=F32)
    U = np.zeros((b, b), F32)
    for k in range(b):
        q = A[k, k]
        s = F32(-1.0) if q >= 0 else F32(1.0)
        if flip:
            s = -s
        S[k] = s
        pv = q - s
        U[k, k] = pv
        U[k, k + 1:] = A[k, k + 1:]
        L[k + 1:, k] = A[k + 1:, k] / pv
        A[k + 1:, k + 1:] -= np.outer(L[k + 1:, k], U[k, k + 1:])
    return L, U, S


def _signed_lu_blocked(Q, nb=16):
    """The kernel's blocked form: 16 x 16 diagonal LUs, panel solves with the
    diagonal blocks' inverses, Schur updates."""
    b = Q.shape[0]
    A = Q.astype(F32).copy()
    S = np.zeros(b, F32)
    for K in range(0, b, nb):
        d = slice(K, K + nb)
        Ld, Ud, Sd = _signed_lu(A[d, d])
        S[d] = Sd
        A[d, d] = np.tril(Ld, -1) + Ud
        if K + nb < b:
            r = slice(K + nb, b)
            A[d, r] = (np.linalg.inv(Ld).astype(F32) @ A[d, r]).astype(F32)
            A[r, d] = (A[r, d] @ _inv_upper(Ud)).astype(F32)
            A[r, r] -= (A[r, d] @ A[d, r]).astype(F32)
    return np.tril(A, -1) + np.eye(b, dtype=F32), np.triu(A), S


def one_pass_ok(Ab):
    """The kernel's test for skipping the second pass: ||R1s^-1||_F^2 <= 144,
    i.e. kappa(R1s) <= 8 ||R1s^-1||_F <= 96 for unit-norm columns."""
    G1 = (Ab.T @ Ab).astype(F32)
    d = np.sqrt(np.diag(G1)).astype(F32)
    R1s = _chol_upper((G1 / np.outer(d, d)).astype(F32))
    return float((_inv_upper(R1s).astype(np.float64) ** 2).sum()) <= 144.0


def cq_block(Ab, flip=False, blocked=False, passes=2):
    """(H block, tau, T) of an r x 64 block by the route's steps (passes=1: R2 = I)."""
    r, b = Ab.shape
    G1 = (Ab.T @ Ab).astype(F32)
    d = np.sqrt(np.diag(G1)).astype(F32)
    R1s = _chol_upper((G1 / np.outer(d, d)).astype(F32))
    R1 = (R1s * d[None, :]).astype(F32)
    M1 = (_inv_upper(R1s) / d[:, None]).astype(F32)
    X = (Ab @ M1).astype(F32)
    R2 = _chol_upper((X.T @ X).astype(F32)) if passes == 2 else np.eye(b, dtype=F32)
    Rinv = (M1 @ _inv_upper(R2)).astype(F32)
    Rc = (R2 @ R1).astype(F32)
    Qt = (Ab[:b] @ Rinv).astype(F32)
    if blocked:
        L, U, S = _signed_lu_blocked(Qt)
    else:
        L, U, S = _signed_lu(Qt, flip=flip)
    M = (Rinv @ _inv_upper(U)).astype(F32)
    H = np.zeros_like(Ab)
    H[:b] = np.triu(S[:, None] * Rc) + np.tril(L, -1)
    H[b:] = (Ab[b:] @ M).astype(F32)
    tau = (-np.diag(U) * S).astype(F32)
    T = -(U * S[None, :]) @ np.linalg.inv(L).T
    return H, tau, T


def _block(kind, r, seed):
    rng = np.random.default_rng(seed)
    if kind == "gauss":
        return rng.standard_normal((r, 64)).astype(F32)
    U, _ = np.linalg.qr(rng.standard_normal((r, r)))
    V, _ = np.linalg.qr(rng.standard_normal((64, 64)))
    s = np.logspace(0, -2, 64)
    return ((U[:, :64] * s) @ V.T).astype(F32)


def _errors(Ab, H, tau, Hr, taur):
    colnorm = np.linalg.norm(Ab.astype(np.float64), axis=0)
    dV = np.abs(np.tril(H, -1).astype(np.float64) - np.tril(Hr, -1)).max()
    dR = (np.abs(np.triu(H[:64]).astype(np.float64) - np.triu(Hr[:64])) / colnorm).max()
    dt = np.abs(tau.astype(np.float64) - taur).max()
    return dV, dR, dt


@pytest.mark.parametrize("blocked", [False, True], ids=["lu", "blocked_lu"])
@pytest.mark.parametrize("kind,r", [("gauss", 65), ("gauss", 300), ("gauss", 2048),
                                    ("cond1e2", 512)])
def test_route_matches_lapack_sgeqrf(kind, r, blocked):
    Ab = _block(kind, r, seed=r)
    H, tau, _ = cq_block(Ab, blocked=blocked)
    Hr, taur, _, info = lapack.sgeqrf(Ab)
    assert info == 0
    assert max(_errors(Ab, H, tau, Hr, taur)) <= tolerance(r)


@pytest.mark.parametrize("r", [512, 2048, 4096])
def test_one_pass_route_matches_lapack(r):
    """Blocks that pass the one-pass test: CholeskyQR with a single pass gives
    the same (V, tau, R) as LAPACK within the tolerance, like two passes."""
    Ab = _block("gauss", r, seed=r + 1)
    assert one_pass_ok(Ab)
    H, tau, _ = cq_block(Ab, passes=1)
    Hr, taur, _, _ = lapack.sgeqrf(Ab)
    assert max(_errors(Ab, H, tau, Hr, taur)) <= tolerance(r)


@pytest.mark.parametrize("r", [128, 160, 1024])
@pytest.mark.parametrize("inv_sum", [140.0, 143.5])
def test_one_pass_at_the_bound_matches_lapack(r, inv_sum):
    """The worst block the one-pass test admits: sum(sigma^-2) just under 144
    with the spectrum that maximises kappa(R1s) (about 34). One pass stays
    within the flat tolerance of LAPACK sgeqrf, at a tenth of it or less."""
    Ab, kappa = near_bound_block(r, inv_sum, seed=r)
    assert kappa > 30
    assert one_pass_ok(Ab)
    H, tau, _ = cq_block(Ab, passes=1, blocked=True)
    Hr, taur, _, _ = lapack.sgeqrf(Ab)
    assert max(_errors(Ab, H, tau, Hr, taur)) <= 0.25 * tolerance(r)


def test_one_pass_test_rejects_just_over_the_bound():
    Ab, _ = near_bound_block(160, 150.0, seed=1)
    assert not one_pass_ok(Ab)


def test_one_pass_test_rejects_ill_conditioned_block():
    Ab = _block("cond1e2", 512, seed=9)  # kappa = 100 inside the block
    assert not one_pass_ok(Ab)


def test_route_matches_oracle(oracle):
    Ab = _block("gauss", 400, seed=3)
    H, tau, _ = cq_block(Ab)
    Ho, tauo = oracle.geqr2(Ab)
    assert max(_errors(Ab, H, tau, Ho, tauo)) <= tolerance(400)


def test_diagonal_t_blocks_are_panel_larft(oracle):
    Ab = _block("gauss", 700, seed=5)
    H, tau, T = cq_block(Ab)
    for q in range(4):
        c = slice(16 * q, 16 * q + 16)
        Tq = oracle.larft(H[16 * q:, c], tau[c])
        assert np.abs(Tq - T[c, c]).max() <= 4 * tolerance(700)


def test_blocked_lu_equals_unblocked():
    rng = np.random.default_rng(11)
    Q, _ = np.linalg.qr(rng.standard_normal((200, 64)))
    Qt = Q[:64].astype(F32)
    L0, U0, S0 = _signed_lu(Qt)
    L1, U1, S1 = _signed_lu_blocked(Qt)
    assert np.array_equal(S0, S1)
    assert np.abs(L0 - L1).max() <= 1e-5 and np.abs(U0 - U1).max() <= 1e-5
    assert np.all(np.abs(np.diag(U1)) >= 1.0)


def test_planted_sign_rule_fails():
    """The opposite sign rule is a valid factorisation too, but not slarfg's:
    R's first diagonal entry flips sign and parity against LAPACK fails."""
    Ab = _block("gauss", 300, seed=7)
    H, tau, _ = cq_block(Ab, flip=True)
    Hr, taur, _, _ = lapack.sgeqrf(Ab)
    assert np.sign(H[0, 0]) == -np.sign(Hr[0, 0])
    assert max(_errors(Ab, H, tau, Hr, taur)) > 100 * tolerance(300)
