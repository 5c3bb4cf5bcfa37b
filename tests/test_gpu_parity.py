"""Parity of the gfx950 HIP path against the CPU oracle, through the C ABI.

Each test prints its case before touching the GPU so a failing run names it,
and every comparison prints its largest errors and tolerance ratio.
Tolerance (tests/parity.py): |dV|, |dtau|, |dR|/||A[:,j]||_2 <= 4 n eps32 for
n > 64 (plus fp32's subnormal floor from a subnormal column on); the
cond-1e6 half of the stress config and near-duplicate columns are gates-only.
Route and schedule choices are passed per call (hip_qr.options); the library
reads no environment variable.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpumode_qr_amd import checker, hip_qr, inputs
from tests.blocks import near_bound_block
from tests.parity import assert_parity

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _say(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _gauss(batch, n, seed, cond=0.0):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(batch, n, n, generator=g)
    if cond:
        A = A * torch.logspace(0, -cond, n)
    return A


def _run(A_cpu, **opts):
    H, tau = hip_qr.geqrf(A_cpu.to(DEV), options=hip_qr.options(**opts) if opts else None)
    torch.cuda.synchronize()
    return H.cpu(), tau.cpu()


def _run_ws(A_cpu, **opts):
    """geqrf with a workspace of our own, so the route codes can be read."""
    b, n, _ = A_cpu.shape
    ws = torch.empty(hip_qr.workspace_bytes(b, n), dtype=torch.uint8, device=DEV)
    H, tau = hip_qr.geqrf(A_cpu.to(DEV), workspace=ws,
                          options=hip_qr.options(**opts) if opts else None)
    torch.cuda.synchronize()
    return H.cpu(), tau.cpu(), hip_qr.route_codes(ws, b, n).cpu()


@pytest.mark.parametrize("n", [1, 2, 3, 8, 17, 32, 33, 48, 63, 64])
@pytest.mark.parametrize("batch", [1, 5])
def test_fused_smalln_vs_oracle(oracle, n, batch):
    _say(f"fused_smalln n={n} batch={batch}")
    A = _gauss(batch, n, seed=100 + n + batch)
    H, tau = hip_qr.fused_smalln(A.to(DEV))
    torch.cuda.synchronize()
    H, tau = H.cpu().numpy(), tau.cpu().numpy()
    H_ref, tau_ref = oracle.geqrf(A.numpy())
    assert_parity(A.numpy(), H, tau, H_ref, tau_ref, what=f"smalln n={n}")
    assert np.all(tau[:, -1] == 0.0)


@pytest.mark.parametrize("n", [64, 40])
@pytest.mark.parametrize("scale", [1e-30, 1e25, 1e-40, 0.0], ids=["tiny", "huge", "denormal", "zero"])
def test_fused_smalln_extreme_columns_vs_oracle(oracle, n, scale):
    """A column outside the fast reflector's range in every panel (matrix k has
    it in column 16 k + 5 of its panel k, one column per matrix): each panel's
    fast pass hands over to the out-of-line safe re-run of that panel, for the
    vectorised n = 64 kernel and the general one."""
    _say(f"fused_smalln extreme columns n={n} scale={scale:g}")
    A = _gauss(5, n, seed=n + 11)
    for b in range(4):
        col = 16 * b + 5
        if col < n:
            A[b, :, col] *= scale
    H, tau = hip_qr.fused_smalln(A.to(DEV))
    torch.cuda.synchronize()
    H_ref, tau_ref = oracle.geqrf(A.numpy())
    assert_parity(A.numpy(), H.cpu().numpy(), tau.cpu().numpy(), H_ref, tau_ref,
                  what=f"smalln extreme n={n} scale={scale:g}")


@pytest.mark.parametrize("n", [65, 80, 96, 100, 128, 144, 176, 192])
def test_fused_midn_vs_oracle(oracle, n):
    """64 < n <= 192 in one launch: a workgroup per matrix, a wave per strip."""
    _say(f"fused mid-n n={n} batch=3")
    A = _gauss(3, n, seed=300 + n)
    H, tau = hip_qr.fused_smalln(A.to(DEV))
    torch.cuda.synchronize()
    H_ref, tau_ref = oracle.geqrf(A.numpy())
    assert_parity(A.numpy(), H.cpu().numpy(), tau.cpu().numpy(), H_ref, tau_ref,
                  what=f"midn n={n}")
    assert np.all(tau.cpu().numpy()[:, -1] == 0.0)


@pytest.mark.parametrize("n", [128, 100])
@pytest.mark.parametrize("scale", [1e-30, 1e25, 1e-40, 0.0], ids=["tiny", "huge", "denormal", "zero"])
def test_fused_midn_extreme_columns_vs_oracle(oracle, n, scale):
    """A column outside the fast reflector's range in a panel of each matrix
    (matrix b: column 16 b + 5 of panel b, last matrix: the last panel's first
    column): the panel's fast pass hands over to the rolled safe path."""
    _say(f"fused mid-n extreme columns n={n} scale={scale:g}")
    nr = (n + 15) // 16
    A = _gauss(nr, n, seed=n + 17)
    for b in range(nr):
        col = min(16 * b + 5, n - 1) if b < nr - 1 else 16 * (nr - 1)
        A[b, :, col] *= scale
    H, tau = hip_qr.fused_smalln(A.to(DEV))
    torch.cuda.synchronize()
    H_ref, tau_ref = oracle.geqrf(A.numpy())
    assert_parity(A.numpy(), H.cpu().numpy(), tau.cpu().numpy(), H_ref, tau_ref,
                  what=f"midn extreme n={n} scale={scale:g}")


def test_fused_midn_strided_input(oracle):
    _say("fused mid-n strided (transposed) input n=150")
    A = _gauss(2, 150, seed=8)
    At = A.transpose(1, 2).contiguous().transpose(1, 2)  # same values, column-major
    H, tau = hip_qr.fused_smalln(At.to(DEV))
    torch.cuda.synchronize()
    H_ref, tau_ref = oracle.geqrf(A.numpy())
    assert_parity(A.numpy(), H.cpu().numpy(), tau.cpu().numpy(), H_ref, tau_ref,
                  what="midn strided n=150")


@pytest.mark.parametrize("n,batch,fused", [(80, 3, True), (176, 40, True), (192, 682, True),
                                           (192, 683, False), (176, 800, False)])
def test_geqrf_mid_n_route_choice(oracle, n, batch, fused):
    """geqrf's default for 64 < n <= 192: the whole matrix in the fused kernel
    up to batch * ceil(n / 16) = 8192 (bit for bit what midn=2 gives), the
    blocked route above. midn=0 is the blocked route throughout."""
    _say(f"mid-n route choice n={n} batch={batch} fused={fused}")
    A = _gauss(batch, n, seed=n + batch).to(DEV)
    H, tau = hip_qr.geqrf(A)
    Hf, tf = hip_qr.geqrf(A, options=hip_qr.options(midn=2))
    Hb, tb = hip_qr.geqrf(A, options=hip_qr.options(midn=0))
    torch.cuda.synchronize()
    assert (torch.equal(H, Hf) and torch.equal(tau, tf)) == fused
    assert not torch.equal(Hf, Hb)  # two different kernels: not the same bits
    res = checker.check(A.cpu(), H.cpu(), tau.cpu())
    assert res.passed, res.as_dict()
    idx = [0, batch - 1]
    A_s = A[idx].cpu().numpy()
    H_ref, tau_ref = oracle.geqrf(A_s, nb=16)
    assert_parity(A_s, H[idx].cpu().numpy(), tau[idx].cpu().numpy(), H_ref, tau_ref,
                  what=f"route choice n={n} b={batch}")


@pytest.mark.parametrize("n,batch,tail", [(352, 3, True), (300, 40, True), (1100, 2, True),
                                          (300, 500, False)])
def test_geqrf_last_columns_in_fused_kernel(oracle, n, batch, tail):
    """The blocked route hands its last r <= 192 columns to the fused mid-n
    kernel, in place, while batch * ceil(r / 16) <= 2048 (midn=2 always,
    midn=0 never), and otherwise its last r <= 64 columns to the small-n
    kernel: the default equals midn=2 bit for bit when the bound holds and
    neither forced route when it does not. All three match the oracle."""
    _say(f"last columns in the fused kernel n={n} batch={batch} tail={tail}")
    A = _gauss(batch, n, seed=n + 2 * batch).to(DEV)
    H, tau = hip_qr.geqrf(A)
    Hf, tf = hip_qr.geqrf(A, options=hip_qr.options(midn=2))
    Hb, tb = hip_qr.geqrf(A, options=hip_qr.options(midn=0))
    torch.cuda.synchronize()
    assert (torch.equal(H, Hf) and torch.equal(tau, tf)) == tail
    assert not torch.equal(H, Hb) and not torch.equal(Hf, Hb)
    idx = [0, batch - 1]
    A_s = A[idx].cpu().numpy()
    H_ref, tau_ref = oracle.geqrf(A_s, nb=16)
    for Hy, ty, what in ((H, tau, "default"), (Hf, tf, "fused tail"), (Hb, tb, "blocked")):
        assert_parity(A_s, Hy[idx].cpu().numpy(), ty[idx].cpu().numpy(), H_ref, tau_ref,
                      what=f"n={n} b={batch} {what}")


@pytest.mark.parametrize("n,batch", [(80, 1500), (192, 600)])
def test_fused_midn_many_matrices(oracle, n, batch):
    """Many workgroups per CU over the launch (the fused kernel's largest
    default batches): gates on the whole batch, oracle parity on three
    matrices spread over it."""
    _say(f"fused mid-n many matrices n={n} batch={batch}")
    A = _gauss(batch, n, seed=n + 3 * batch)
    H, tau = hip_qr.fused_smalln(A.to(DEV))
    torch.cuda.synchronize()
    H, tau = H.cpu(), tau.cpu()
    assert torch.isfinite(H).all() and torch.isfinite(tau).all()
    res = checker.check(A, H, tau)
    assert res.passed, res.as_dict()
    idx = [0, batch // 2, batch - 1]
    H_ref, tau_ref = oracle.geqrf(A[idx].numpy())
    assert_parity(A[idx].numpy(), H[idx].numpy(), tau[idx].numpy(), H_ref, tau_ref,
                  what=f"midn many n={n} b={batch}")


def test_fused_midn_padded_input_bitwise(oracle):
    """Unit column stride with padded rows and batch is read in place; the
    column-major view of the same values gives the same bits."""
    n = 100
    _say(f"fused mid-n padded input (n={n})")
    base = torch.randn(2, n + 3, n + 7, generator=torch.Generator().manual_seed(5))
    Ap = base.to(DEV)[:, 1:n + 1, 2:n + 2]
    Ac = Ap.transpose(1, 2).contiguous().transpose(1, 2)
    Hp, tp = hip_qr.fused_smalln(Ap)
    Hc, tc = hip_qr.fused_smalln(Ac)
    torch.cuda.synchronize()
    assert torch.equal(Hp, Hc) and torch.equal(tp, tc)
    H_ref, tau_ref = oracle.geqrf(Ap.cpu().numpy())
    assert_parity(Ap.cpu().numpy(), Hp.cpu().numpy(), tp.cpu().numpy(), H_ref, tau_ref,
                  what="midn padded n=100")


def test_fused_smalln_strided_input(oracle):
    _say("fused_smalln strided (transposed) input n=40")
    A = _gauss(3, 40, seed=7)
    At = A.transpose(1, 2).contiguous().transpose(1, 2)  # same values, column-major strides
    assert not At.is_contiguous()
    H, tau = hip_qr.geqrf(At.to(DEV))
    torch.cuda.synchronize()
    H_ref, tau_ref = oracle.geqrf(A.numpy())
    assert_parity(A.numpy(), H.cpu().numpy(), tau.cpu().numpy(), H_ref, tau_ref)


def _oracle_panels(oracle, blk, nfact):
    """Oracle blocked factorisation of the first nfact 16-wide panels of blk
    (r, width): returns (H, taus, Ts) with the trailing columns updated."""
    H = blk.copy()
    r = H.shape[0]
    taus, Ts = [], []
    for q in range(nfact):
        c0 = 16 * q
        Hq, tq = oracle.geqr2(H[c0:, c0:c0 + 16])
        H[c0:, c0:c0 + 16] = Hq
        Tq = oracle.larft(Hq, tq)
        if H.shape[1] > c0 + 16:
            H[c0:, c0 + 16:] = oracle.larfb_lt(Hq, Tq, H[c0:, c0 + 16:])
        taus.append(tq)
        Ts.append(Tq)
    return H, taus, Ts


@pytest.mark.parametrize("r,kw", [(16, 16), (17, 16), (40, 16), (64, 16), (100, 16), (256, 16),
                                  (300, 16), (777, 16), (1024, 16), (2048, 16), (2049, 16),
                                  (3000, 16), (64, 5), (20, 13)])
def test_panel_vs_oracle(oracle, r, kw):
    _say(f"panel p=0 r={r} kw={kw}")
    g = torch.Generator().manual_seed(r * 31 + kw)
    P = torch.randn(3, r, kw, generator=g)
    Hp, tau, T = hip_qr.panel(P.to(DEV))
    torch.cuda.synchronize()
    Hp, tau, T = Hp.cpu().numpy(), tau.cpu().numpy(), T.cpu().numpy()
    for b in range(3):
        Hr, tr = oracle.geqr2(P[b].numpy())
        Tr = oracle.larft(Hr, tr)
        tol = 4 * r * 2**-23
        colnorm = np.linalg.norm(P[b].numpy().astype(np.float64), axis=0)
        up = np.triu(np.ones((r, kw), bool))
        dH = np.abs(Hp[b].astype(np.float64) - Hr)
        assert (np.where(up, dH / colnorm, 0)).max() <= tol, "R"
        assert (np.where(~up, dH, 0)).max() <= tol, "V"
        assert np.abs(tau[b] - tr).max() <= tol, "tau"
        assert np.abs(T[b, :kw, :kw] - Tr).max() <= 4 * tol, "T"
        assert np.all(T[b, kw:, :] == 0) and np.all(T[b, :, kw:] == 0)


@pytest.mark.parametrize("r,p,kw", [(48, 1, 16), (100, 2, 16), (300, 3, 16), (512, 7, 16),
                                    (2048, 3, 16), (90, 5, 10), (3000, 2, 16)])
def test_panel_left_looking_vs_oracle(oracle, r, p, kw):
    _say(f"panel left-looking r={r} p={p} kw={kw}")
    g = torch.Generator().manual_seed(r + 7 * p + kw)
    blk = torch.randn(2, r, 16 * p + kw, generator=g).numpy()
    for b in range(2):
        # panels 0..p-1 factored by the oracle; panel p still raw
        Hpre, _, Ts = _oracle_panels(oracle, np.concatenate(
            [blk[b][:, :16 * p], np.zeros((r, 0), np.float32)], axis=1), p)
        start = np.concatenate([Hpre, blk[b][:, 16 * p:]], axis=1)
        T_prev = torch.from_numpy(np.stack(Ts)[None]).to(DEV)
        Hg, tau, T = hip_qr.panel(torch.from_numpy(start[None]).to(DEV), p=p, T_prev=T_prev)
        torch.cuda.synchronize()
        Hg, tau, T = Hg.cpu().numpy()[0], tau.cpu().numpy()[0], T.cpu().numpy()[0]
        Href, taus, Trefs = _oracle_panels(oracle, blk[b], p + 1)
        assert np.array_equal(Hg[:, :16 * p], start[:, :16 * p])  # earlier panels untouched
        tol = 4 * r * 2**-23
        colnorm = np.linalg.norm(blk[b][:, 16 * p:].astype(np.float64), axis=0)
        up = np.triu(np.ones((r, kw), bool), k=-16 * p)
        dH = np.abs(Hg[:, 16 * p:].astype(np.float64) - Href[:, 16 * p:])
        assert (np.where(up, dH / colnorm, 0)).max() <= tol, "R"
        assert (np.where(~up, dH, 0)).max() <= tol, "V"
        assert np.abs(tau - taus[p]).max() <= tol, "tau"
        assert np.abs(T[:kw, :kw] - Trefs[p]).max() <= 4 * tol, "T"


@pytest.mark.parametrize("r,p,kw", [(100, 0, 16), (120, 3, 16), (200, 2, 16), (250, 3, 9)])
def test_panel_many_matrices_vs_oracle(oracle, r, p, kw):
    """More matrices than CUs: panels of up to 256 rows run the 4-wave kernel.
    Three distinct blocks, each repeated 100 times, against the oracle."""
    _say(f"panel batch 300 r={r} p={p} kw={kw}")
    g = torch.Generator().manual_seed(r + 11 * p + kw)
    blk = torch.randn(3, r, 16 * p + kw, generator=g).numpy()
    starts, T_prev, refs = [], [], []
    for b in range(3):
        Hpre, _, Ts = _oracle_panels(oracle, blk[b][:, :16 * p], p) if p else (
            np.zeros((r, 0), np.float32), None, [])
        starts.append(np.concatenate([Hpre, blk[b][:, 16 * p:]], axis=1))
        T_prev.append(np.stack(Ts) if p else None)
        refs.append(_oracle_panels(oracle, blk[b], p + 1))
    reps = 100
    start = torch.from_numpy(np.repeat(np.stack(starts), reps, axis=0)).to(DEV)
    Tp = torch.from_numpy(np.repeat(np.stack(T_prev), reps, axis=0)).to(DEV) if p else None
    Hg, tau, T = hip_qr.panel(start, p=p, T_prev=Tp)
    torch.cuda.synchronize()
    Hg, tau, T = Hg.cpu().numpy(), tau.cpu().numpy(), T.cpu().numpy()
    tol = 4 * r * 2**-23
    up = np.triu(np.ones((r, kw), bool), k=-16 * p)
    for i in range(3 * reps):
        b = i // reps
        Href, taus, Trefs = refs[b]
        colnorm = np.linalg.norm(blk[b][:, 16 * p:].astype(np.float64), axis=0)
        dH = np.abs(Hg[i][:, 16 * p:].astype(np.float64) - Href[:, 16 * p:])
        assert (np.where(up, dH / colnorm, 0)).max() <= tol, ("R", i)
        assert (np.where(~up, dH, 0)).max() <= tol, ("V", i)
        assert np.abs(tau[i] - taus[p]).max() <= tol, ("tau", i)
        assert np.abs(T[i][:kw, :kw] - Trefs[p]).max() <= 4 * tol, ("T", i)
        if i % reps:  # identical inputs give identical bits
            assert np.array_equal(Hg[i], Hg[i - 1]) and np.array_equal(tau[i], tau[i - 1])


@pytest.mark.parametrize("m,k", [(16, 16), (64, 16), (300, 32), (1000, 64), (40, 7)])
def test_larft_vs_oracle(oracle, m, k):
    _say(f"larft m={m} k={k}")
    g = torch.Generator().manual_seed(m + k)
    P = torch.randn(2, m, k, generator=g)
    Vs, taus, Trefs = [], [], []
    for b in range(2):
        Hr, tr = oracle.geqr2(P[b].numpy())
        Vs.append(Hr)
        taus.append(tr)
        Trefs.append(oracle.larft(Hr, tr))
    V = torch.from_numpy(np.stack(Vs)).to(DEV)
    tau = torch.from_numpy(np.stack(taus)).to(DEV)
    T = hip_qr.larft(V, tau)
    torch.cuda.synchronize()
    T = T.cpu().numpy()
    for b in range(2):
        assert np.abs(T[b] - Trefs[b]).max() <= 16 * m * 2**-23


@pytest.mark.parametrize("r,nblk,c", [(16, 1, 1), (64, 1, 48), (100, 2, 77), (512, 4, 448),
                                      (1030, 3, 200), (2048, 4, 40), (300, 8, 33), (2500, 2, 20)])
def test_wy_update_vs_oracle(oracle, r, nblk, c):
    _say(f"wy_update r={r} nblk={nblk} c={c}")
    g = torch.Generator().manual_seed(r + 3 * c + nblk)
    blk = torch.randn(2, r, 16 * nblk + c, generator=g).numpy()
    starts, Ts, refs = [], [], []
    for b in range(2):
        Hp, _, Tb = _oracle_panels(oracle, blk[b][:, :16 * nblk], nblk)
        starts.append(np.concatenate([Hp, blk[b][:, 16 * nblk:]], axis=1))
        Ts.append(np.stack(Tb))
        refs.append(_oracle_panels(oracle, blk[b], nblk)[0][:, 16 * nblk:])
    out = hip_qr.wy_update(torch.from_numpy(np.stack(starts)).to(DEV),
                           torch.from_numpy(np.stack(Ts)).to(DEV))
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for b in range(2):
        assert np.array_equal(out[b, :, :16 * nblk], starts[b][:, :16 * nblk])  # V untouched
        scale = max(1.0, float(np.abs(blk[b]).max()))
        assert np.abs(out[b, :, 16 * nblk:] - refs[b]).max() <= 16 * r * 2**-23 * scale


@pytest.mark.parametrize("n", [65, 80, 96, 128, 129, 176, 200, 352, 512, 700, 1100])
def test_geqrf_blocked_vs_oracle(oracle, n):
    _say(f"geqrf blocked n={n}")
    A = _gauss(3, n, seed=n)
    H, tau = _run(A, midn=0)  # the blocked route also for n <= 192
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what=f"n={n}")
    res = checker.check(A, H, tau)
    assert res.passed, res.as_dict()


@pytest.mark.parametrize("n", [65, 97, 129, 150, 200, 257, 270, 333])
def test_geqrf_default_route_vs_oracle(oracle, n):
    """The default route at sizes whose last columns are a ragged fused tail:
    the whole matrix in the mid-n kernel (n <= 192), or outer blocks and then
    the last n - 64 k <= 192 columns in place (r = 136, 129, 142, 141: last
    strips of 8, 1, 14 and 13 columns)."""
    _say(f"geqrf default route n={n}")
    A = _gauss(2, n, seed=n + 29)
    H, tau = _run(A)
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what=f"default n={n}")
    res = checker.check(A, H, tau)
    assert res.passed, res.as_dict()


def test_geqrf_matches_mkl_golden_fixtures():
    from tests.test_oracle import _golden

    for name, (A, H_ref, tau_ref) in _golden().items():
        if name == "rank1_n16":
            continue
        _say(f"golden {name}")
        H, tau = _run(torch.from_numpy(A))
        assert_parity(A, H.numpy(), tau.numpy(), H_ref, tau_ref, what=name)


@pytest.mark.parametrize("n", [24, 100])
def test_geqrf_known_answers(n):
    _say(f"known answers n={n}")
    g = torch.Generator().manual_seed(n)
    U = torch.triu(torch.randn(2, n, n, generator=g))
    H, tau = _run(U)
    assert torch.equal(H, U) and torch.all(tau == 0)
    A = torch.randn(2, n, n, generator=g)
    A[:, :, n // 3] = 0.0
    H, tau = _run(A)
    assert torch.all(tau[:, n // 3] == 0) and torch.all(H[:, n // 3, n // 3] == 0)
    assert torch.all(tau[:, -1] == 0)


@pytest.mark.parametrize("shape", inputs.BENCHMARK_SHAPES,
                         ids=[f"b{s['batch']}_n{s['n']}" for s in inputs.BENCHMARK_SHAPES])
def test_official_shapes(oracle, shape):
    # The seven ranked GPUMODE shapes (reference inputs.py:20-28): FP64 gates on
    # the whole batch; elementwise parity with the oracle on two matrices where
    # the oracle takes seconds (n <= 352).
    _say(f"official shape b{shape['batch']} n{shape['n']}")
    prob = inputs.make_benchmark_problem(shape, seed=7, device="cpu")
    A = prob.tensor
    H, tau = _run(A)
    res = checker.check(A, H, tau)
    assert res.passed, res.as_dict()
    if shape["n"] <= 352:
        H_ref, tau_ref = oracle.geqrf(A[:2].numpy(), nb=16)
        assert_parity(A[:2].numpy(), H[:2].numpy(), tau[:2].numpy(), H_ref, tau_ref,
                      what=f"n={shape['n']}")


@pytest.mark.parametrize("n", [32, 176, 512])
def test_stress_suite_gates(n):
    for prob in inputs.stress_cases(n=n, batch=4, device="cpu"):
        _say(f"stress {prob.name}")
        H, tau = _run(prob.tensor)
        res = checker.check(prob.tensor, H, tau)
        assert res.passed, (prob.name, res.as_dict())


def test_config1_parity_and_gates(oracle):
    _say("config 1 (b64 n32)")
    A = inputs.config_tensor(inputs.config_spec(1))
    H, tau = _run(A)
    assert checker.check(A, H, tau).passed
    H_ref, tau_ref = oracle.geqrf(A.numpy())
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what="cfg1")
    Hm, tm = torch.geqrf(A)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), Hm.numpy(), tm.numpy(), what="vs MKL")


def test_config2_parity_and_gates(oracle):
    _say("config 2 (b2048 n64)")
    A = inputs.config_tensor(inputs.config_spec(2))
    H, tau = _run(A)
    assert checker.check(A, H, tau).passed
    H_ref, tau_ref = oracle.geqrf(A.numpy())
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what="cfg2 full batch")


def test_config4_gates_and_sampled_parity(oracle):
    _say("config 4 (b64 n1024)")
    A = inputs.config_tensor(inputs.config_spec(4))
    H, tau = _run(A)
    assert checker.check(A, H, tau).passed
    idx = [0, 21, 37, 63]
    H_ref, tau_ref = oracle.geqrf(A[idx].numpy(), nb=16)
    assert_parity(A[idx].numpy(), H[idx].numpy(), tau[idx].numpy(), H_ref, tau_ref,
                  what="cfg4 sampled")


def test_config5_gates_and_gaussian_half_parity(oracle):
    _say("config 5 (b16 n2048)")
    A = inputs.config_tensor(inputs.config_spec(5))
    H, tau = _run(A)
    assert torch.isfinite(H).all() and torch.isfinite(tau).all()
    res = checker.check(A, H, tau)
    assert res.passed, res.as_dict()
    n = A.shape[-1]
    assert torch.all(tau[8:, n // 3] == 0)  # zeroed column -> identity reflector
    idx = [8, 11, 15]
    H_ref, tau_ref = oracle.geqrf(A[idx].numpy(), nb=16)
    assert_parity(A[idx].numpy(), H[idx].numpy(), tau[idx].numpy(), H_ref, tau_ref,
                  what="cfg5 Gaussian half")


@pytest.mark.parametrize("route", [False, True], ids=["default", "route512"])
def test_config3_full_batch_gates_and_sampled_parity(oracle, route):
    """All 640 matrices as the benchmark runs them (more than 64 matrices: by
    default every block takes the 4-wave Householder panels and the b640
    trailing-update shapes), and with the CholeskyQR2 route on the first,
    512-row block (cholqr_min_rows=512). Gates on the whole batch, oracle
    parity on five matrices spread over it."""
    _say(f"config 3 (b640 n512), full batch, route={route}")
    A = inputs.config_tensor(inputs.config_spec(3))
    H, tau, codes = _run_ws(A, **({"cholqr_min_rows": 512} if route else {}))
    assert torch.isfinite(H).all() and torch.isfinite(tau).all()
    res = checker.check(A, H, tau)
    assert res.passed, res.as_dict()
    if route:
        assert bool((codes != 1).all())  # no matrix left the route in its block
    idx = [0, 157, 320, 481, 639]
    H_ref, tau_ref = oracle.geqrf(A[idx].numpy(), nb=16)
    assert_parity(A[idx].numpy(), H[idx].numpy(), tau[idx].numpy(), H_ref, tau_ref,
                  what="cfg3 sampled")


def test_input_not_modified_and_repeatable():
    _say("A unchanged, two calls bit-identical (n=300)")
    A = _gauss(4, 300, seed=9).to(DEV)
    A0 = A.clone()
    H1, t1 = hip_qr.geqrf(A)
    H2, t2 = hip_qr.geqrf(A)
    torch.cuda.synchronize()
    assert torch.equal(A, A0)
    assert torch.equal(H1, H2) and torch.equal(t1, t2)


@pytest.mark.parametrize("n,cols", [(100, (5, 37, 70)), (300, (20, 150, 290))])
@pytest.mark.parametrize("scale", [1e-30, 1e25, 1e-40], ids=["tiny", "huge", "denormal"])
def test_blocked_extreme_columns_vs_oracle(oracle, n, cols, scale):
    """Columns far outside the fast reflector's range (sigma under 2^-100, over
    2^100, or underflowing to zero) in the first panel and in later panels with
    left-looking updates: the panel's fast pass hands them to the general pass,
    whose slarfg scaling the oracle restates (oracle/qr_oracle.c)."""
    _say(f"extreme columns n={n} cols={cols} scale={scale:g}")
    A = _gauss(2, n, seed=n + 7)
    A[0, :, cols[0]] *= scale
    A[1, :, cols[1]] *= scale
    A[1, :, cols[2]] *= scale
    H, tau = _run(A, midn=0)
    assert torch.isfinite(H).all() and torch.isfinite(tau).all()
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what=f"n={n} x{scale:g}")


@pytest.mark.parametrize("scale", [1e-30, 1e25, 1e-40], ids=["tiny", "huge", "denormal"])
def test_default_route_extreme_columns_vs_oracle(oracle, scale):
    """The default route at n = 300, batch 2: CholeskyQR2 on the 300- and
    236-row outer blocks (column 20 fails its guard and goes back to the
    panels), then the last 172 columns in the fused mid-n kernel in place,
    where columns 150, 200 (zero) and 290 take its rare path: the panel is
    refactored from its saved copy with slarfg's scaled branches."""
    _say(f"default route extreme columns n=300 scale={scale:g}")
    A = _gauss(2, 300, seed=301)
    A[0, :, 20] *= scale
    A[0, :, 200] = 0.0
    A[1, :, 150] *= scale
    A[1, :, 290] *= scale
    H, tau = _run(A)
    Hf, tf = _run(A, midn=2)
    assert torch.equal(H, Hf) and torch.equal(tau, tf)  # the tail is the fused kernel's
    assert torch.isfinite(H).all() and torch.isfinite(tau).all()
    assert tau[0, 200] == 0
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref,
                  what=f"default n=300 x{scale:g}")


def test_side_stream_and_strided_input_bitwise():
    """The call runs on the caller's current stream (a non-default one here), and
    a transposed (column-major) input takes the same kernels after the strided
    copy: both give the contiguous, default-stream result bit for bit."""
    _say("side stream + transposed input (n=300)")
    A = _gauss(3, 300, seed=21).to(DEV)
    H0, t0 = hip_qr.geqrf(A)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        H1, t1 = hip_qr.geqrf(A)
    torch.cuda.current_stream().wait_stream(side)
    At = A.transpose(1, 2).contiguous().transpose(1, 2)  # same values, strides (n^2, 1, n)
    assert At.stride() == (300 * 300, 1, 300) and torch.equal(At, A)
    H2, t2 = hip_qr.geqrf(At)
    torch.cuda.synchronize()
    assert torch.equal(H0, H1) and torch.equal(t0, t1)
    assert torch.equal(H0, H2) and torch.equal(t0, t2)


def test_concurrent_host_threads_bitwise():
    """Two host threads, each on its own stream, factor different matrices at
    the same time. Both calls use the library's shared look-ahead stream
    (n > 128), and the b8 n700 calls take the CholeskyQR2 route for their first
    three outer blocks. Every result equals the one of a lone call, bit for bit."""
    import threading

    _say("two host threads, two streams, shared look-ahead stream")
    A1 = _gauss(3, 300, seed=5).to(DEV)
    A2 = _gauss(8, 700, seed=6).to(DEV)
    ref = {"a": hip_qr.geqrf(A1), "b": hip_qr.geqrf(A2)}
    torch.cuda.synchronize()
    results, errors = {}, []

    def work(key, A):
        try:
            st = torch.cuda.Stream()
            outs = []
            with torch.cuda.stream(st):
                for _ in range(6):
                    outs.append(hip_qr.geqrf(A))
            st.synchronize()
            results[key] = outs
        except Exception as exc:  # reported by the main thread
            errors.append(exc)

    threads = [threading.Thread(target=work, args=("a", A1)),
               threading.Thread(target=work, args=("b", A2))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    for key in ("a", "b"):
        H0, t0 = ref[key]
        assert len(results[key]) == 6
        for H, tau in results[key]:
            assert torch.equal(H, H0) and torch.equal(tau, t0)


@pytest.mark.parametrize("lookahead", ["1", "0"])
@pytest.mark.parametrize("n", [100, 700, 1100])
def test_first_block_reads_padded_input_directly(n, lookahead):
    """Input with a unit column stride but padded rows and batch (row stride
    n + 7, batch stride (n + 3) (n + 7)) is read in place by the first outer
    block's kernels; a column-major view of the same values goes through the
    strided copy first. Both give the same bits, with and without look-ahead."""
    opts = hip_qr.options(lookahead=int(lookahead), midn=0)
    _say(f"padded input read directly (n={n}, lookahead={lookahead})")
    batch = 2
    base = torch.randn(batch, n + 3, n + 7, generator=torch.Generator().manual_seed(n))
    Ap = base.to(DEV)[:, 1:n + 1, 2:n + 2]
    assert Ap.stride() == ((n + 3) * (n + 7), n + 7, 1)
    Ac = Ap.transpose(1, 2).contiguous().transpose(1, 2)
    assert Ac.stride(2) == n and torch.equal(Ac, Ap)
    Hp, tp = hip_qr.geqrf(Ap, options=opts)
    Hc, tc = hip_qr.geqrf(Ac, options=opts)
    torch.cuda.synchronize()
    assert torch.equal(Hp, Hc) and torch.equal(tp, tc)
    assert torch.equal(Ap, Ac)  # the input is left as it was


# (700, 64): the early blocks need more than one round of workgroups and split
# their update over two streams, the late ones fit in one round and run as one
# launch; (300, 3) and (1100, 2) fit in one round from early on.
@pytest.mark.parametrize("n,batch", [(300, 3), (1100, 2), (700, 64)])
def test_lookahead_schedule_is_bitwise_identical(n, batch):
    # The look-ahead schedule only splits the trailing update into disjoint
    # column ranges on two streams: results must not change by a single bit.
    _say(f"look-ahead on/off n={n}")
    A = _gauss(batch, n, seed=n + 1).to(DEV)
    H0, t0 = hip_qr.geqrf(A, options=hip_qr.options(lookahead=0))
    torch.cuda.synchronize()
    H1, t1 = hip_qr.geqrf(A, options=hip_qr.options(lookahead=1))
    torch.cuda.synchronize()
    assert torch.equal(H0, H1) and torch.equal(t0, t1)


@pytest.mark.parametrize("P", [1, 2, 3, 8])
def test_outer_block_widths(oracle, P):
    _say(f"outer block of {P} panels, n=400")
    A = _gauss(2, 400, seed=P)
    H, tau = _run(A, outer_panels=P)
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what=f"P={P}")


@pytest.mark.parametrize("n", [48, 200])
def test_tau_range_and_zero_columns(n):
    _say(f"tau range n={n}")
    g = torch.Generator().manual_seed(n)
    A = torch.randn(6, n, n, generator=g)
    A[2, :, n // 3] = 0.0
    H, tau = hip_qr.geqrf(A.to(DEV))
    tau = tau.cpu()
    nz = tau[tau != 0]
    assert bool(((nz >= 1 - 1e-6) & (nz <= 2 + 1e-6)).all())
    assert tau[2, n // 3] == 0 and bool((tau[:, -1] == 0).all())
    assert nz.numel() == tau.numel() - 7


EPS32 = 2.0**-23


@pytest.mark.parametrize("n,batch", [(16, 3), (40, 2), (64, 3), (100, 2), (200, 2), (513, 2)])
def test_orgqr_matches_householder_product(n, batch):
    # Q from (H, tau) is backward stable whatever A's conditioning: compare with
    # fp64 householder_product of the same factors, elementwise, and check
    # orthogonality and Q R = A.
    _say(f"orgqr n={n}")
    A = _gauss(batch, n, seed=3 * n + 1).to(DEV)
    H, tau = hip_qr.geqrf(A)
    Q = hip_qr.orgqr(H, tau)
    torch.cuda.synchronize()
    Q64 = torch.linalg.householder_product(H.double().cpu(), tau.double().cpu())
    err = (Q.double().cpu() - Q64).abs().max().item()
    assert err <= 4 * n * EPS32, err
    I = torch.eye(n, dtype=torch.float64)
    orth = (Q64.transpose(1, 2) @ Q.double().cpu() - I).abs().max().item()
    assert orth <= 100 * n * EPS32, orth
    R = torch.triu(H.double().cpu())
    resid = (Q.double().cpu() @ R - A.double().cpu()).abs().max().item()
    assert resid <= 20 * n * EPS32 * A.abs().max().item() * n ** 0.5, resid


@pytest.mark.parametrize("n,m,batch", [(64, 24, 2), (100, 37, 2), (200, 16, 1), (513, 70, 2)])
def test_ormqr_both_sides_and_round_trip(n, m, batch):
    _say(f"ormqr n={n} m={m}")
    A = _gauss(batch, n, seed=n + m).to(DEV)
    H, tau = hip_qr.geqrf(A)
    g = torch.Generator().manual_seed(m)
    C = torch.randn(batch, n, m, generator=g).to(DEV)
    QtC = hip_qr.ormqr(H, tau, C, transpose=True)
    QC = hip_qr.ormqr(H, tau, C, transpose=False)
    back = hip_qr.ormqr(H, tau, QtC, transpose=False)
    torch.cuda.synchronize()
    Q64 = torch.linalg.householder_product(H.double().cpu(), tau.double().cpu())
    C64 = C.double().cpu()
    scale = C64.abs().max().item() * n ** 0.5
    tol = 4 * n * EPS32 * scale
    assert (QtC.double().cpu() - Q64.transpose(1, 2) @ C64).abs().max().item() <= tol
    assert (QC.double().cpu() - Q64 @ C64).abs().max().item() <= tol
    assert (back.double().cpu() - C64).abs().max().item() <= 2 * tol
    # Q^T A is R: zero below the diagonal, triu(H) on and above it.
    QtA = hip_qr.ormqr(H, tau, A, transpose=True).double().cpu()
    R = torch.triu(H.double().cpu())
    assert (QtA - R).abs().max().item() <= 20 * n * EPS32 * A.abs().max().item() * n ** 0.5


def test_orgqr_on_smalln_and_official_b20_n32():
    _say("orgqr on fused small-n factors")
    prob = inputs.make_benchmark_problem(inputs.BENCHMARK_SHAPES[0], seed=11, device="cpu")
    A = prob.tensor.to(DEV)
    H, tau = hip_qr.geqrf(A)
    Q = hip_qr.orgqr(H, tau)
    Q64 = torch.linalg.householder_product(H.double().cpu(), tau.double().cpu())
    assert (Q.double().cpu() - Q64).abs().max().item() <= 4 * 32 * EPS32


def test_variant_registry_runs_hip_path():
    from gpumode_qr_amd.variants import CHAMPION, VARIANTS

    _say("registry champion call")
    A = _gauss(2, 70, seed=1).to(DEV)
    H, tau = VARIANTS[CHAMPION](A)
    torch.cuda.synchronize()
    assert checker.check(A, H, tau).passed


def test_run_baseline_db_record_schema(tmp_path):
    """The DB record keeps the reference's keys (dbwrite.py:61-93; each
    benchmark_results entry: shape, name, correctness, timing) and carries the new
    per-shape fields under extra."""
    import json

    from gpumode_qr_amd import run_baseline

    _say("run_baseline --configs 1 --cpu-baseline (DB record)")
    rc = run_baseline.main(["--configs", "1", "--warmup", "1", "--iters", "3", "--cpu-baseline",
                            "--db-dir", str(tmp_path)])
    assert rc == 0
    (path,) = list(tmp_path.glob("*_hh_mi355x.json"))
    rec = json.loads(path.read_text())
    assert list(rec) == ["impl", "git_commit", "date", "rocm_version", "docker_image",
                         "torch_version", "gpu_name", "hip_visible_devices",
                         "benchmark_results", "extra"]
    (res,) = rec["benchmark_results"]
    assert list(res) == ["shape", "name", "correctness", "timing"]
    assert res["correctness"]["passed"]
    extra = rec["extra"]
    for key in ("warmup", "iters", "all_benchmarks_pass", "stress_pass", "stress_results"):
        assert key in extra  # the reference's own extra keys
    (ps,) = extra["per_shape"]
    assert ps["name"] == res["name"]
    gflops = 4.0 / 3.0 * 32**3 * 64 / (res["timing"]["median_ms"] * 1e-3) / 1e9
    assert ps["gflops"] == pytest.approx(gflops, rel=1e-9)
    assert ps["pct_peak"] == pytest.approx(100.0 * gflops / 157_300.0, rel=1e-9)
    assert ps["cpu_geqrf_ms"] > 0 and extra["cpu_cores"] >= 1
    assert ps["counters"]["smalln"]["launches_per_call"] == 1.0
    assert set(ps["counters"]) == {"smalln"}  # n = 32 runs the one fused launch


# --------------------------------------------------------------------------
# Outer blocks by CholeskyQR2 + Householder reconstruction (qr_cholqr.hip).
# cholqr_min_rows=65 (with midn=0 for n <= 192) sends every full 64-column
# block through the route (by
# default blocks of >= 128 rows in calls of <= 64 matrices, >= 576 above);
# cholqr=0 switches it off. Route codes of the last route block: 0 two
# passes, 1 Householder panels (guard failed), 2 one pass.

EVERY_BLOCK = {"cholqr_min_rows": 65, "midn": 0}


@pytest.mark.parametrize("n", [128, 129, 200, 256, 300, 513, 1100])
def test_cholqr_route_vs_oracle(oracle, n):
    _say(f"cholqr route (every full block) n={n}")
    A = _gauss(3, n, seed=n + 11)
    H, tau = _run(A, **EVERY_BLOCK)
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what=f"cholqr n={n}")
    res = checker.check(A, H, tau)
    assert res.passed, res.as_dict()


def test_cholqr_route_cond1e2_svd(oracle):
    """Haar-SVD input of cond 1e2 with every block on the route. (Its first
    64 columns are well conditioned: 64 random combinations of 512 singular
    directions. The two-pass path is pinned by the near-bound and forced
    two-pass tests.)"""
    _say("cholqr route, cond-1e2 SVD input b2 n512")
    A = inputs.svd_matrices(2, 512, 2.0, torch.Generator().manual_seed(5)).float()
    H, tau = _run(A, **EVERY_BLOCK)
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what="cholqr svd")
    res = checker.check(A, H, tau)
    assert res.passed, res.as_dict()


@pytest.mark.parametrize("shape", [(60, 1024), (8, 2048), (2, 4096)],
                         ids=["b60_n1024", "b8_n2048", "b2_n4096"])
def test_cholqr_default_route_official_shapes_vs_oracle(oracle, shape):
    """The shapes where the route factors most of V, tau and R by default
    (every block of >= 128 rows): the official inputs (columns scaled by
    logspace(0, -cond, n)), gates on the batch and oracle parity on one
    matrix. The route codes show the last route block's path."""
    batch, n = shape
    spec = next(s for s in inputs.BENCHMARK_SHAPES if (s["batch"], s["n"]) == shape)
    _say(f"cholqr default route, official shape b{batch} n{n}")
    A = inputs.make_benchmark_problem(spec, seed=7, device="cpu").tensor
    H, tau, codes = _run_ws(A)
    res = checker.check(A, H, tau)
    assert res.passed, res.as_dict()
    assert bool((codes != 1).all()), codes
    H_ref, tau_ref = oracle.geqrf(A[:1].numpy(), nb=16)
    assert_parity(A[:1].numpy(), H[:1].numpy(), tau[:1].numpy(), H_ref, tau_ref,
                  what=f"b{batch} n{n} matrix 0")


@pytest.mark.parametrize("inv_sum,code", [(140.0, 2), (152.0, 0)], ids=["one_pass", "two_pass"])
def test_cholqr_one_pass_bound_vs_oracle(oracle, inv_sum, code):
    """First block of n = 160 (the only route block of the call) at the
    one-pass bound: sum(sigma^-2) of the scaled Gram just under 144 takes one
    pass at kappa about 33, just over it takes two. Both match the oracle at
    the flat tolerance."""
    n = 160
    _say(f"cholqr one-pass bound n={n} sum(1/sigma^2)={inv_sum}")
    g = torch.Generator().manual_seed(41)
    A = torch.randn(2, n, n, generator=g)
    for b in range(2):
        blk, kappa = near_bound_block(n, inv_sum, seed=b)
        A[b, :, :64] = torch.from_numpy(blk)
    H, tau, codes = _run_ws(A, midn=0)
    print(f"[gpu-case] near-bound kappa(R1s) about {kappa:.1f}, codes {codes.tolist()}",
          flush=True)
    assert codes.tolist() == [code, code], codes
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref,
                  what=f"one-pass bound code {code}")


def test_cholqr_one_pass_only_sends_two_pass_blocks_to_the_panels(oracle):
    """cholqr_one_pass = 2: the block just over the one-pass bound, which the
    default would take in two passes, is factored by the Householder panels
    instead (route code 1, no pass-2 launch); a Gaussian block still takes
    one pass. Both match the oracle at the flat tolerance."""
    n = 160
    _say("cholqr one pass only, n=160")
    g = torch.Generator().manual_seed(43)
    A = torch.randn(2, n, n, generator=g)
    blk, _ = near_bound_block(n, 152.0, seed=0)
    A[0, :, :64] = torch.from_numpy(blk)
    H, tau, codes = _run_ws(A, cholqr_one_pass=2, midn=0)
    assert codes.tolist() == [1, 2], codes
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what="one pass only")


@pytest.mark.parametrize("n", [300, 2048])
def test_cholqr_forced_two_passes_vs_oracle(oracle, n):
    """The first block of a Gaussian matrix (the only route block with
    cholqr_min_rows = n) takes one pass by default; cholqr_one_pass=0 forces
    the second pass for the same input."""
    _say(f"cholqr forced two passes n={n}")
    A = _gauss(2, n, seed=n + 21)
    H1, t1, c1 = _run_ws(A, cholqr_min_rows=n)
    H2, t2, c2 = _run_ws(A, cholqr_one_pass=0, cholqr_min_rows=n)
    assert c1.tolist() == [2, 2] and c2.tolist() == [0, 0], (c1, c2)
    assert not torch.equal(H1, H2)  # the two paths round differently
    idx = [0] if n > 1024 else [0, 1]
    H_ref, tau_ref = oracle.geqrf(A[idx].numpy(), nb=16)
    for H, tau, what in ((H1, t1, "one pass"), (H2, t2, "two passes")):
        assert_parity(A[idx].numpy(), H[idx].numpy(), tau[idx].numpy(), H_ref, tau_ref,
                      what=f"n={n} {what}")


# A block whose Gram is singular, out of range, or too ill-conditioned for
# CholeskyQR2 falls back to the Householder panels for that matrix only; the
# other matrices of the batch keep the route in the same block.
@pytest.mark.parametrize("n,cols", [(300, (20, 150, 290)), (700, (5, 400, 650))])
@pytest.mark.parametrize("kind", ["zero", "tiny", "huge", "denormal", "near_dup"])
def test_cholqr_fallback_vs_oracle(oracle, n, cols, kind):
    _say(f"cholqr fallback {kind} n={n} cols={cols}")
    A = _gauss(3, n, seed=n + 3)
    for b, c in ((0, cols[0]), (1, cols[1]), (1, cols[2])):
        if kind == "zero":
            A[b, :, c] = 0.0
        elif kind == "near_dup":  # columns c and c+1 agree to 1e-6: scaled pivot ~1e-12
            A[b, :, c + 1 if c + 1 < n else c - 1] = A[b, :, c] * (1 + 1e-6)
        else:
            A[b, :, c] *= {"tiny": 1e-30, "huge": 1e25, "denormal": 1e-40}[kind]
    H, tau = _run(A, **EVERY_BLOCK)
    assert torch.isfinite(H).all() and torch.isfinite(tau).all()
    if kind != "near_dup":  # near-duplicate columns: kappa ~1e7, gates only
        H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
        assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref,
                      what=f"cholqr fallback {kind}")
    if kind in ("zero", "near_dup"):
        res = checker.check(A, H, tau)
        assert res.passed, res.as_dict()


@pytest.mark.parametrize("kind", ["zero", "tiny", "denormal"])
def test_cholqr_fallback_route_codes(kind):
    """n = 160 with only the first block on the route: a zero, tiny (1e-30
    outside the Gram's [1e-30, 1e30] diagonal range once squared) or
    subnormal column in it sends that matrix, and only it, to the panels."""
    n = 160
    _say(f"cholqr fallback route code {kind} n={n}")
    A = _gauss(3, n, seed=77)
    A[1, :, 30] = 0.0 if kind == "zero" else A[1, :, 30] * (1e-30 if kind == "tiny" else 1e-40)
    _, _, codes = _run_ws(A, midn=0)
    assert codes.tolist() == [2, 1, 2], codes


@pytest.mark.parametrize("n,batch", [(300, 3), (1100, 2), (700, 64)])
def test_cholqr_lookahead_and_repeat_bitwise(n, batch):
    _say(f"cholqr route look-ahead on/off and repeat n={n} b={batch}")
    A = _gauss(batch, n, seed=n + 5).to(DEV)
    off = hip_qr.options(lookahead=0, **EVERY_BLOCK)
    on = hip_qr.options(lookahead=1, **EVERY_BLOCK)
    H0, t0 = hip_qr.geqrf(A, options=off)
    torch.cuda.synchronize()
    H1, t1 = hip_qr.geqrf(A, options=on)
    H2, t2 = hip_qr.geqrf(A, options=on)
    torch.cuda.synchronize()
    assert torch.equal(H0, H1) and torch.equal(t0, t1)
    assert torch.equal(H1, H2) and torch.equal(t1, t2)


def test_cholqr_off_matches_on_within_tolerance(oracle):
    _say("cholqr on vs off, b4 n600")
    A = _gauss(4, 600, seed=77)
    Hh, th = _run(A, cholqr=0)
    Hc, tc = _run(A, **EVERY_BLOCK)
    assert not torch.equal(Hh, Hc)  # the two routes round differently
    assert_parity(A.numpy(), Hc.numpy(), tc.numpy(), Hh.numpy().astype(np.float64),
                  th.numpy().astype(np.float64), what="cholqr vs householder")
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), Hh.numpy(), th.numpy(), H_ref, tau_ref, what="householder only")


@pytest.mark.parametrize("kind", ["upper", "block_diag"])
def test_cholqr_exact_zero_structure(oracle, kind):
    """Exact zeros below a diagonal give slarfg's tau = 0: upper-triangular input
    stays a fixed point (H == A, tau == 0) and a block-diagonal matrix matches
    the oracle, because such blocks leave the CholeskyQR2 route."""
    _say(f"cholqr route, exact-zero structure {kind} n=300")
    A = _gauss(2, 300, seed=9)
    if kind == "upper":
        A = torch.triu(A)
        A.diagonal(dim1=1, dim2=2).abs_().add_(1.0)
    else:
        mask = torch.zeros(300, 300, dtype=torch.bool)
        for s0 in range(0, 300, 100):
            mask[s0:s0 + 100, s0:s0 + 100] = True
        A = torch.where(mask, A, torch.zeros(()))
    H, tau = _run(A, **EVERY_BLOCK)
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    assert_parity(A.numpy(), H.numpy(), tau.numpy(), H_ref, tau_ref, what=f"cholqr {kind}")
    if kind == "upper":
        assert torch.equal(tau, torch.zeros_like(tau))
        assert torch.equal(H, A)


@pytest.mark.parametrize("n,batch", [(300, 3), (700, 5)])
def test_cholqr_fused_variant(oracle, n, batch):
    """The fused Gram + per-matrix kernels (cholqr_fused=1: the last
    workgroup of a matrix to finish runs its per-matrix step, whichever it is)
    match the oracle, and each variant is bit-identical with look-ahead on and
    off. The two variants split the Gram rows over different wave counts, so
    they round differently from each other."""
    _say(f"cholqr fused and separate kernels n={n} b={batch}")
    A = _gauss(batch, n, seed=n + 9)
    A[1, :, 100] = 0.0  # one matrix takes the fallback panels in one block
    Ad = A.to(DEV)
    out = {}
    for fused in (0, 1):
        for la in (0, 1):
            opts = hip_qr.options(cholqr_fused=fused, lookahead=la, **EVERY_BLOCK)
            out[fused, la] = hip_qr.geqrf(Ad, options=opts)
    torch.cuda.synchronize()
    for fused in (0, 1):
        (H0, t0), (H1, t1) = out[fused, 0], out[fused, 1]
        assert torch.equal(H0, H1) and torch.equal(t0, t1), fused
    H_ref, tau_ref = oracle.geqrf(A.numpy(), nb=16)
    for fused in (0, 1):
        H, tau = out[fused, 1]
        assert_parity(A.numpy(), H.cpu().numpy(), tau.cpu().numpy(), H_ref, tau_ref,
                      what=f"fused={fused} n={n}")


def test_options_out_of_range_are_rejected():
    _say("route options validation")
    A = _gauss(1, 100, seed=1).to(DEV)
    for bad in ({"cholqr": 2}, {"cholqr_min_rows": 64}, {"outer_panels": 9},
                {"lookahead": -1}, {"cholqr_one_pass": 3}):
        with pytest.raises(Exception) as ei:
            hip_qr.geqrf(A, options=hip_qr.options(**bad))
        assert getattr(ei.value, "status", None) == 1, bad
