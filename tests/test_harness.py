"""Host-side harness: inputs, checker, registry, CLI paths that need no GPU."""

from __future__ import annotations

import math

import pytest
import torch

from gpumode_qr_amd import EPS32, bench, checker, inputs, variants
from gpumode_qr_amd import run_baseline


def test_eps32():
    assert EPS32 == 2.0**-23


def test_benchmark_shapes_are_the_official_seven():
    assert [(s["batch"], s["n"], s["cond"]) for s in inputs.BENCHMARK_SHAPES] == [
        (20, 32, 1), (40, 176, 1), (40, 352, 1), (640, 512, 2), (60, 1024, 2), (8, 2048, 1),
        (2, 4096, 1),
    ]


def test_config_specs():
    assert [(c["batch"], c["n"]) for c in inputs.CONFIGS] == [
        (64, 32), (2048, 64), (640, 512), (64, 1024), (16, 2048),
    ]


def test_config1_is_manual_seed_0_randn():
    A = inputs.config_tensor(inputs.config_spec(1))
    torch.manual_seed(0)
    assert torch.equal(A, torch.randn(64, 32, 32))


def test_inputs_are_deterministic_and_cpu_generated():
    a = inputs.make_benchmark_problem({"batch": 2, "n": 16, "cond": 2}, seed=3, device="cpu")
    b = inputs.make_benchmark_problem({"batch": 2, "n": 16, "cond": 2}, seed=3, device="cpu")
    assert torch.equal(a.tensor, b.tensor)
    # columns scaled by logspace(0, -cond, n)
    col = a.tensor.abs().mean(dim=(0, 1))
    assert col[0] > 10 * col[-1]


def test_svd_matrices_have_the_requested_spectrum():
    g = torch.Generator().manual_seed(0)
    A = inputs.svd_matrices(2, 48, 2.0, g)
    s = torch.linalg.svdvals(A.double())
    ref = torch.logspace(0, -2, 48, dtype=torch.float64)
    assert torch.allclose(s, ref.expand_as(s), rtol=1e-5, atol=1e-7)


def test_stress5_structure_small():
    spec = dict(inputs.config_spec(5), batch=4, n=48, name="cfg5_small")
    A = inputs.config_tensor(spec)
    n = 48
    assert torch.all(A[2:, :, n // 3] == 0)
    assert A[2:, :, (2 * n) // 3].abs().mean() > 1e3
    s = torch.linalg.svdvals(A[:2].double())
    assert float(s.max() / s.min()) == pytest.approx(1e6, rel=1e-2)


def test_stress_cases_cover_the_nine_structures():
    probs = inputs.stress_cases(n=16, batch=2, device="cpu")
    assert [p.meta["kind"] for p in probs] == [
        "dense", "dense", "rank_deficient", "near_rank_deficient", "banded", "row_scaled",
        "near_collinear", "upper_triangular", "clustered_scale",
    ]
    assert all(p.tensor.shape == (2, 16, 16) for p in probs)


def test_config1_end_to_end_on_cpu_with_torch_geqrf():
    A = inputs.config_tensor(inputs.config_spec(1))
    H, tau = torch.geqrf(A)
    res = checker.check(A, H, tau)
    assert res.passed
    assert res.factor_threshold == pytest.approx(20 * 32 * EPS32)
    assert res.orth_threshold == pytest.approx(100 * 32 * EPS32)
    assert res.factor_residual < res.factor_threshold / 10


def test_checker_chunks_consistently(monkeypatch):
    g = torch.Generator().manual_seed(1)
    A = torch.randn(6, 12, 12, generator=g)
    H, tau = torch.geqrf(A)
    full = checker.check(A, H, tau)
    monkeypatch.setattr(checker, "_chunk", lambda b, n: 2)
    chunked = checker.check(A, H, tau)
    assert chunked.factor_residual == pytest.approx(full.factor_residual)
    assert chunked.orth_residual == pytest.approx(full.orth_residual)


def test_geomean():
    assert bench.geomean([1.0, 4.0]) == pytest.approx(2.0)
    assert math.isnan(bench.geomean([]))
    with pytest.raises(ValueError):
        bench.geomean([1.0, 0.0])
    assert bench.qr_flops(2, 3) == pytest.approx(2 * 4 / 3 * 27)


def test_registry_and_list():
    assert variants.CHAMPION in variants.VARIANTS
    rows = variants.describe_variants()
    assert rows[0][0] == variants.CHAMPION and rows[0][2]
    assert rows[-1][1].status == "baseline"
    text = variants.format_variant_list()
    assert "★ hh_mi355x" in text


def test_cli_list_and_no_gpu_exit_codes(capsys):
    assert run_baseline.main(["--list"]) == 0
    assert "Champion: hh_mi355x" in capsys.readouterr().out
    if not torch.cuda.is_available():
        assert run_baseline.main(["--no-write", "--shapes", "32"]) == 1


def test_hip_path_refuses_cpu_tensors():
    from gpumode_qr_amd import hip_qr

    with pytest.raises(ValueError):
        hip_qr.geqrf(torch.zeros(2, 8, 8))
    with pytest.raises(TypeError):
        hip_qr.geqrf(torch.zeros(2, 8, 8, dtype=torch.float64))


@pytest.mark.parametrize("chunk", [None, 1, 2])
@pytest.mark.parametrize("kind", ["nan_in_v", "all_nan", "inf_in_tau", "nan_in_r"])
def test_checker_fails_on_nan_and_inf(monkeypatch, chunk, kind):
    # A factorisation holding NaN or Inf must fail the gates, whichever chunk
    # of the batch it sits in (Python's max(0.0, nan) is 0.0).
    g = torch.Generator().manual_seed(2)
    A = torch.randn(5, 10, 10, generator=g)
    H, tau = torch.geqrf(A)
    if chunk is not None:
        monkeypatch.setattr(checker, "_chunk", lambda b, n: chunk)
    assert checker.check(A, H, tau).passed
    H, tau = H.clone(), tau.clone()
    if kind == "nan_in_v":
        H[3, 7, 2] = float("nan")
    elif kind == "all_nan":
        H.fill_(float("nan"))
        tau.fill_(float("nan"))
    elif kind == "inf_in_tau":
        tau[1, 4] = float("inf")
    else:
        H[0, 1, 5] = float("nan")
    res = checker.check(A, H, tau)
    assert not res.passed, res.as_dict()
    assert not res.factor_pass or not res.orth_pass
