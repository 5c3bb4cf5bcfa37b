"""Correctness + benchmark runner for a QR implementation; writes one DB record.

Counterpart of the reference's scripts/run_baseline.py (flags, flow and exit
codes follow :66-252):

    python -m gpumode_qr_amd.run_baseline --impl hh_mi355x [--stress] [--iters 10]
    python -m gpumode_qr_amd.run_baseline --list
    python -m gpumode_qr_amd.run_baseline --compare [--impls a,b] [--shapes 512,1024]
    python -m gpumode_qr_amd.run_baseline --impl hh_mi355x --configs 2,3,4,5

Exit codes: 0 all gates pass, 1 no torch / no GPU, 2 a gate failed.
``--configs`` selects the five headline configs instead of the official shapes.

The record keeps the reference's schema (dbwrite.py:61-93): each
``benchmark_results`` entry holds exactly ``shape``, ``name``, ``correctness`` and
``timing``. The fields the reference does not have go under ``extra``:
``per_shape`` (GFLOP/s, % of the MI355X FP32 matrix peak, the CPU ``torch.geqrf``
time with ``--cpu-baseline``, and this library's per-kernel launch counters),
``cpu_cores`` and ``fp32_peak_gflops``.
"""

from __future__ import annotations

import argparse
import os
import statistics
import sys
import time
from pathlib import Path

from .variants import CHAMPION, VARIANTS as _VARIANTS, format_variant_list

REPO_ROOT = Path(__file__).resolve().parents[1]
BASELINE = "torch_geqrf"
# MI355X dense FP32 matrix (MFMA) peak, GFLOP/s.
FP32_PEAK_GFLOPS = 157_300.0
# Calls traced per shape for the per-kernel counters.
COUNTER_CALLS = 3
ALL_IMPLS = sorted(set(_VARIANTS) | {BASELINE})

try:  # torch is needed only for the benchmarking paths, not for --list
    import torch

    from . import bench, checker, dbwrite, inputs
    from .reference import REGISTRY as _REF_REGISTRY

    REGISTRY = {**_REF_REGISTRY, **_VARIANTS}
    _HAVE_TORCH = True
except ModuleNotFoundError:  # pragma: no cover
    _HAVE_TORCH = False
    REGISTRY = {}


def select_shapes(spec: str | None) -> list[dict]:
    """Shapes by comma-separated name (``b640_n512_cond2``) or ``n`` value."""
    if not spec:
        return list(inputs.BENCHMARK_SHAPES)
    tokens = {t.strip() for t in spec.split(",") if t.strip()}
    picked = [
        s for s in inputs.BENCHMARK_SHAPES
        if f"b{s['batch']}_n{s['n']}_cond{s['cond']}" in tokens or str(s["n"]) in tokens
    ]
    if not picked:
        raise SystemExit(f"no benchmark shapes matched --shapes={spec!r}")
    return picked


def _problems(shapes: list[dict] | None, configs: list[int] | None, device: str):
    if configs:
        for c in configs:
            yield inputs.make_config_problem(c, device=device)
    else:
        for shape in shapes if shapes is not None else inputs.BENCHMARK_SHAPES:
            yield inputs.make_benchmark_problem(shape, device=device)


def run_correctness_stress(fn, device: str) -> list[dict]:
    results = []
    for n in (32, 176, 512):
        for prob in inputs.stress_cases(n=n, batch=4, device=device):
            H, tau = fn(prob.tensor)
            torch.cuda.synchronize()
            res = checker.check(prob.tensor, H, tau)
            results.append({"case": prob.name, **prob.meta, **res.as_dict()})
            status = "PASS" if res.passed else "FAIL"
            print(f"[stress] {prob.name:>28} {status} "
                  f"factor={res.factor_residual:.2e}/{res.factor_threshold:.2e} "
                  f"orth={res.orth_residual:.2e}/{res.orth_threshold:.2e}")
    return results


def cpu_cores() -> int:
    """Cores torch's CPU geqrf may use: all the cores this process may run on."""
    return len(os.sched_getaffinity(0))


def cpu_geqrf_ms(A: torch.Tensor, reps: int = 3) -> float:
    """Median wall time of torch.geqrf (MKL) on a CPU copy of A, all cores."""
    torch.set_num_threads(cpu_cores())
    Ac = A.detach().to("cpu")
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        torch.geqrf(Ac)
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


def kernel_counters(fn, A: torch.Tensor, calls: int = COUNTER_CALLS) -> dict:
    """Per-kernel launches, time and algorithmic rates per call of fn(A), from the
    library's launch tracer (HIP events around each launch of its kernels)."""
    from . import _lib

    names = list(_lib.KERNELS)
    _lib.trace_reset()
    _lib.trace_enable(names)
    try:
        for _ in range(calls):
            fn(A)
        torch.cuda.synchronize()
    finally:
        _lib.trace_enable(None)
    out = {}
    for nm in names:
        d = _lib.trace_read(nm)
        if not d["launches"]:
            continue
        sec = d["ms"] * 1e-3
        out[nm] = {
            "launches_per_call": d["launches"] / calls,
            "ms_per_call": d["ms"] / calls,
            "tflops": d["flops"] / sec / 1e12 if sec > 0 else 0.0,
            "gbs": d["bytes"] / sec / 1e9 if sec > 0 else 0.0,
        }
    _lib.trace_reset()
    return out


def run_benchmarks(fn, device: str, warmup: int, iters: int, shapes: list[dict] | None = None,
                   configs: list[int] | None = None, cpu_baseline: bool = False,
                   counters: bool = False) -> tuple[list[dict], list[dict]]:
    """Returns (benchmark_results in the reference's schema, per-shape extras)."""
    results, extras = [], []
    for prob in _problems(shapes, configs, device):
        H, tau = fn(prob.tensor)
        torch.cuda.synchronize()
        chk = checker.check(prob.tensor, H, tau)
        del H, tau
        timing = bench.benchmark(fn, prob.tensor, warmup=warmup, iters=iters)
        gflops = bench.qr_flops(prob.batch, prob.n) / (timing.median * 1e-3) / 1e9
        shape = {k: prob.meta[k] for k in ("batch", "n", "cond") if k in prob.meta}
        results.append({
            "shape": shape or {"batch": prob.batch, "n": prob.n},
            "name": prob.name,
            "correctness": chk.as_dict(),
            "timing": timing.as_dict(),
        })
        ext = {"name": prob.name, "gflops": gflops, "pct_peak": 100.0 * gflops / FP32_PEAK_GFLOPS}
        if cpu_baseline:
            ext["cpu_geqrf_ms"] = cpu_geqrf_ms(prob.tensor)
        if counters:
            ext["counters"] = kernel_counters(fn, prob.tensor)
        extras.append(ext)
        status = "PASS" if chk.passed else "FAIL"
        cpu = f" cpu={ext['cpu_geqrf_ms']:.1f}ms" if cpu_baseline else ""
        print(f"[bench] {prob.name:>28} {status} median={timing.median:.3f}ms "
              f"min={timing.min:.3f}ms {gflops:.0f} GFLOP/s ({ext['pct_peak']:.1f}% peak)"
              f"{cpu} factor={chk.factor_residual:.2e} orth={chk.orth_residual:.2e}")
    gm = bench.geomean([r["timing"]["median_ms"] for r in results])
    print(f"[bench] geomean(median) across {len(results)} problems = {gm:.4f} ms")
    return results, extras


def run_compare(impls: list[str], device: str, warmup: int, iters: int, shapes, configs) -> int:
    print(f"device={torch.cuda.get_device_name(0)} torch={torch.__version__} hip={torch.version.hip}")
    summary = []
    for impl in impls:
        print(f"=== {impl}{'  (champion)' if impl == CHAMPION else ''} ===")
        res, _ = run_benchmarks(REGISTRY[impl], device, warmup, iters, shapes, configs)
        gm = bench.geomean([r["timing"]["median_ms"] for r in res])
        summary.append((impl, gm, all(r["correctness"]["passed"] for r in res)))
        print()
    summary.sort(key=lambda t: t[1])
    best = summary[0][1] if summary else float("nan")
    print("Compare ranking (geomean of per-problem median_ms; lower is better):")
    for rank, (impl, gm, ok) in enumerate(summary, 1):
        champ = " ★" if impl == CHAMPION else ""
        print(f"  {rank:>2} {impl + champ:<32} {gm:>12.4f} ms {gm / best:>7.2f}x  "
              f"{'PASS' if ok else 'FAIL'}")
    return 0 if all(ok for _, _, ok in summary) else 2


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--impl", default=CHAMPION, choices=ALL_IMPLS)
    ap.add_argument("--device", default="cuda")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--stress", action="store_true", help="run the correctness stress suite")
    ap.add_argument("--docker-image", default=None)
    ap.add_argument("--db-dir", default=str(REPO_ROOT / "db"))
    ap.add_argument("--no-write", action="store_true")
    ap.add_argument("--list", action="store_true", help="list registered variants; no GPU")
    ap.add_argument("--compare", action="store_true", help="rank several variants; no DB write")
    ap.add_argument("--impls", default=None, help="comma-separated impls for --compare")
    ap.add_argument("--shapes", default=None, help="official shapes by name or n (default: all 7)")
    ap.add_argument("--configs", default=None, help="headline configs, e.g. 2,3,4,5")
    ap.add_argument("--cpu-baseline", action="store_true",
                    help="also time torch.geqrf on CPU copies of each input (extra.per_shape)")
    args = ap.parse_args(argv)

    if args.list:
        print(format_variant_list())
        return 0
    if not _HAVE_TORCH:
        print("ERROR: torch is not importable", file=sys.stderr)
        return 1
    if not torch.cuda.is_available():
        print("ERROR: no GPU visible to torch", file=sys.stderr)
        return 1

    configs = [int(c) for c in args.configs.split(",")] if args.configs else None
    shapes = None if configs else select_shapes(args.shapes)
    if args.compare:
        impls = ([t.strip() for t in args.impls.split(",") if t.strip()]
                 if args.impls else [CHAMPION, BASELINE])
        unknown = [i for i in impls if i not in REGISTRY]
        if unknown:
            raise SystemExit(f"unknown impls for --compare: {unknown}")
        return run_compare(impls, args.device, args.warmup, args.iters, shapes, configs)

    fn = REGISTRY[args.impl]
    print(f"impl={args.impl} device={torch.cuda.get_device_name(0)} "
          f"torch={torch.__version__} hip={torch.version.hip}")
    stress = run_correctness_stress(fn, args.device) if args.stress else []
    results, per_shape = run_benchmarks(fn, args.device, args.warmup, args.iters, shapes,
                                        configs, cpu_baseline=args.cpu_baseline,
                                        counters=args.impl in _VARIANTS)
    all_pass = all(r["correctness"]["passed"] for r in results)
    stress_pass = all(r["passed"] for r in stress) if stress else None
    gm_med = bench.geomean([r["timing"]["median_ms"] for r in results])
    gm_min = bench.geomean([r["timing"]["min_ms"] for r in results])
    if not args.no_write:
        meta = dbwrite.collect_metadata(str(REPO_ROOT), args.docker_image)
        path = dbwrite.write_result(args.db_dir, args.impl, meta, results, extra={
            "warmup": args.warmup,
            "iters": args.iters,
            "all_benchmarks_pass": all_pass,
            "stress_pass": stress_pass,
            "stress_results": stress,
            "geomean_median_ms": gm_med,
            "geomean_min_ms": gm_min,
            "per_shape": per_shape,
            "cpu_cores": cpu_cores() if args.cpu_baseline else None,
            "fp32_peak_gflops": FP32_PEAK_GFLOPS,
        })
        print(f"wrote {path}")
    return 0 if all_pass and (stress_pass is not False) else 2


if __name__ == "__main__":
    raise SystemExit(main())
