"""Correctness + benchmark runner for a QR implementation; writes one DB record.

Counterpart of the reference's scripts/run_baseline.py (flags, flow and exit
codes follow :66-252):

    python -m gpumode_qr_amd.run_baseline --impl hh_mi355x [--stress] [--iters 10]
    python -m gpumode_qr_amd.run_baseline --list
    python -m gpumode_qr_amd.run_baseline --compare [--impls a,b] [--shapes 512,1024]
    python -m gpumode_qr_amd.run_baseline --impl hh_mi355x --configs 2,3,4,5

Exit codes: 0 all gates pass, 1 no torch / no GPU, 2 a gate failed.
``--configs`` selects the five headline configs instead of the official shapes.
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

from .variants import CHAMPION, VARIANTS as _VARIANTS, format_variant_list

REPO_ROOT = Path(__file__).resolve().parents[1]
BASELINE = "torch_geqrf"
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


def run_benchmarks(fn, device: str, warmup: int, iters: int, shapes: list[dict] | None = None,
                   configs: list[int] | None = None) -> list[dict]:
    results = []
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
            "gflops": gflops,
        })
        status = "PASS" if chk.passed else "FAIL"
        print(f"[bench] {prob.name:>28} {status} median={timing.median:.3f}ms "
              f"min={timing.min:.3f}ms {gflops:.0f} GFLOP/s "
              f"factor={chk.factor_residual:.2e} orth={chk.orth_residual:.2e}")
    gm = bench.geomean([r["timing"]["median_ms"] for r in results])
    print(f"[bench] geomean(median) across {len(results)} problems = {gm:.4f} ms")
    return results


def run_compare(impls: list[str], device: str, warmup: int, iters: int, shapes, configs) -> int:
    print(f"device={torch.cuda.get_device_name(0)} torch={torch.__version__} hip={torch.version.hip}")
    summary = []
    for impl in impls:
        print(f"=== {impl}{'  (champion)' if impl == CHAMPION else ''} ===")
        res = run_benchmarks(REGISTRY[impl], device, warmup, iters, shapes, configs)
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
    results = run_benchmarks(fn, args.device, args.warmup, args.iters, shapes, configs)
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
        })
        print(f"wrote {path}")
    return 0 if all_pass and (stress_pass is not False) else 2


if __name__ == "__main__":
    raise SystemExit(main())
