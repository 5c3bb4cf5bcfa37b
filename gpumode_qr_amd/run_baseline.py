"""Check, time and record a registered QR variant from the command line.

    python -m gpumode_qr_amd.run_baseline --impl hh_mi355x [--stress] [--iters 10]
    python -m gpumode_qr_amd.run_baseline --list
    python -m gpumode_qr_amd.run_baseline --compare [--impls a,b] [--shapes 512,1024]
    python -m gpumode_qr_amd.run_baseline --impl hh_mi355x --configs 2,3,4,5 --cpu-baseline

The command line and the exit codes are those of the reference's
scripts/run_baseline.py (flags at :157-183; exit codes at :190-197, :152,
:252), so its users call this one the same way: 0 when every gate passes,
1 without torch or a GPU, 2 when a gate fails. Added here: ``--configs``
(the five headline workloads in place of the seven official shapes) and
``--cpu-baseline`` (torch.geqrf on the host's cores, same inputs).

Each benchmarked problem is gated (FP64 checker) on the very input it is
timed on. Unless ``--no-write``, one record goes to ``--db-dir`` in the
reference's DB schema (dbwrite.py). The reference's ``extra`` keys are kept;
the additions sit beside them: ``per_shape`` (GFLOP/s, % of the MI355X FP32
matrix peak, the CPU time with ``--cpu-baseline``, the library's per-kernel
launch counters), ``cpu_cores``, ``fp32_peak_gflops`` and ``route_options``.
"""

from __future__ import annotations

import argparse
import os
import statistics
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path

from .variants import CHAMPION, VARIANTS as _VARIANTS, format_variant_list

REPO_ROOT = Path(__file__).resolve().parents[1]
BASELINE = "torch_geqrf"
FP32_PEAK_GFLOPS = 157_300.0  # MI355X dense FP32 matrix (MFMA) peak
COUNTER_CALLS = 3  # traced calls per problem for the per-kernel counters
STRESS_SIZES = (32, 176, 512)  # the stress suite's orders, 4 matrices each
ALL_IMPLS = sorted(set(_VARIANTS) | {BASELINE})


def shape_name(shape: dict) -> str:
    return f"b{shape['batch']}_n{shape['n']}_cond{shape['cond']}"


def select_shapes(spec: str | None, shapes: list[dict]) -> list[dict]:
    """Official shapes named by ``b640_n512_cond2`` or by their n; all if empty."""
    if not spec:
        return list(shapes)
    wanted = {tok.strip() for tok in spec.split(",") if tok.strip()}
    chosen = [s for s in shapes if shape_name(s) in wanted or str(s["n"]) in wanted]
    if not chosen:
        raise SystemExit(f"no benchmark shapes matched --shapes={spec!r}")
    return chosen


@dataclass
class Measured:
    """One gated and timed problem."""

    name: str
    shape: dict
    check: object  # checker.CheckResult
    timing: object  # bench.TimingResult
    per_shape: dict = field(default_factory=dict)

    def db_entry(self) -> dict:
        """Entry of ``benchmark_results`` (exactly the reference's four keys)."""
        return {"shape": self.shape, "name": self.name, "correctness": self.check.as_dict(),
                "timing": self.timing.as_dict()}


class Harness:
    """The GPU side of a run; every method needs torch and a visible GPU."""

    def __init__(self, device: str, warmup: int, iters: int):
        import torch

        from . import bench, checker, inputs

        self.torch, self.bench, self.checker, self.inputs = torch, bench, checker, inputs
        self.device, self.warmup, self.iters = device, warmup, iters

    # -- inputs ---------------------------------------------------------------
    def problems(self, shapes: list[dict] | None, configs: list[int] | None):
        if configs:
            return [self.inputs.make_config_problem(c, device=self.device) for c in configs]
        return [self.inputs.make_benchmark_problem(s, device=self.device)
                for s in (shapes or self.inputs.BENCHMARK_SHAPES)]

    # -- measurements ---------------------------------------------------------
    def gate(self, fn, A):
        H, tau = fn(A)
        self.torch.cuda.synchronize()
        return self.checker.check(A, H, tau)

    def measure(self, fn, prob, cpu_baseline: bool = False, counters: bool = False) -> Measured:
        chk = self.gate(fn, prob.tensor)
        timing = self.bench.benchmark(fn, prob.tensor, warmup=self.warmup, iters=self.iters)
        rate = self.bench.qr_flops(prob.batch, prob.n) / (timing.median * 1e-3) / 1e9
        shape = {k: prob.meta[k] for k in ("batch", "n", "cond") if k in prob.meta}
        m = Measured(prob.name, shape or {"batch": prob.batch, "n": prob.n}, chk, timing,
                     {"name": prob.name, "gflops": rate,
                      "pct_peak": 100.0 * rate / FP32_PEAK_GFLOPS})
        if cpu_baseline:
            m.per_shape["cpu_geqrf_ms"] = self.cpu_geqrf_ms(prob.tensor)
        if counters:
            m.per_shape["counters"] = self.kernel_counters(fn, prob.tensor)
        return m

    def cpu_geqrf_ms(self, A, reps: int = 3) -> float:
        """Median wall time of torch.geqrf (LAPACK) on a host copy, all cores."""
        torch = self.torch
        torch.set_num_threads(cpu_cores())
        host = A.detach().cpu()
        walls = []
        for _ in range(reps):
            t0 = time.perf_counter()
            torch.geqrf(host)
            walls.append(time.perf_counter() - t0)
        return 1e3 * statistics.median(walls)

    def kernel_counters(self, fn, A) -> dict:
        """Launches, HIP-event time and algorithmic rates per call of fn(A), for
        each kernel family of the library (its launch tracer)."""
        from . import _lib

        _lib.trace_reset()
        _lib.trace_enable(list(_lib.KERNELS))
        try:
            for _ in range(COUNTER_CALLS):
                fn(A)
            self.torch.cuda.synchronize()
        finally:
            _lib.trace_enable(None)
        out = {}
        for name in _lib.KERNELS:
            t = _lib.trace_read(name)
            if t["launches"] == 0:
                continue
            sec = t["ms"] * 1e-3
            out[name] = {"launches_per_call": t["launches"] / COUNTER_CALLS,
                         "ms_per_call": t["ms"] / COUNTER_CALLS,
                         "tflops": t["flops"] / sec / 1e12 if sec > 0 else 0.0,
                         "gbs": t["bytes"] / sec / 1e9 if sec > 0 else 0.0}
        _lib.trace_reset()
        return out

    def stress(self, fn) -> list[dict]:
        """Gates on the nine stress structures at each of STRESS_SIZES."""
        rows = []
        for n in STRESS_SIZES:
            for prob in self.inputs.stress_cases(n=n, batch=4, device=self.device):
                res = self.gate(fn, prob.tensor)
                rows.append({"case": prob.name, **prob.meta, **res.as_dict()})
                print(f"  stress {prob.name:<26} {_verdict(res.passed)}  "
                      f"factor {res.factor_residual:9.2e} (<= {res.factor_threshold:.2e})  "
                      f"orth {res.orth_residual:9.2e} (<= {res.orth_threshold:.2e})")
        return rows

    def run_all(self, fn, problems, **kw) -> list[Measured]:
        done = []
        for prob in problems:
            m = self.measure(fn, prob, **kw)
            done.append(m)
            extra = (f"  cpu {m.per_shape['cpu_geqrf_ms']:.1f} ms"
                     if "cpu_geqrf_ms" in m.per_shape else "")
            print(f"  {m.name:<28} {_verdict(m.check.passed)}  median {m.timing.median:8.3f} ms"
                  f"  min {m.timing.min:8.3f} ms  {m.per_shape['gflops']:9.0f} GFLOP/s"
                  f" ({m.per_shape['pct_peak']:.1f}% peak){extra}"
                  f"  factor {m.check.factor_residual:.2e}  orth {m.check.orth_residual:.2e}")
        print(f"  geomean of medians over {len(done)} problems: "
              f"{self.bench.geomean([m.timing.median for m in done]):.4f} ms")
        return done


def _verdict(ok: bool) -> str:
    return "PASS" if ok else "FAIL"


def cpu_cores() -> int:
    """Cores this process may run on (the CPU baseline uses all of them)."""
    return len(os.sched_getaffinity(0))


def _registry() -> dict:
    from .reference import REGISTRY

    return {**REGISTRY, **_VARIANTS}


def compare(h: Harness, impls: list[str], problems) -> int:
    """Rank variants by the geomean of their medians; no record is written."""
    reg = _registry()
    torch = h.torch
    print(f"device {torch.cuda.get_device_name(0)}, torch {torch.__version__}, "
          f"hip {torch.version.hip}; {len(impls)} variants over {len(problems)} problems")
    table = []
    for impl in impls:
        print(f"-- {impl}{' (champion)' if impl == CHAMPION else ''}")
        done = h.run_all(reg[impl], problems)
        table.append((h.bench.geomean([m.timing.median for m in done]), impl,
                      all(m.check.passed for m in done)))
    table.sort()
    best = table[0][0]
    print("ranking by geomean of per-problem median ms (lower is better):")
    for rank, (gm, impl, ok) in enumerate(table, 1):
        star = " *" if impl == CHAMPION else ""
        print(f"  {rank:>2}. {impl + star:<30} {gm:12.4f} ms  x{gm / best:6.2f}  {_verdict(ok)}")
    return 0 if all(ok for _, _, ok in table) else 2


def parse_args(argv):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--impl", default=CHAMPION, choices=ALL_IMPLS)
    ap.add_argument("--device", default="cuda")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--stress", action="store_true", help="also gate the stress suite")
    ap.add_argument("--docker-image", default=None)
    ap.add_argument("--db-dir", default=str(REPO_ROOT / "db"))
    ap.add_argument("--no-write", action="store_true")
    ap.add_argument("--list", action="store_true", help="list the registered variants; no GPU")
    ap.add_argument("--compare", action="store_true", help="rank variants; writes no record")
    ap.add_argument("--impls", default=None, help="comma-separated variants for --compare")
    ap.add_argument("--shapes", default=None, help="official shapes by name or n (default: all)")
    ap.add_argument("--configs", default=None, help="headline workloads instead, e.g. 2,3,4,5")
    ap.add_argument("--cpu-baseline", action="store_true",
                    help="also time torch.geqrf on host copies of each input")
    return ap.parse_args(argv)


def main(argv: list[str] | None = None) -> int:
    args = parse_args(argv)
    if args.list:
        print(format_variant_list())
        return 0
    try:
        import torch
    except ModuleNotFoundError:
        print("ERROR: torch is not importable", file=sys.stderr)
        return 1
    if not torch.cuda.is_available():
        print("ERROR: no GPU visible to torch", file=sys.stderr)
        return 1

    from . import inputs

    h = Harness(args.device, args.warmup, args.iters)
    configs = [int(c) for c in args.configs.split(",")] if args.configs else None
    shapes = None if configs else select_shapes(args.shapes, inputs.BENCHMARK_SHAPES)
    problems = h.problems(shapes, configs)
    reg = _registry()
    if args.compare:
        impls = ([t.strip() for t in args.impls.split(",") if t.strip()] if args.impls
                 else [CHAMPION, BASELINE])
        unknown = [i for i in impls if i not in reg]
        if unknown:
            raise SystemExit(f"unknown impls for --compare: {unknown}")
        return compare(h, impls, problems)

    ours = args.impl in _VARIANTS
    print(f"impl {args.impl} on {torch.cuda.get_device_name(0)} (torch {torch.__version__}, "
          f"hip {torch.version.hip})")
    fn = reg[args.impl]
    stress = h.stress(fn) if args.stress else []
    done = h.run_all(fn, problems, cpu_baseline=args.cpu_baseline, counters=ours)
    all_pass = all(m.check.passed for m in done)
    stress_pass = all(r["passed"] for r in stress) if stress else None
    if not args.no_write:
        from . import dbwrite

        extra = {
            "warmup": args.warmup,
            "iters": args.iters,
            "all_benchmarks_pass": all_pass,
            "stress_pass": stress_pass,
            "stress_results": stress,
            "geomean_median_ms": h.bench.geomean([m.timing.median for m in done]),
            "geomean_min_ms": h.bench.geomean([m.timing.min for m in done]),
            "per_shape": [m.per_shape for m in done],
            "cpu_cores": cpu_cores() if args.cpu_baseline else None,
            "fp32_peak_gflops": FP32_PEAK_GFLOPS,
        }
        if ours:
            from . import _lib

            extra["route_options"] = _lib.default_options().as_dict()
        path = dbwrite.write_record(args.db_dir, args.impl,
                                    dbwrite.provenance(str(REPO_ROOT), args.docker_image),
                                    [m.db_entry() for m in done], extra)
        print(f"wrote {path}")
    return 0 if all_pass and stress_pass is not False else 2


if __name__ == "__main__":
    raise SystemExit(main())
