"""Run only the QR forward pass on one config's input, for profilers.

    python -m gpumode_qr_amd.profile_run --config 4 --calls 3

Unlike ``bench.py`` this runs no FP64 gates (they call torch's
householder_product) and no torch.geqrf, so a ``rocprofv3 --pmc`` pass over it
sees the library's own kernels and nothing else. Every call of ``geqrf``
launches the same kernels, so per-dispatch counters divide cleanly by call.
``k_copy_in`` reads ``batch * n * n * 4`` bytes and writes as many: it is the
known-size copy that calibrates FETCH_SIZE / WRITE_SIZE.
"""

from __future__ import annotations

import argparse
import sys


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, default=4, help="1..5 (the benchmark configs)")
    ap.add_argument("--calls", type=int, default=3)
    args = ap.parse_args(argv)

    import torch

    from . import _lib, hip_qr, inputs

    if not torch.cuda.is_available():
        print("profile_run needs a GPU", file=sys.stderr)
        return 1
    _lib.load()
    prob = inputs.make_config_problem(args.config, device="cuda")
    A = prob.tensor
    b, n = prob.batch, prob.n
    ws = torch.empty(max(1, hip_qr.workspace_bytes(b, n)), dtype=torch.uint8, device="cuda")
    print(f"[profile_run] {prob.name}: batch={b} n={n}, copy-in bytes per call "
          f"{b * n * n * 4} read + {b * n * n * 4} written", flush=True)
    for i in range(args.calls):
        hip_qr.geqrf(A, workspace=ws)
        torch.cuda.synchronize()
        print(f"[profile_run] call {i + 1}/{args.calls} done", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
