"""Run only the QR forward pass on one config's input, for profilers.

    python -m gpumode_qr_amd.profile_run --config 4 --calls 3
    python -m gpumode_qr_amd.profile_run --shape 2x4096 --calls 3

Unlike ``bench.py`` this runs no FP64 gates (they call torch's
householder_product) and no torch.geqrf, so a ``rocprofv3 --pmc`` pass over it
sees the library's own kernels and nothing else. Every call of ``geqrf``
launches the same kernels, so per-dispatch counters divide cleanly by call.

Before the calls it runs one ``torch.neg(A, out=C)``: an elementwise kernel
that reads ``batch * n * n * 4`` bytes and writes as many, the known-size
transfer that calibrates FETCH_SIZE / WRITE_SIZE.

``--shape BxN`` factors B seeded N(0,1) matrices of order N instead of a config
(the official shapes' sizes, e.g. 2x4096).

``--layout colmajor`` passes the same matrices as a column-major view, which
geqrf first copies into H with ``k_copy_in`` (with the row-major default the
first outer block reads A in place and there is no copy).
"""

from __future__ import annotations

import argparse
import sys


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, default=4, help="1..5 (the benchmark configs)")
    ap.add_argument("--shape", default=None, help="BxN: B seeded N(0,1) matrices of order N")
    ap.add_argument("--calls", type=int, default=3)
    ap.add_argument("--layout", choices=("rowmajor", "colmajor"), default="rowmajor",
                    help="colmajor: a column-major view of the same matrices (adds k_copy_in)")
    args = ap.parse_args(argv)

    import torch

    from . import _lib, hip_qr, inputs

    if not torch.cuda.is_available():
        print("profile_run needs a GPU", file=sys.stderr)
        return 1
    _lib.load()
    if args.shape:
        b_, n_ = (int(x) for x in args.shape.lower().split("x"))
        g = torch.Generator().manual_seed(n_)
        A = torch.randn(b_, n_, n_, generator=g).to("cuda")
        prob = inputs.Problem(name=f"b{b_}_n{n_}_gauss", tensor=A, meta={})
    else:
        prob = inputs.make_config_problem(args.config, device="cuda")
        A = prob.tensor
    if args.layout == "colmajor":
        A = A.transpose(-1, -2).contiguous().transpose(-1, -2)
    b, n = prob.batch, prob.n
    ws = torch.empty(max(1, hip_qr.workspace_bytes(b, n)), dtype=torch.uint8, device="cuda")
    print(f"[profile_run] {prob.name}: batch={b} n={n} layout={args.layout}; calibration "
          f"kernel (neg) reads {b * n * n * 4} bytes and writes as many", flush=True)
    C = torch.empty_like(A)
    torch.neg(A, out=C)  # calibration: b n^2 4 bytes read, as many written
    torch.cuda.synchronize()
    del C
    for i in range(args.calls):
        hip_qr.geqrf(A, workspace=ws)
        torch.cuda.synchronize()
        print(f"[profile_run] call {i + 1}/{args.calls} done", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
