"""Write tests/golden/geqrf_mkl.npz: small seeded inputs and the (H, tau) that
LAPACK (MKL sgeqrf, reached through torch.geqrf on the CPU) returns for them.

The reference repository holds no golden arrays (its correctness evidence is
the FP64 gate residuals in db/*.json), so these vectors come from an
independent LAPACK implementation on the same contract the reference checks
against (src/qrbench/checker.py, reference.py:18-20). They pin the oracle's
slarfg branches, including the rescaling paths (tiny / huge / zero columns).

Run from the repo root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "geqrf_mkl.npz"


def cases() -> dict[str, np.ndarray]:
    g = torch.Generator().manual_seed(20260101)

    def randn(*shape):
        return torch.randn(*shape, generator=g, dtype=torch.float32)

    out: dict[str, torch.Tensor] = {}
    for n in (1, 2, 3, 5, 8, 16, 33, 64):
        out[f"gauss_n{n}"] = randn(3, n, n)
    a = randn(3, 24, 24)
    a[:, :, 5] = 0.0
    out["zero_col_n24"] = a
    a = randn(3, 24, 24)
    a[:, :, 7] *= 1e4
    out["big_col_n24"] = a
    a = randn(3, 24, 24)
    a[:, :, 3] *= 1e-30  # squares underflow fp32: scaled-norm path
    out["tiny_col_n24"] = a
    a = randn(3, 24, 24)
    a[:, :, 4] *= 1e25  # squares overflow fp32: scaled-norm path
    out["huge_col_n24"] = a
    a = randn(3, 24, 24)
    a[:, :, 2] *= 1e-40  # denormal column: slarfg's safmin rescale loop
    out["denormal_col_n24"] = a
    out["upper_tri_n20"] = torch.triu(randn(3, 20, 20))
    out["rank1_n16"] = randn(3, 16, 1) @ randn(3, 1, 16)
    return {k: v.numpy() for k, v in out.items()}


def main() -> None:
    arrays = {}
    for name, A in cases().items():
        H, tau = torch.geqrf(torch.from_numpy(A))
        arrays[f"{name}__A"] = A
        arrays[f"{name}__H"] = H.contiguous().numpy()
        arrays[f"{name}__tau"] = tau.contiguous().numpy()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({len(arrays) // 3} cases)")


if __name__ == "__main__":
    main()
