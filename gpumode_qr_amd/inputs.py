"""Problem generation: official benchmark shapes, the five headline configs,
and the correctness stress structures.

API follows the reference's src/qrbench/inputs.py:20-135 (``BENCHMARK_SHAPES``,
``Problem``, ``make_benchmark_problem``, ``stress_cases``). One deliberate
difference: every input is drawn from a seeded **CPU** ``torch.Generator`` and
then copied to the target device, so the same seed gives bit-identical inputs on
every box and the CPU baseline factors exactly the matrices the GPU factors.
(The reference draws from a device generator, inputs.py:46-49.)

The headline configs (``CONFIGS``) are:
  1. batch 64,   n 32,   iid N(0,1), torch.manual_seed(0)   (CPU plumbing)
  2. batch 2048, n 64,   iid N(0,1)
  3. batch 640,  n 512,  U diag(s) V^T, U, V Haar, s = logspace(0, -2, n)
  4. batch 64,   n 1024, iid N(0,1)
  5. batch 16,   n 2048, 8 x U diag(logspace(0, -6, n)) V^T and 8 Gaussian
     matrices with column n//3 zeroed and column 2n//3 scaled by 1e4.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from pathlib import Path

import torch

# The seven ranked shapes of the GPUMODE task (reference inputs.py:20-28).
BENCHMARK_SHAPES: list[dict] = [
    {"batch": 20, "cond": 1, "n": 32},
    {"batch": 40, "cond": 1, "n": 176},
    {"batch": 40, "cond": 1, "n": 352},
    {"batch": 640, "cond": 2, "n": 512},
    {"batch": 60, "cond": 2, "n": 1024},
    {"batch": 8, "cond": 1, "n": 2048},
    {"batch": 2, "cond": 1, "n": 4096},
]

# The five headline benchmark configs (name -> spec).
CONFIGS: list[dict] = [
    {"cfg": 1, "name": "cfg1_b64_n32_gauss", "batch": 64, "n": 32, "kind": "gauss", "seed": 0},
    {"cfg": 2, "name": "cfg2_b2048_n64_gauss", "batch": 2048, "n": 64, "kind": "gauss", "seed": 2},
    {"cfg": 3, "name": "cfg3_b640_n512_svd_cond1e2", "batch": 640, "n": 512, "kind": "svd",
     "log10_cond": 2.0, "seed": 3},
    {"cfg": 4, "name": "cfg4_b64_n1024_gauss", "batch": 64, "n": 1024, "kind": "gauss", "seed": 4},
    {"cfg": 5, "name": "cfg5_b16_n2048_stress", "batch": 16, "n": 2048, "kind": "stress5",
     "log10_cond": 6.0, "seed": 5},
]


@dataclass
class Problem:
    name: str
    tensor: torch.Tensor  # (batch, n, n) float32
    meta: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return self.tensor.shape[0]

    @property
    def n(self) -> int:
        return self.tensor.shape[-1]


def _cpu_gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def _column_scaled_dense(batch: int, n: int, cond: float, seed: int) -> torch.Tensor:
    """N(0,1) matrix with columns scaled by logspace(0, -cond, n) (reference inputs.py:52-60)."""
    a = torch.randn(batch, n, n, generator=_cpu_gen(seed), dtype=torch.float32)
    scale = torch.logspace(0, -float(cond), n, dtype=torch.float32)
    return a * scale


def make_benchmark_problem(shape: dict, seed: int = 0, device: str | torch.device = "cuda") -> Problem:
    """One of the official shapes, e.g. ``{"batch": 640, "cond": 2, "n": 512}``."""
    batch, n, cond = shape["batch"], shape["n"], shape["cond"]
    t = _column_scaled_dense(batch, n, cond, seed).to(device)
    return Problem(name=f"b{batch}_n{n}_cond{cond}", tensor=t, meta=dict(shape))


def _haar(batch: int, n: int, g: torch.Generator) -> torch.Tensor:
    """Haar-distributed orthogonal matrices (fp64): Q of a Gaussian with the
    column signs fixed by sign(diag R)."""
    G = torch.randn(batch, n, n, generator=g, dtype=torch.float64)
    Hq, tq = torch.geqrf(G)
    Q = torch.linalg.householder_product(Hq, tq)
    d = torch.diagonal(Hq, dim1=-2, dim2=-1)
    sign = torch.where(d < 0, -1.0, 1.0).to(torch.float64)
    return Q * sign.unsqueeze(-2)


def svd_matrices(batch: int, n: int, log10_cond: float, g: torch.Generator) -> torch.Tensor:
    """A = U diag(s) V^T, U, V Haar, s = logspace(0, -log10_cond, n); formed in
    fp64, returned as fp32."""
    s = torch.logspace(0, -float(log10_cond), n, dtype=torch.float64)
    out = torch.empty(batch, n, n, dtype=torch.float32)
    step = max(1, min(batch, (1 << 26) // (n * n)))  # bound fp64 temporaries
    for b0 in range(0, batch, step):
        b1 = min(batch, b0 + step)
        U = _haar(b1 - b0, n, g)
        V = _haar(b1 - b0, n, g)
        out[b0:b1] = ((U * s) @ V.transpose(-2, -1)).to(torch.float32)
    return out


def _cache_path(spec: dict) -> Path | None:
    root = os.environ.get("QR_INPUT_CACHE")
    if not root:
        return None
    return Path(root) / f"{spec['name']}_seed{spec['seed']}.pt"


_MEMO: dict[tuple, torch.Tensor] = {}


def config_tensor(spec: dict) -> torch.Tensor:
    """CPU fp32 input of a headline config (deterministic for its seed).

    Generated tensors are memoised per process (treat them as read-only); set
    QR_INPUT_CACHE to a directory to also keep them across processes."""
    key = tuple(sorted((k, str(v)) for k, v in spec.items()))
    if key in _MEMO:
        return _MEMO[key]
    A = _config_tensor(spec)
    _MEMO[key] = A
    return A


def _config_tensor(spec: dict) -> torch.Tensor:
    cache = _cache_path(spec)
    if cache is not None and cache.exists():
        return torch.load(cache, weights_only=True)
    b, n, seed, kind = spec["batch"], spec["n"], spec["seed"], spec["kind"]
    if kind == "gauss":
        if spec["cfg"] == 1:
            torch.manual_seed(seed)  # config 1 is defined by torch.manual_seed(0)
            A = torch.randn(b, n, n, dtype=torch.float32)
        else:
            A = torch.randn(b, n, n, generator=_cpu_gen(seed), dtype=torch.float32)
    elif kind == "svd":
        A = svd_matrices(b, n, spec["log10_cond"], _cpu_gen(seed))
    elif kind == "stress5":
        g = _cpu_gen(seed)
        half = b // 2
        A = torch.empty(b, n, n, dtype=torch.float32)
        A[:half] = svd_matrices(half, n, spec["log10_cond"], g)
        G = torch.randn(b - half, n, n, generator=g, dtype=torch.float32)
        G[:, :, n // 3] = 0.0
        G[:, :, (2 * n) // 3] *= 1e4
        A[half:] = G
    else:
        raise ValueError(f"unknown config kind {kind!r}")
    if cache is not None:
        cache.parent.mkdir(parents=True, exist_ok=True)
        torch.save(A, cache)
    return A


def config_spec(cfg: int) -> dict:
    """The workload whose ``"cfg"`` number is ``cfg`` (1-5)."""
    for spec in CONFIGS:
        if spec["cfg"] == cfg:
            return spec
    raise KeyError(f"no workload numbered {cfg}")


def make_config_problem(cfg: int, device: str | torch.device = "cuda") -> Problem:
    spec = config_spec(cfg)
    return Problem(name=spec["name"], tensor=config_tensor(spec).to(device), meta=dict(spec))


def _dense(batch, n, cond, g):
    a = torch.randn(batch, n, n, generator=g, dtype=torch.float32)
    return a * torch.logspace(0, -float(cond), n, dtype=torch.float32)


def stress_cases(n: int, batch: int = 4, seed: int = 1234,
                 device: str | torch.device = "cuda") -> list[Problem]:
    """The nine correctness-only structures of the reference's stress suite
    (inputs.py:84-135), drawn from one seeded CPU generator in the same order."""
    g = _cpu_gen(seed)
    out: list[Problem] = []

    def add(name, t, **meta):
        out.append(Problem(name=f"{name}_n{n}", tensor=t.contiguous().to(device), meta=meta))

    add("dense_cond1", _dense(batch, n, 1, g), kind="dense", cond=1)
    add("dense_cond4", _dense(batch, n, 4, g), kind="dense", cond=4)
    r = max(1, n // 2)
    u = torch.randn(batch, n, r, generator=g, dtype=torch.float32)
    v = torch.randn(batch, r, n, generator=g, dtype=torch.float32)
    add("rank_deficient", u @ v, kind="rank_deficient", rank=r)
    tiny = 1e-6 * torch.randn(batch, n, n, generator=g, dtype=torch.float32)
    add("near_rank_deficient", u @ v + tiny, kind="near_rank_deficient", rank=r)
    full = torch.randn(batch, n, n, generator=g, dtype=torch.float32)
    bw = max(1, n // 16)
    idx = torch.arange(n)
    add("banded", full * ((idx[None, :] - idx[:, None]).abs() <= bw), kind="banded", bandwidth=bw)
    base = torch.randn(batch, n, n, generator=g, dtype=torch.float32)
    add("row_scaled", base * torch.logspace(0, -6, n, dtype=torch.float32).view(1, n, 1),
        kind="row_scaled")
    direction = torch.randn(batch, n, 1, generator=g, dtype=torch.float32)
    perturb = 1e-4 * torch.randn(batch, n, n, generator=g, dtype=torch.float32)
    add("near_collinear", direction + perturb, kind="near_collinear")
    add("upper_triangular", torch.triu(torch.randn(batch, n, n, generator=g, dtype=torch.float32)),
        kind="upper_triangular")
    clustered = torch.randn(batch, n, n, generator=g, dtype=torch.float32)
    cscale = torch.ones(n, dtype=torch.float32)
    cscale[n // 2:] = 1e-5
    add("clustered_scale", clustered * cscale, kind="clustered_scale")
    return out
