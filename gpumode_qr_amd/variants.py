"""Variant registry: every variant is ``fn(A) -> (H, tau)`` in torch.geqrf form.

Mirrors the reference's plugin API (src/qrbench/variants.py:102,106,920,
1180-1296): ``VARIANTS`` maps names to callables, ``CHAMPION`` names the
current best, ``VARIANT_INFO`` carries a one-line description and a status, and
``format_variant_list()`` renders ``--list``. The module imports without torch
so ``--list`` works on a host with no GPU stack.

Registered variants:
  ``hh_mi355x``  (champion) the gfx950 HIP path: fused small-n kernel for
                 n <= 64, otherwise 16-wide panel kernel + fp32-MFMA compact-WY
                 trailing update. It replaces the reference champion
                 ``hh_panel_tuned`` (variants.py:876-917). Kernel or launch
                 failures raise; there is no silent torch.geqrf fallback inside
                 it, so a timing is always a timing of the HIP kernels.
  ``hh_mi355x_safe`` the same, but a failed call falls back to torch.geqrf,
                 matching the reference's error convention (variants.py:752-755).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

QRImpl = Callable[..., tuple]

CHAMPION = "hh_mi355x"


def _hh_mi355x(A):
    from .hip_qr import geqrf

    return geqrf(A)


def _hh_mi355x_safe(A):
    from . import _lib
    from .hip_qr import geqrf

    try:
        return geqrf(A)
    except (_lib.QRError, RuntimeError, ValueError):
        import torch

        return torch.geqrf(A)


VARIANTS: dict[str, QRImpl] = {
    "hh_mi355x": _hh_mi355x,
    "hh_mi355x_safe": _hh_mi355x_safe,
}


@dataclass(frozen=True)
class VariantInfo:
    description: str
    status: str  # active | killed | experimental | baseline


VARIANT_INFO: dict[str, VariantInfo] = {
    "torch_geqrf": VariantInfo(
        "rocSOLVER/LAPACK batched geqrf baseline (torch.geqrf)", "baseline"
    ),
    "hh_mi355x": VariantInfo(
        "gfx950 HIP: fused small-n (n<=64) / 16-wide panel + fp32-MFMA WY trailing update",
        "active",
    ),
    "hh_mi355x_safe": VariantInfo(
        "hh_mi355x with a torch.geqrf fallback on launch failure (reference error convention)",
        "experimental",
    ),
}


def describe_variants() -> list[tuple[str, VariantInfo, bool]]:
    """``(name, info, is_champion)`` for every registered impl: champion first,
    then active, experimental, killed, baseline; alphabetical within a group."""
    names = set(VARIANTS) | set(VARIANT_INFO) | {"torch_geqrf"}
    order = {"active": 0, "experimental": 1, "killed": 2, "baseline": 3}

    def info_for(name: str) -> VariantInfo:
        return VARIANT_INFO.get(name, VariantInfo("(no description)", "experimental"))

    def key(name: str):
        return (0 if name == CHAMPION else 1, order.get(info_for(name).status, 9), name)

    return [(n, info_for(n), n == CHAMPION) for n in sorted(names, key=key)]


def format_variant_list() -> str:
    rows = describe_variants()
    lines = ["Registered QR implementations (★ = current champion):", ""]
    width = max((len(n) for n, _, _ in rows), default=12)
    for name, info, champ in rows:
        mark = "★" if champ else " "
        lines.append(f"  {mark} {name:<{width}}  [{info.status:^12}]  {info.description}")
    lines.append("")
    lines.append(f"Champion: {CHAMPION}")
    lines.append("Compare live:  python -m gpumode_qr_amd.run_baseline --compare")
    return "\n".join(lines)
