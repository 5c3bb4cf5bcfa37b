"""Build libqr_gfx950.so in-tree with hipcc for gfx950.

Usage: ``python -m gpumode_qr_amd.csrc.build`` (also called by
``__graft_entry__.build()``). Each ``.hip`` file is compiled to an object in
parallel, then linked into ``gpumode_qr_amd/libqr_gfx950.so``. The default
build also compiles ``qr_fastcall.c`` (the CPython binding of ``qr_geqrf_f32``)
with the host C compiler into ``gpumode_qr_amd/_qr_fastcall*.so``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
REPO = PKG.parent
OUT_DIR = PKG / "_build"
LIB = PKG / "libqr_gfx950.so"
FASTCALL = PKG / ("_qr_fastcall" + sysconfig.get_config_var("EXT_SUFFIX"))
ARCH = "gfx950"

SOURCES = [
    "qr_smalln.hip", "qr_midn.hip", "qr_blocked.hip", "qr_cholqr.hip", "qr_apply.hip", "qr_larft.hip",
    "qr_copy.hip", "qr_orgqr_smalln.hip", "qr_api.hip",
]

# -packed-fp32-ops: keep hipcc from forming v_pk_{add,mul,fma}_f32 (the host
# pass warns that it does not know the feature; that is expected).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _compile(src: str, out_dir: Path = OUT_DIR, defines: tuple[str, ...] = ()) -> Path:
    obj = out_dir / (Path(src).stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *(f"-D{d}" for d in defines), "-c", str(CSRC / src), "-o",
           str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed on {src}")
    return obj


def build(verbose: bool = False, out: Path = LIB, defines: tuple[str, ...] = ()) -> Path:
    """Compile and link the library to ``out``; ``defines`` are extra ``-D`` tuning
    macros (the defaults in the sources are the tuned ones)."""
    obj_dir = OUT_DIR if out == LIB else OUT_DIR / out.stem
    obj_dir.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(lambda src: _compile(src, obj_dir, defines), SOURCES))
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc link failed")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    if out == LIB:
        build_fastcall(verbose)
    return out


def build_fastcall(verbose: bool = False) -> Path:
    """The CPython binding of ``qr_geqrf_f32`` (``qr_fastcall.c``): Python's
    headers only, no HIP."""
    cc = os.environ.get("CC") or shutil.which("gcc") or "cc"
    tmp = FASTCALL.with_name(FASTCALL.name + ".tmp")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", "-Werror",
           f"-I{sysconfig.get_paths()['include']}", str(CSRC / "qr_fastcall.c"), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("C compiler failed on qr_fastcall.c")
    os.replace(tmp, FASTCALL)
    if verbose:
        print(f"built {FASTCALL}")
    return FASTCALL


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser()
    ap.add_argument("--out", type=Path, default=LIB)
    ap.add_argument("-D", dest="defines", action="append", default=[])
    a = ap.parse_args()
    build(verbose=True, out=a.out.resolve(), defines=tuple(a.defines))
