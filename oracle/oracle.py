"""numpy/ctypes front end of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only to check or time against it. The product
path in ``gpumode_qr_amd`` never imports it.

All arrays are numpy float32, C-contiguous, row-major, shaped like the torch
tensors of the reference contract: ``A``/``H`` ``(batch, n, n)``, ``tau``
``(batch, n)`` (reference: src/qrbench/reference.py:15-20).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libqr_oracle.so"
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (gcc only; seconds)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.qro_snrm2.restype = ctypes.c_float
        lib.qro_snrm2.argtypes = [ctypes.c_int, _f32p, ctypes.c_long]
        lib.qro_slapy2.restype = ctypes.c_float
        lib.qro_slapy2.argtypes = [ctypes.c_float, ctypes.c_float]
        lib.qro_slarfg.restype = None
        lib.qro_slarfg.argtypes = [ctypes.c_int, _f32p, _f32p, ctypes.c_long, _f32p]
        lib.qro_geqr2.restype = None
        lib.qro_geqr2.argtypes = [ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_long, _f32p]
        lib.qro_larft.restype = None
        lib.qro_larft.argtypes = [
            ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_long, _f32p, _f32p, ctypes.c_long,
        ]
        lib.qro_larfb_lt.restype = None
        lib.qro_larfb_lt.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_long,
            _f32p, ctypes.c_long, _f32p, ctypes.c_long,
        ]
        lib.qro_geqrf.restype = None
        lib.qro_geqrf.argtypes = [ctypes.c_int, _f32p, ctypes.c_long, _f32p, ctypes.c_int]
        lib.qro_geqrf_batched.restype = None
        lib.qro_geqrf_batched.argtypes = [
            ctypes.c_int, ctypes.c_int, _f32p, _f32p, _f32p, ctypes.c_int,
        ]
        lib.qro_orgqr.restype = None
        lib.qro_orgqr.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def slarfg(alpha: float, x) -> tuple[float, np.ndarray, float]:
    """Reflector of [alpha; x]: returns (beta, v_essential, tau)."""
    lib = _load()
    x = _f32(x).copy()
    a = ctypes.c_float(alpha)
    t = ctypes.c_float(0.0)
    lib.qro_slarfg(x.size + 1, ctypes.byref(a), _ptr(x) if x.size else _f32p(), 1, ctypes.byref(t))
    return float(a.value), x, float(t.value)


def snrm2(x) -> float:
    x = _f32(x)
    return float(_load().qro_snrm2(x.size, _ptr(x) if x.size else _f32p(), 1))


def geqr2(A) -> tuple[np.ndarray, np.ndarray]:
    """Unblocked QR of one m x n matrix: returns (H, tau)."""
    H = _f32(A).copy()
    m, n = H.shape
    tau = np.zeros(min(m, n), dtype=np.float32)
    _load().qro_geqr2(m, n, _ptr(H), n, _ptr(tau))
    return H, tau


def larft(V, tau) -> np.ndarray:
    """T (k x k) of the reflectors stored below the diagonal of V (m x k)."""
    V = _f32(V)
    tau = _f32(tau)
    m, k = V.shape
    T = np.zeros((k, k), dtype=np.float32)
    _load().qro_larft(m, k, _ptr(V), k, _ptr(tau), _ptr(T), k)
    return T


def larfb_lt(V, T, C) -> np.ndarray:
    """C - V T^T V^T C with V unit lower (m x k), T upper (k x k), C (m x c)."""
    V = _f32(V)
    T = _f32(T)
    C = _f32(C).copy()
    m, k = V.shape
    c = C.shape[1]
    _load().qro_larfb_lt(m, c, k, _ptr(V), k, _ptr(T), k, _ptr(C), c)
    return C


def geqrf(A, nb: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Batched QR (batch, n, n) -> (H, tau); nb <= 0 is unblocked."""
    A = _f32(A)
    squeeze = A.ndim == 2
    if squeeze:
        A = A[None]
    b, n, n2 = A.shape
    assert n == n2
    H = np.empty_like(A)
    tau = np.empty((b, n), dtype=np.float32)
    if b and n:
        _load().qro_geqrf_batched(b, n, _ptr(A), _ptr(H), _ptr(tau), int(nb))
    if squeeze:
        return H[0], tau[0]
    return H, tau


def orgqr(H, tau) -> np.ndarray:
    """Q = H_0 ... H_{n-1} of one square (H, tau)."""
    H = _f32(H)
    tau = _f32(tau)
    n = H.shape[0]
    Q = np.empty((n, n), dtype=np.float32)
    _load().qro_orgqr(n, _ptr(H), _ptr(tau), _ptr(Q))
    return Q
