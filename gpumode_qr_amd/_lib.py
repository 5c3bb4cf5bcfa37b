"""ctypes binding of libqr_gfx950.so (declared in include/qr_gfx950.h).

The library is built in-tree by ``python -m gpumode_qr_amd.csrc.build`` (or
``__graft_entry__.build()``). There is no fallback: if the shared library is
missing, every entry point raises. ``QR_GFX950_LIB`` names another build of
the same library (for example one built with different tuning defines).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

DEFAULT_LIB_PATH = Path(__file__).resolve().parent / "libqr_gfx950.so"
LIB_PATH = Path(os.environ.get("QR_GFX950_LIB") or DEFAULT_LIB_PATH)


class Options(ctypes.Structure):
    """struct qr_options of include/qr_gfx950.h (route and schedule choices)."""

    _fields_ = [
        ("cholqr", ctypes.c_int),
        ("cholqr_min_rows", ctypes.c_int),
        ("cholqr_one_pass", ctypes.c_int),
        ("cholqr_fused", ctypes.c_int),
        ("lookahead", ctypes.c_int),
        ("outer_panels", ctypes.c_int),
        ("midn", ctypes.c_int),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


# Every symbol include/qr_gfx950.h declares, with (restype, argtypes).
_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_size = ctypes.c_size_t

SIGNATURES: dict[str, tuple] = {
    "qr_status_string": (ctypes.c_char_p, [_int]),
    "qr_abi_version": (_int, []),
    "qr_max_n": (_int, []),
    "qr_geqrf_f32_workspace": (_size, [_int, _int]),
    "qr_geqrf_f32": (
        _int,
        [_ptr, _i64, _i64, _i64, _ptr, _ptr, _int, _int, _ptr, _size, _ptr],
    ),
    "qr_default_options": (None, [ctypes.POINTER(Options)]),
    "qr_geqrf_f32_ex": (
        _int,
        [_ptr, _i64, _i64, _i64, _ptr, _ptr, _int, _int, _ptr, _size, ctypes.POINTER(Options),
         _ptr],
    ),
    "qr_geqrf_f32_route_codes_offset": (_size, [_int, _int]),
    "qr_geqrf_f32_noalloc": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _int, _int, _ptr]),
    "qr_fused_smalln_f32": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _int, _int, _ptr]),
    "qr_panel_f32": (
        _int,
        [_ptr, _i64, _i64, _int, _int, _int, _int, _ptr, _i64, _ptr, _i64, _int, _ptr],
    ),
    "qr_larft_f32": (
        _int,
        [_ptr, _i64, _i64, _int, _int, _ptr, _i64, _ptr, _i64, _i64, _int, _ptr],
    ),
    "qr_ormqr_f32_workspace": (_size, [_int, _int]),
    "qr_ormqr_f32": (
        _int,
        [_ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _int, _int, _int, _int, _ptr, _size, _ptr],
    ),
    "qr_orgqr_f32": (
        _int,
        [_ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _int, _int, _ptr, _size, _ptr],
    ),
    "qr_wy_update_f32": (
        _int,
        [_ptr, _i64, _i64, _int, _int, _int, _int, _ptr, _i64, _int, _ptr],
    ),
    "qr_trace_enable": (_int, [ctypes.c_uint]),
    "qr_trace_reset": (_int, []),
    "qr_trace_read": (
        _int,
        [
            _int,
            ctypes.POINTER(_int),
            ctypes.POINTER(ctypes.c_double),
            ctypes.POINTER(ctypes.c_double),
            ctypes.POINTER(ctypes.c_double),
        ],
    ),
}

# qr_kernel_id values of include/qr_gfx950.h
KERNELS = {"smalln": 0, "panel": 1, "trail": 2, "copy": 3, "larft": 4, "apply": 5, "cholqr": 6}

ABI_VERSION = 5

QR_OK = 0


class QRError(RuntimeError):
    """A nonzero qr_status returned by the HIP library."""

    def __init__(self, func: str, status: int, text: str):
        super().__init__(f"{func} failed: status {status} ({text})")
        self.status = status


_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m gpumode_qr_amd.csrc.build` "
                "(there is no CPU or library fallback for this path)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.qr_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"{LIB_PATH} ABI {lib.qr_abi_version()} != expected {ABI_VERSION}; rebuild it"
            )
        _lib = lib
    return _lib


def trace_enable(names: list[str] | None) -> None:
    """Trace the launches of the named kernels (None or [] disables tracing)."""
    mask = 0
    for nm in names or []:
        mask |= 1 << KERNELS[nm]
    check("qr_trace_enable", load().qr_trace_enable(mask))


def trace_reset() -> None:
    check("qr_trace_reset", load().qr_trace_reset())


def trace_read(name: str) -> dict:
    """Launch count, summed event ms, summed algorithmic flops/bytes of a kernel."""
    cnt = _int(0)
    ms = ctypes.c_double(0.0)
    fl = ctypes.c_double(0.0)
    by = ctypes.c_double(0.0)
    check("qr_trace_read", load().qr_trace_read(KERNELS[name], ctypes.byref(cnt), ctypes.byref(ms),
                                                 ctypes.byref(fl), ctypes.byref(by)))
    return {"launches": cnt.value, "ms": ms.value, "flops": fl.value, "bytes": by.value}


def default_options() -> Options:
    """The options qr_geqrf_f32 runs with."""
    o = Options()
    load().qr_default_options(ctypes.byref(o))
    return o


def check(func: str, status: int) -> None:
    if status != QR_OK:
        text = load().qr_status_string(status).decode()
        raise QRError(func, status, text)
