"""The C-ABI library loads and exports every symbol include/*.h declares.

No compute call is made here: argument-validation paths return before any HIP
call, so these run without a GPU.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from gpumode_qr_amd import _lib

INCLUDE = Path(__file__).resolve().parents[1] / "include"


def _declared_functions() -> set[str]:
    names = set()
    for hdr in INCLUDE.glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", hdr.read_text(), flags=re.S)
        for m in re.finditer(r"\b(?:int|size_t|void|const char\*)\s+(qr_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from gpumode_qr_amd.csrc import build

        build.build()
    return _lib.load()


def test_header_declares_the_bound_symbols():
    assert _declared_functions() == set(_lib.SIGNATURES)


def test_every_declared_symbol_is_exported(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_abi_and_limits(lib):
    assert lib.qr_abi_version() == _lib.ABI_VERSION
    assert lib.qr_max_n() == 4096
    assert lib.qr_status_string(0) == b"ok"
    assert lib.qr_status_string(3) == b"workspace too small"
    assert lib.qr_status_string(99) == b"unknown status"


def test_workspace_query(lib):
    assert lib.qr_geqrf_f32_workspace(64, 32) == 0  # fused route needs none
    assert lib.qr_geqrf_f32_workspace(0, 512) == 0
    ws = lib.qr_geqrf_f32_workspace(640, 512)
    assert ws >= 640 * 8 * 16 * 16 * 4
    assert ws % 256 == 0


def test_argument_validation_without_launch(lib):
    p = ctypes.c_void_p(0x1000)
    h = ctypes.c_void_p(0x10000000)
    t = ctypes.c_void_p(0x20000000)
    # empty problems are a successful no-op
    assert lib.qr_geqrf_f32(None, 0, 0, 0, None, None, 0, 8, None, 0, None) == 0
    assert lib.qr_geqrf_f32(None, 0, 0, 0, None, None, 4, 0, None, 0, None) == 0
    # negative sizes, too-large n, null pointers, negative strides
    assert lib.qr_geqrf_f32(p, 1, 1, 1, h, t, -1, 8, None, 0, None) == 1
    assert lib.qr_geqrf_f32(p, 1, 1, 1, h, t, 1, 5000, None, 0, None) == 2
    assert lib.qr_geqrf_f32(None, 64, 8, 1, h, t, 1, 8, None, 0, None) == 1
    assert lib.qr_geqrf_f32(p, -64, 8, 1, h, t, 1, 8, None, 0, None) == 1
    # H overlapping A
    assert lib.qr_geqrf_f32(h, 64, 8, 1, h, t, 1, 8, None, 0, None) == 1
    # workspace missing for the blocked route
    assert lib.qr_geqrf_f32(p, 200 * 200, 200, 1, h, t, 1, 200, None, 0, None) == 3
    # kernel-level entry points
    assert lib.qr_fused_smalln_f32(p, 200 * 200, 200, 1, h, t, 1, 200, None) == 2
    assert lib.qr_panel_f32(h, 100, 10, 0, 0, 10, 17, t, 17, t, 256, 1, None) == 1  # kw > 16
    assert lib.qr_panel_f32(h, 9000, 90, 0, 8, 200, 16, t, 90, t, 4096, 1, None) == 1  # p >= 8
    assert lib.qr_panel_f32(h, 9000, 90, 0, 2, 40, 16, t, 90, t, 512, 1, None) == 1  # r < 16p+kw
    assert lib.qr_larft_f32(h, 100, 70, 100, 70, t, 70, t, 4900, 70, 1, None) == 2
    assert lib.qr_wy_update_f32(h, 1000, 50, 0, 9, 200, 4, t, 4096, 1, None) == 1  # nblk > 8
    assert lib.qr_wy_update_f32(h, 1000, 50, 0, 2, 5000, 4, t, 512, 1, None) == 2  # r > 4096
    # orgqr / ormqr
    assert lib.qr_ormqr_f32_workspace(2, 100) >= 2 * 7 * 256 * 4  # one 16 x 16 T per panel
    assert lib.qr_ormqr_f32_workspace(0, 100) == 0
    assert lib.qr_ormqr_f32(h, 10000, 100, t, 100, p, 10000, 100, 100, 100, 2, 1, h, 1 << 20,
                            None) == 1  # trans not 0/1
    assert lib.qr_ormqr_f32(h, 10000, 100, t, 100, p, 10000, 100, 100, 100, 1, 1, None, 0,
                            None) == 3  # no workspace
    assert lib.qr_ormqr_f32(h, 10000, 50, t, 100, p, 10000, 100, 100, 100, 1, 1, h, 1 << 20,
                            None) == 1  # ldh < n
    assert lib.qr_ormqr_f32(h, 1, 5000, t, 5000, p, 1, 5000, 5000, 8, 1, 1, h, 1 << 30,
                            None) == 2  # n > 4096
    assert lib.qr_ormqr_f32(h, 0, 0, t, 0, p, 0, 0, 0, 8, 1, 1, None, 0, None) == 0  # n = 0
    assert lib.qr_orgqr_f32(h, 10000, 100, t, 100, h, 10000, 100, 100, 1, h, 1 << 20,
                            None) == 1  # Q overlaps H


def test_route_options_defaults_and_validation(lib):
    o = _lib.default_options()
    assert o.as_dict() == {"cholqr": 1, "cholqr_min_rows": 0, "cholqr_one_pass": 1,
                           "cholqr_fused": 0, "lookahead": 1, "outer_panels": 0, "midn": 1}
    p = ctypes.c_void_p(0x1000)
    h = ctypes.c_void_p(0x10000000)
    t = ctypes.c_void_p(0x20000000)
    ex = lib.qr_geqrf_f32_ex
    assert ex(p, 200 * 200, 200, 1, h, t, 1, 200, None, 0, None, None) == 3  # NULL: defaults
    for field, bad in (("cholqr", 2), ("cholqr_min_rows", 64), ("cholqr_min_rows", 5000),
                       ("cholqr_one_pass", -1), ("cholqr_one_pass", 3), ("cholqr_fused", 2),
                       ("lookahead", 7),
                       ("outer_panels", 9), ("outer_panels", -1), ("midn", 3), ("midn", -1)):
        o = _lib.default_options()
        setattr(o, field, bad)
        assert ex(p, 200 * 200, 200, 1, h, t, 1, 200, None, 0, ctypes.byref(o), None) == 1, field
    o = _lib.default_options()
    o.cholqr_min_rows = 65
    assert ex(p, 200 * 200, 200, 1, h, t, 1, 200, None, 0, ctypes.byref(o), None) == 3


def test_route_codes_lie_inside_the_workspace(lib):
    for batch, n in ((1, 65), (2, 4096), (64, 1024), (640, 512), (2048, 128)):
        off = lib.qr_geqrf_f32_route_codes_offset(batch, n)
        assert 0 < off and off + 4 * batch <= lib.qr_geqrf_f32_workspace(batch, n)
        assert off % 4 == 0
    assert lib.qr_geqrf_f32_route_codes_offset(8, 64) == 0  # fused small-n route: none


def test_fastcall_binding_matches_ctypes(lib):
    """geqrf's CPython binding of qr_geqrf_f32 (built with the library) returns
    the library's own status codes on the validation paths, and rejects
    arguments that do not fit the C parameters instead of truncating them."""
    from gpumode_qr_amd import hip_qr
    from gpumode_qr_amd.csrc import build

    if not build.FASTCALL.exists():
        build.build_fastcall()
        pytest.skip("binding built by this test: rerun to load it")
    fn = hip_qr._geqrf_entry(lib)
    assert hip_qr._qr_fastcall is not None and fn is hip_qr._qr_fastcall.geqrf
    cases = [
        (0, 1, 1, 1, 0, 0, -1, 4, None, 0, 0),       # negative batch
        (0, 1, 1, 1, 0, 0, 4, -1, None, 0, 0),       # negative n
        (0, 1, 1, 1, 0, 0, 1, 70000, None, 0, 0),    # n above qr_max_n
        (0, 1, 1, 1, 0, 0, 1, 4, None, 0, 0),        # null pointers
        (16, 64 * 64, 64, 1, 16, 16, 3, 64, None, 0, 0),  # H aliases A
    ]
    for args in cases:
        assert fn(*args) == lib.qr_geqrf_f32(*args) != 0, args
    with pytest.raises(OverflowError):
        fn(0, 1, 1, 1, 0, 0, 2**31, 4, None, 0, 0)
    with pytest.raises(OverflowError):
        fn(0, 1, 1, 1, 0, 0, 1, 4, None, -1, 0)
    with pytest.raises(TypeError):
        fn(0, 1, 1, 1, 0, 0, 1, 4, None, 0)
