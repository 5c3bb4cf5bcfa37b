"""Torch-facing wrappers of the gfx950 QR kernels.

``geqrf(A) -> (H, tau)`` is the drop-in forward pass: same contract as
``torch.geqrf`` and the reference's variants (src/qrbench/reference.py:15-20,
src/qrbench/variants.py:102): ``A`` is ``(batch, n, n)`` float32 on a GPU and is
not modified; ``H`` (row-major contiguous) holds R on and above the diagonal and
the essential Householder vectors below it; ``tau`` is ``(batch, n)``. All work
is enqueued on torch's current stream of ``A``'s device; nothing synchronises.

The other functions expose the individual kernels (panel, larft, WY update) for
the parity tests. Torch is only used for device memory and the stream.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

try:  # CPython binding of qr_geqrf_f32 (csrc/qr_fastcall.c), built with the library
    from . import _qr_fastcall
except ImportError:
    _qr_fastcall = None

PANEL = 16  # panel width of the blocked route
SMALL_N = 64  # largest n of the fused one-wave-per-matrix route (no workspace)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# Raw handle of the current stream of a device index, and the current device
# index. torch's own accessors cost about 0.1 us where the public
# current_stream(...).cuda_stream costs about 2 us; geqrf's host work sits inside
# every event-timed call, so it uses them when this torch build has them.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_cur_device = getattr(torch._C, "_cuda_getDevice", None)


def _stream_of(index: int) -> int:
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def _current_device() -> int:
    return _cur_device() if _cur_device is not None else torch.cuda.current_device()


# qr_geqrf_f32 as geqrf calls it, and the library it was taken from: through
# the CPython binding when it is built (about 0.1 us per call against about 1 us
# for ctypes' conversion of eleven arguments; the call sits inside every
# event-timed call), else through ctypes. Both call the same library function.
_geqrf_lib = None
_geqrf_fn = None


def _geqrf_entry(lib):
    global _geqrf_lib, _geqrf_fn
    if _geqrf_lib is not lib:
        if _qr_fastcall is not None:
            _qr_fastcall.bind(ctypes.cast(lib.qr_geqrf_f32, ctypes.c_void_p).value)
            _geqrf_fn = _qr_fastcall.geqrf
        else:
            _geqrf_fn = lib.qr_geqrf_f32
        _geqrf_lib = lib
    return _geqrf_fn


def _check_input(A: torch.Tensor) -> None:
    if not isinstance(A, torch.Tensor):
        raise TypeError("A must be a torch.Tensor")
    shape = A.shape
    if len(shape) != 3 or shape[1] != shape[2]:
        raise ValueError(f"A must be (batch, n, n); got {tuple(shape)}")
    if A.dtype is not torch.float32:
        raise TypeError(f"A must be float32; got {A.dtype}")
    if not A.is_cuda:
        raise ValueError("A must be on a GPU device (the HIP path has no CPU fallback)")


def workspace_bytes(batch: int, n: int) -> int:
    return int(_lib.load().qr_geqrf_f32_workspace(batch, n))


def options(**changes) -> _lib.Options:
    """Route options (``struct qr_options``): the defaults with ``changes``
    applied, e.g. ``options(cholqr=0)`` or ``options(lookahead=0)``."""
    o = _lib.default_options()
    for name, value in changes.items():
        if not hasattr(o, name):
            raise TypeError(f"unknown route option {name!r}")
        setattr(o, name, int(value))
    return o


def geqrf(A: torch.Tensor, workspace: torch.Tensor | None = None,
          options: _lib.Options | None = None):
    """Batched compact-Householder QR on the GPU: ``(H, tau)`` like torch.geqrf.

    ``options`` (from :func:`options`) selects a non-default route or
    schedule; None runs the defaults. The host work between the caller's
    stream position and the launch is kept small (it is inside every
    event-timed call): no workspace query for n <= 64, no device switch when
    ``A`` is on the current device.
    """
    _check_input(A)
    lib = _lib.load()
    b, n, _ = A.shape
    H = A.new_empty((b, n, n))  # float32 on A's device, like A
    tau = A.new_empty((b, n))
    if b == 0 or n == 0:
        return H, tau
    need = 0 if n <= SMALL_N else int(lib.qr_geqrf_f32_workspace(b, n))
    if need:
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=A.device)
        ws_ptr, ws_len = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    else:
        ws_ptr, ws_len = None, 0
    sb, sr, sc = A.stride()
    args = (A.data_ptr(), sb, sr, sc, H.data_ptr(), tau.data_ptr(), b, n, ws_ptr, ws_len)
    index = A.get_device()
    if options is None:
        fn = _geqrf_entry(lib)
        call = lambda: fn(*args, _stream_of(index))  # noqa: E731
    else:
        call = lambda: lib.qr_geqrf_f32_ex(*args, ctypes.byref(options),  # noqa: E731
                                           _stream_of(index))
    if index == _current_device():
        st = call()
    else:
        with torch.cuda.device(index):
            st = call()
    if st:
        _lib.check("qr_geqrf_f32", st)
    return H, tau


def route_codes(workspace: torch.Tensor, batch: int, n: int) -> torch.Tensor:
    """Route of each matrix in the last 64-column block that took the
    CholeskyQR2 route in the last geqrf call with this workspace:
    0 two passes, 1 Householder panels (guard failed), 2 one pass."""
    off = int(_lib.load().qr_geqrf_f32_route_codes_offset(batch, n))
    if off == 0:
        raise ValueError(f"no CholeskyQR2 workspace for batch={batch}, n={n}")
    return workspace[off:off + 4 * batch].view(torch.int32).clone()


def fused_smalln(A: torch.Tensor):
    """Kernel (a) alone, one launch: n <= 64 one wavefront per matrix,
    64 < n <= 192 one workgroup per matrix (a wavefront per 16-column strip)."""
    _check_input(A)
    lib = _lib.load()
    b, n, _ = A.shape
    H = torch.empty((b, n, n), dtype=torch.float32, device=A.device)
    tau = torch.empty((b, n), dtype=torch.float32, device=A.device)
    sb, sr, sc = A.stride()
    with torch.cuda.device(A.device):
        st = lib.qr_fused_smalln_f32(
            A.data_ptr(), sb, sr, sc, H.data_ptr(), tau.data_ptr(), b, n, _stream(A.device)
        )
    _lib.check("qr_fused_smalln_f32", st)
    return H, tau


def panel(P: torch.Tensor, p: int = 0, T_prev: torch.Tensor | None = None):
    """Kernel (b) alone on a batch of (r, 16 p + kw) blocks (kw <= 16).

    Panels 0..p-1 of each block must already be factored in place (V below the
    diagonal) with their 16 x 16 T factors in ``T_prev`` (batch, p, 16, 16).
    Panel p (columns 16p..16p+kw-1) first gets Q_{0..p-1}^T applied, then is
    factored. Returns ``(H_blk, tau_p, T_p)``: the block with panel p factored in
    geqrf packing, its kw reflector coefficients and its 16 x 16 T (zero beyond
    kw), like the reference's ``hh_panel_qr`` minus the explicit V
    (src/qrbench/triton_kernels.py:912-967).
    """
    if P.dim() != 3 or P.dtype != torch.float32 or P.device.type != "cuda":
        raise ValueError("P must be a (batch, r, width) float32 GPU tensor")
    lib = _lib.load()
    b, r, width = P.shape
    kw = width - PANEL * p
    Hp = P.contiguous().clone()
    tau = torch.zeros((b, width), dtype=torch.float32, device=P.device)
    T = torch.zeros((b, p + 1, PANEL, PANEL), dtype=torch.float32, device=P.device)
    if p:
        T[:, :p] = T_prev
    with torch.cuda.device(P.device):
        st = lib.qr_panel_f32(
            Hp.data_ptr(), r * width, width, 0, p, r, kw, tau.data_ptr(), width, T.data_ptr(),
            (p + 1) * PANEL * PANEL, b, _stream(P.device),
        )
    _lib.check("qr_panel_f32", st)
    return Hp, tau[:, PANEL * p:], T[:, p]


def larft(V: torch.Tensor, tau: torch.Tensor):
    """Kernel (c) alone: T (k x k) of reflectors stored below the diagonal of V."""
    if V.dim() != 3 or tau.dim() != 2:
        raise ValueError("V must be (batch, m, k) and tau (batch, k)")
    lib = _lib.load()
    b, m, k = V.shape
    Vc = V.contiguous()
    tc = tau.contiguous()
    T = torch.empty((b, k, k), dtype=torch.float32, device=V.device)
    with torch.cuda.device(V.device):
        st = lib.qr_larft_f32(
            Vc.data_ptr(), m * k, k, m, k, tc.data_ptr(), k, T.data_ptr(), k * k, k, b,
            _stream(V.device),
        )
    _lib.check("qr_larft_f32", st)
    return T


def wy_update(Hblk: torch.Tensor, T: torch.Tensor):
    """Kernel (d) alone: ``Hblk`` (batch, r, 16 nblk + c) holds nblk factored
    16-wide panels (V below the diagonal) followed by c columns C; ``T``
    (batch, nblk, 16, 16) their T factors. Returns a copy with C replaced by
    Q^T C = (H_{nblk-1} ... H_0) C."""
    lib = _lib.load()
    b, r, width = Hblk.shape
    nblk = T.shape[1]
    c = width - PANEL * nblk
    out = Hblk.contiguous().clone()
    Tc = T.contiguous()
    with torch.cuda.device(Hblk.device):
        st = lib.qr_wy_update_f32(
            out.data_ptr(), r * width, width, 0, nblk, r, c, Tc.data_ptr(),
            nblk * PANEL * PANEL, b, _stream(Hblk.device),
        )
    _lib.check("qr_wy_update_f32", st)
    return out


def _ormqr_into(H: torch.Tensor, tau: torch.Tensor, C: torch.Tensor, trans: bool) -> None:
    lib = _lib.load()
    b, n, m = C.shape
    need = int(lib.qr_ormqr_f32_workspace(b, n))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=C.device)
    with torch.cuda.device(C.device):
        st = lib.qr_ormqr_f32(
            H.data_ptr(), H.stride(0), H.stride(1), tau.data_ptr(), tau.stride(0), C.data_ptr(),
            C.stride(0), C.stride(1), n, m, int(trans), b, ws.data_ptr(), need,
            _stream(C.device),
        )
    _lib.check("qr_ormqr_f32", st)


def _check_factors(H: torch.Tensor, tau: torch.Tensor) -> None:
    _check_input(H)
    b, n, _ = H.shape
    if tau.shape != (b, n) or tau.dtype != torch.float32 or tau.device != H.device:
        raise ValueError(f"tau must be float32 ({b}, {n}) on {H.device}")


def ormqr(H: torch.Tensor, tau: torch.Tensor, C: torch.Tensor, transpose: bool = False):
    """``Q^T C`` (``transpose=True``) or ``Q C`` for the Q of ``(H, tau)`` from
    :func:`geqrf`; ``C`` is ``(batch, n, m)`` and is not modified (LAPACK sormqr,
    side 'L')."""
    _check_factors(H, tau)
    b, n, _ = H.shape
    if C.dim() != 3 or C.shape[:2] != (b, n) or C.dtype != torch.float32 or C.device != H.device:
        raise ValueError(f"C must be float32 ({b}, {n}, m) on {H.device}")
    out = C.contiguous().clone()
    if out.numel():
        _ormqr_into(H.contiguous(), tau.contiguous(), out, transpose)
    return out


def orgqr(H: torch.Tensor, tau: torch.Tensor) -> torch.Tensor:
    """Q (batch, n, n) of ``(H, tau)`` from :func:`geqrf`, like
    ``torch.linalg.householder_product(H, tau)`` (LAPACK sorgqr)."""
    _check_factors(H, tau)
    lib = _lib.load()
    b, n, _ = H.shape
    Hc, tc = H.contiguous(), tau.contiguous()
    Q = torch.empty((b, n, n), dtype=torch.float32, device=H.device)
    if Q.numel() == 0:
        return Q
    need = int(lib.qr_ormqr_f32_workspace(b, n))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=H.device)
    with torch.cuda.device(H.device):
        st = lib.qr_orgqr_f32(
            Hc.data_ptr(), Hc.stride(0), Hc.stride(1), tc.data_ptr(), tc.stride(0), Q.data_ptr(),
            Q.stride(0), Q.stride(1), n, b, ws.data_ptr(), need, _stream(H.device),
        )
    _lib.check("qr_orgqr_f32", st)
    return Q
