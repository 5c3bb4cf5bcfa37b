"""qr_geqrf_f32_noalloc, the allocation-free variant of qr_geqrf_f32, through
the C ABI.

Its workspace is a static 64 MiB device array shared by every call on a GPU,
which keeps the last call's contents; so two calls in a row, the second on a
smaller input, must each give exactly what qr_geqrf_f32 gives with a fresh
workspace of its own (bit for bit: the variant runs the same kernels with the
look-ahead stream off, which does not change a bit), and match the oracle.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from gpumode_qr_amd import _lib, inputs
from tests.parity import assert_parity

pytestmark = pytest.mark.gpu

DEV = "cuda"
SCRATCH_BYTES = 64 << 20  # QR_NOALLOC_SCRATCH_BYTES


def _say(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _outputs(A):
    b, n, _ = A.shape
    return A.new_empty((b, n, n)), A.new_empty((b, n))


def _noalloc(A):
    lib = _lib.load()
    H, tau = _outputs(A)
    st = lib.qr_geqrf_f32_noalloc(A.data_ptr(), *A.stride(), H.data_ptr(), tau.data_ptr(),
                                  A.shape[0], A.shape[-1], _stream())
    return st, H, tau


def _with_workspace(A):
    lib = _lib.load()
    b, n, _ = A.shape
    H, tau = _outputs(A)
    need = int(lib.qr_geqrf_f32_workspace(b, n))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=A.device)
    st = lib.qr_geqrf_f32(A.data_ptr(), *A.stride(), H.data_ptr(), tau.data_ptr(), b, n,
                          ctypes.c_void_p(ws.data_ptr()), need, _stream())
    return st, H, tau


def _gauss(batch, n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(batch, n, n, generator=g)


@pytest.mark.parametrize("shapes", [((6, 700), (3, 300)), ((4, 2048), (2, 1100)),
                                    ((40, 176), (8, 64))],
                         ids=["700_then_300", "2048_then_1100", "176_then_64"])
def test_noalloc_two_calls_second_smaller(oracle, shapes):
    for i, (b, n) in enumerate(shapes):
        _say(f"noalloc call {i + 1}: b{b} n{n}")
        A = _gauss(b, n, seed=n + i)
        Ad = A.to(DEV)
        st1, H1, t1 = _noalloc(Ad)
        st2, H2, t2 = _with_workspace(Ad)
        torch.cuda.synchronize()
        assert st1 == 0 and st2 == 0, (st1, st2)
        assert torch.equal(H1, H2) and torch.equal(t1, t2)
        k = min(b, 2)
        H_ref, tau_ref = oracle.geqrf(A[:k].numpy(), nb=16)
        assert_parity(A[:k].numpy(), H1[:k].cpu().numpy(), t1[:k].cpu().numpy(), H_ref, tau_ref,
                      what=f"noalloc b{b} n{n}")


def test_noalloc_largest_benchmark_workspace():
    # The 640 x 512 x 512 workload needs the largest workspace of the
    # benchmark configs (46 MiB): it fits, and matches qr_geqrf_f32.
    _say("noalloc b640 n512 (cond-1e2 SVD workload)")
    A = inputs.config_tensor(inputs.config_spec(3)).to(DEV)
    assert _lib.load().qr_geqrf_f32_workspace(640, 512) <= SCRATCH_BYTES
    st1, H1, t1 = _noalloc(A)
    st2, H2, t2 = _with_workspace(A)
    torch.cuda.synchronize()
    assert st1 == 0 and st2 == 0
    assert torch.equal(H1, H2) and torch.equal(t1, t2)


def test_noalloc_rejects_a_workspace_beyond_the_array():
    # 2048 matrices of n = 128 need 148 MiB: QR_EWORKSPACE before any launch.
    _say("noalloc size limit")
    lib = _lib.load()
    assert lib.qr_geqrf_f32_workspace(2048, 128) > SCRATCH_BYTES
    A = torch.zeros(2048, 128, 128, device=DEV)
    st, _, _ = _noalloc(A)
    assert st == 3
    assert lib.qr_status_string(st) == b"workspace too small"
