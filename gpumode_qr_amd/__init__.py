"""gpumode_qr_amd -- batched compact-Householder QR (fp32, torch.geqrf layout)
on AMD MI355X (gfx950) with hand-written HIP kernels behind a C ABI.

Same harness surface as the reference's ``qrbench`` package
(jamesETsmith/gpumode_qr, src/qrbench/__init__.py):

- ``inputs``:    benchmark shapes, the five headline configs, stress cases
- ``checker``:   FP64 factor-residual / orthogonality gates
- ``reference``: the ``torch.geqrf`` baseline and the run registry
- ``variants``:  the variant registry (``VARIANTS``, ``CHAMPION``)
- ``bench``:     HIP-event timing harness and geomean
- ``dbwrite``:   one JSON record per run
- ``hip_qr``:    the gfx950 kernels (``geqrf`` is the drop-in forward pass)
"""

EPS32 = 2.0**-23  # float32 machine epsilon, as in the reference's qrbench/__init__.py:11

__all__ = ["EPS32"]
