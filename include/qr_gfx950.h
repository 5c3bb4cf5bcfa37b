/*
 * qr_gfx950.h -- C ABI of libqr_gfx950.so: batched compact-Householder QR
 * (fp32, torch.geqrf layout) with hand-written gfx950 HIP kernels.
 *
 * Every pointer is a device pointer on the current HIP device; every call is
 * asynchronous on `stream` (an opaque hipStream_t; NULL is the null stream) and
 * returns a qr_status. Matrices are row-major: element (i, j) of matrix b of H
 * is H[b * sHb + i * ldh + j]. No call allocates device memory or synchronises
 * (the launch tracer at the end records and reads HIP events).
 *
 * The reference's plugin boundary is a Python callable
 * `fn(A: (batch, n, n) fp32) -> (H, tau)` registered by name
 * (reference src/qrbench/reference.py:15, src/qrbench/variants.py:102,920);
 * gpumode_qr_amd/variants.py wraps qr_geqrf_f32 behind exactly that signature.
 */
#ifndef QR_GFX950_H
#define QR_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum qr_status {
  QR_OK = 0,
  QR_EINVAL = 1,       /* bad argument: sizes, strides, null pointers, aliasing */
  QR_EUNSUPPORTED = 2, /* n outside the supported range */
  QR_EWORKSPACE = 3,   /* workspace smaller than qr_geqrf_f32_workspace() */
  QR_ELAUNCH = 4       /* a HIP launch failed (hipGetLastError) */
} qr_status;

/* Kernel identifiers for the launch tracer (bit i of the trace mask). */
typedef enum qr_kernel_id {
  QR_KERNEL_SMALLN = 0,   /* kernel (a) */
  QR_KERNEL_PANEL = 1,    /* kernel (b) */
  QR_KERNEL_WY_W2 = 2,    /* kernel (d), W2 = T^T V^T C */
  QR_KERNEL_WY_APPLY = 3, /* kernel (d), C -= V W2 */
  QR_KERNEL_COPY = 4,     /* strided A -> H copy */
  QR_KERNEL_LARFT = 5     /* kernel (c) */
} qr_kernel_id;

/* Human-readable text for a qr_status value (static storage). */
const char* qr_status_string(int status);

/* Library ABI version (bumped on any signature change). */
int qr_abi_version(void);

/* Largest n that qr_geqrf_f32 accepts. */
int qr_max_n(void);

/* Bytes of device workspace qr_geqrf_f32 needs for (batch, n); 0 if none. */
size_t qr_geqrf_f32_workspace(int batch, int n);

/*
 * Full factorisation, replacing the champion variant's forward pass
 * (reference src/qrbench/variants.py:876-917 -> :761-805 for n > 128 and
 * :698-758 for n <= 128; baseline torch.geqrf at src/qrbench/reference.py:18-20).
 * A: (batch, n, n) with element strides (sAb, sAr, sAc), read only.
 * H: contiguous (batch, n, n) output, R on and above the diagonal, essential
 *    Householder vectors below it. tau: contiguous (batch, n) output.
 * H must not overlap A.
 */
int qr_geqrf_f32(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H, float* tau,
                 int batch, int n, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Kernel (a): fused small-n factorisation, n <= 64, one wavefront per matrix.
 * Replaces hh_fused_qr / _hh_fused_qr_kernel (reference
 * src/qrbench/triton_kernels.py:641-755). Same arguments as qr_geqrf_f32.
 */
int qr_fused_smalln_f32(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                        float* tau, int batch, int n, void* stream);

/*
 * Kernel (b): in-place factorisation of the r x kw panel (kw <= 16, r >= kw)
 * whose top-left element is H[b*sHb + j0*ldh + j0], writing tau[b*sTaub + j0 + i]
 * and the panel's 16 x 16 upper T (row-major, zero beyond kw) to T[b*sTb ...].
 * Replaces hh_panel_qr / _hh_panel_kernel (reference
 * src/qrbench/triton_kernels.py:787-967), which returns (H_p, V, tau, T).
 */
int qr_panel_f32(float* H, int64_t sHb, int64_t ldh, int j0, int r, int kw, float* tau,
                 int64_t sTaub, float* T, int64_t sTb, int batch, void* stream);

/*
 * Kernel (c): T (k x k, row stride ldt) of the k <= 64 reflectors stored below
 * the diagonal of V (m x k, row stride ldv) with coefficients tau.
 * Replaces the T build of reference src/qrbench/triton_kernels.py:886-909.
 */
int qr_larft_f32(const float* V, int64_t sVb, int64_t ldv, int m, int k, const float* tau,
                 int64_t sTaub, float* T, int64_t sTb, int64_t ldt, int batch, void* stream);

/*
 * Kernel (d): C -= V T^T V^T C for the 16-wide reflector block of the panel at
 * (j0, j0) and the c columns right of it (C = H[.. j0 .., j0+16 : j0+16+c]),
 * r rows. T as written by qr_panel_f32. Workspace: 16 * c floats per matrix.
 * Replaces the trailing GEMMs of reference src/qrbench/variants.py:800-804.
 */
int qr_wy_update_f32(float* H, int64_t sHb, int64_t ldh, int j0, int r, int c, const float* T,
                     int64_t sTb, void* workspace, size_t workspace_bytes, int batch,
                     void* stream);

/*
 * Launch tracer (measurement only; no counterpart in the reference, whose
 * timing is torch.cuda.Event around whole calls, src/qrbench/bench.py:57-77).
 * While bit k of `kernel_mask` is set, every launch of kernel k made by the
 * calls above is bracketed by two HIP events recorded on the launch stream,
 * together with that launch's algorithmic flops and bytes.
 * qr_trace_read waits for the recorded events of one kernel and returns the
 * launch count, the summed event time (ms) and the summed flops and bytes.
 */
int qr_trace_enable(unsigned kernel_mask);
int qr_trace_reset(void);
int qr_trace_read(int kernel, int* launches, double* total_ms, double* flops, double* bytes);

#ifdef __cplusplus
}
#endif

#endif /* QR_GFX950_H */
