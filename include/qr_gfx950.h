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
  QR_KERNEL_SMALLN = 0, /* kernel (a) */
  QR_KERNEL_PANEL = 1,  /* kernel (b), incl. its left-looking block update */
  QR_KERNEL_TRAIL = 2,  /* kernel (d), trailing compact-WY update */
  QR_KERNEL_COPY = 3,   /* A -> H copy (only for A without a unit column stride) */
  QR_KERNEL_LARFT = 4,  /* kernel (c) */
  QR_KERNEL_APPLY = 5,  /* block-reflector application of orgqr / ormqr */
  QR_KERNEL_CHOLQR = 6  /* CholeskyQR2 + reconstruction of a 64-column block (its 4-5 launches) */
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
 * Outer blocks of >= 128 rows (calls of at most 64 matrices; >= 576 rows above)
 * are factored by CholeskyQR2 with Householder reconstruction (the CholeskyQR
 * route of references/nvidia_winner_sol_combo.md:1051-1052), with the same
 * (V, tau, R) output; matrices it cannot factor to that standard take the
 * Householder panels.
 * A: (batch, n, n) with element strides (sAb, sAr, sAc), read only. With
 *    sAc == 1 the kernels read A in place; other layouts are first copied
 *    into H.
 * H: contiguous (batch, n, n) output, R on and above the diagonal, essential
 *    Householder vectors below it. tau: contiguous (batch, n) output.
 * H must not overlap A.
 */
int qr_geqrf_f32(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H, float* tau,
                 int batch, int n, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Route and schedule choices of qr_geqrf_f32_ex. The library reads no
 * environment variable: a call runs with exactly the options it is given
 * (qr_geqrf_f32 uses qr_default_options). No counterpart in the reference,
 * whose variants are separate registered functions (src/qrbench/variants.py:
 * 920-1163); these select among the schedules of this one variant, for tests
 * and measurements. Every choice gives the same (V, tau, R) within the parity
 * tolerance; look-ahead and the panel count within an outer block give the
 * same bits.
 */
typedef struct qr_options {
  int cholqr;          /* 1 (default): 64-column outer blocks of >= cholqr_min_rows rows take
                          the CholeskyQR2 route; 0: Householder panels for every block */
  int cholqr_min_rows; /* 0 (default): 128 rows in calls of <= 64 matrices, 576 above;
                          else the row bound itself (>= 65) */
  int cholqr_one_pass; /* 1 (default): one CholeskyQR pass where ||R1s^-1||_F^2 <= 144,
                          else two; 0: always two; 2: one pass only, a matrix that would
                          need the second takes the Householder panels for that block (no
                          pass-2 launches). The fused variant always takes two. */
  int cholqr_fused;    /* 0 (default): five launches per block; 1: Gram and per-matrix
                          steps fused (the last workgroup of a matrix does its step) */
  int lookahead;       /* 1 (default): rest of the trailing update on a second stream */
  int outer_panels;    /* 16-wide panels per outer block, 1..8; 0 (default): 4. The
                          CholeskyQR2 route needs 4. */
  int midn;            /* 64 < n <= 192: 1 (default) the one-launch fused kernel when
                          batch * ceil(n / 16) <= 8192, else the blocked route, whose last
                          r <= 192 columns the kernel factors in place when batch *
                          ceil(r / 16) <= 2048, and whose last r <= 64 columns the small-n
                          kernel factors in place; 0: the blocked route throughout; 2: the
                          fused kernels for every such matrix and last block */
} qr_options;

/* Fills *opts with the defaults qr_geqrf_f32 runs with. */
void qr_default_options(qr_options* opts);

/*
 * qr_geqrf_f32 with explicit route options (NULL: the defaults). Returns
 * QR_EINVAL for an option outside its documented range.
 */
int qr_geqrf_f32_ex(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H, float* tau,
                    int batch, int n, void* workspace, size_t workspace_bytes,
                    const qr_options* opts, void* stream);

/*
 * Byte offset, within a qr_geqrf_f32 workspace for (batch, n), of `batch`
 * int32 route codes written by the last 64-column block that took the
 * CholeskyQR2 route in a call: 0 two passes, 1 Householder panels (the
 * matrix failed the route's guard), 2 one pass. Diagnostic only (tests read
 * it to know which route a matrix took); no counterpart in the reference.
 */
size_t qr_geqrf_f32_route_codes_offset(int batch, int n);

/* Size of the static device workspace of qr_geqrf_f32_noalloc (per GPU). */
#define QR_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/*
 * qr_geqrf_f32 for callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * No counterpart in the reference. The workspace is a static device array of
 * QR_NOALLOC_SCRATCH_BYTES (64 MiB) that each GPU the library runs on holds
 * until the process ends; the call allocates nothing, creates no stream or
 * event, and enqueues every kernel on `stream` (no look-ahead stream), with
 * results bit-identical to qr_geqrf_f32's. Returns QR_EWORKSPACE when
 * qr_geqrf_f32_workspace(batch, n) exceeds the array (about 880 matrices of
 * n = 512, 110 of n = 1024 up to 64). Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (two streams, two host threads)
 * race, and must be ordered by the caller. The first call on a device looks
 * up the array's device address (hipGetSymbolAddress).
 */
int qr_geqrf_f32_noalloc(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                         float* tau, int batch, int n, void* stream);

/*
 * Kernel (a): fused whole-matrix factorisation in one launch, n <= 192: one
 * wavefront per matrix for n <= 64; one workgroup per matrix (a wavefront per
 * 16-column strip, the matrix held in registers) for 64 < n <= 192.
 * Replaces hh_fused_qr / _hh_fused_qr_kernel (reference
 * src/qrbench/triton_kernels.py:641-755) and the fused route of
 * make_hh_fused_smalln (src/qrbench/variants.py:739-758, n <= 128). Same
 * arguments as qr_geqrf_f32; QR_EUNSUPPORTED above n = 192.
 */
int qr_fused_smalln_f32(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                        float* tau, int batch, int n, void* stream);

/*
 * Kernel (b): factor panel p (0 <= p < 8, width kw <= 16) of the outer block
 * whose top-left element is H[b*sHb + j0*ldh + j0] and which has r rows.
 * The panel's columns are j0+16p .. j0+16p+kw-1 and its diagonal starts at row
 * j0+16p. Panels 0..p-1 of the same block must already be factored, with their
 * 16 x 16 upper T factors at T[b*sTb + 256q]; they are applied to the panel's
 * columns first (left-looking). Writes V / R in place, tau[b*sTaub + j0+16p+i]
 * and the panel's T (zero beyond kw) at T[b*sTb + 256p].
 * Replaces hh_panel_qr / _hh_panel_kernel (reference
 * src/qrbench/triton_kernels.py:787-967), which returns (H_p, V, tau, T), and
 * the in-block part of the trailing GEMMs (src/qrbench/variants.py:800-804).
 */
int qr_panel_f32(float* H, int64_t sHb, int64_t ldh, int j0, int p, int r, int kw, float* tau,
                 int64_t sTaub, float* T, int64_t sTb, int batch, void* stream);

/*
 * Kernel (c): T (k x k, row stride ldt) of the k <= 64 reflectors stored below
 * the diagonal of V (m x k, row stride ldv) with coefficients tau.
 * Replaces the T build of reference src/qrbench/triton_kernels.py:886-909.
 */
int qr_larft_f32(const float* V, int64_t sVb, int64_t ldv, int m, int k, const float* tau,
                 int64_t sTaub, float* T, int64_t sTb, int64_t ldt, int batch, void* stream);

/*
 * Kernel (d): C := Q^T C for the nblk <= 8 factored 16-wide panels of the outer
 * block at (j0, j0) (r rows; their T factors at T[b*sTb + 256q]), where C is
 * the c columns starting at column j0 + 16*nblk, rows j0 .. j0+r-1. The blocks
 * are applied in order 0..nblk-1, each as C -= V_q T_q^T V_q^T C.
 * Replaces the trailing GEMMs of reference src/qrbench/variants.py:800-804.
 */
int qr_wy_update_f32(float* H, int64_t sHb, int64_t ldh, int j0, int nblk, int r, int c,
                     const float* T, int64_t sTb, int batch, void* stream);

/*
 * Bytes of device workspace qr_ormqr_f32 / qr_orgqr_f32 need for (batch, n):
 * the 16 x 16 T of every 16-wide panel.
 */
size_t qr_ormqr_f32_workspace(int batch, int n);

/*
 * Apply Q of a factorisation (H, tau) from qr_geqrf_f32 (n x n, row stride ldh)
 * to C (n x m, row stride ldc) in place: trans = 1 gives C := Q^T C, trans = 0
 * gives C := Q C, with Q = H_0 H_1 ... H_{n-1} (LAPACK sormqr, side = 'L').
 * T of each panel is rebuilt from (H, tau) (larft), then the 16-wide block
 * reflectors are applied with FP32 MFMA. No counterpart kernel in the
 * reference: its consumers of (H, tau) call torch's householder_product and
 * matmul (src/qrbench/checker.py:129-158).
 */
int qr_ormqr_f32(const float* H, int64_t sHb, int64_t ldh, const float* tau, int64_t sTaub,
                 float* C, int64_t sCb, int64_t ldc, int n, int m, int trans, int batch,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Form Q (n x n, row stride ldq; must not overlap H) of a factorisation
 * (H, tau): Q := Q I (LAPACK sorgqr). Replaces
 * torch.linalg.householder_product(H, tau) as used by the reference's gates
 * (src/qrbench/checker.py:129). n <= 64 runs one launch (a wavefront per
 * matrix, Q formed in registers); larger n the per-panel T rebuild and the
 * block-reflector application.
 */
int qr_orgqr_f32(const float* H, int64_t sHb, int64_t ldh, const float* tau, int64_t sTaub,
                 float* Q, int64_t sQb, int64_t ldq, int n, int batch, void* workspace,
                 size_t workspace_bytes, void* stream);

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
