/*
 * qr_oracle.h -- CPU restatement of batched compact-Householder QR (fp32),
 * used ONLY by the tests, the smoke check and the CPU baseline (tests/,
 * __graft_entry__.smoke(), bench.py's cpu_baseline leg). It is never linked
 * into, or called by, the product path.
 *
 * Storage is row-major: element (i, j) of a matrix with row stride `ld`
 * lives at A[i * ld + j]. This is the layout torch uses for a contiguous
 * (batch, n, n) tensor, and the layout the reference's kernels index
 * (src/qrbench/triton_kernels.py:678-680).
 */
#ifndef QR_ORACLE_H
#define QR_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

/* Scaled 2-norm of x (n entries, stride incx): LAPACK snrm2 semantics. */
float qro_snrm2(int n, const float* x, long incx);

/* sqrt(x^2 + y^2) without destructive over/underflow: LAPACK slapy2. */
float qro_slapy2(float x, float y);

/* Elementary reflector generation, LAPACK slarfg semantics. */
void qro_slarfg(int n, float* alpha, float* x, long incx, float* tau);

/* Unblocked Householder QR of an m x n block (LAPACK sgeqr2). */
void qro_geqr2(int m, int n, float* A, long lda, float* tau);

/* Forward, column-wise compact-WY factor T (k x k, row stride ldt) of the
 * k reflectors stored below the diagonal of V (m x k): LAPACK slarft('F','C'). */
void qro_larft(int m, int k, const float* V, long ldv, const float* tau,
               float* T, long ldt);

/* C := (I - V T V^T)^T C = C - V T^T V^T C for an m x c block C:
 * LAPACK slarfb('L','T','F','C'). V is unit lower-triangular (m x k). */
void qro_larfb_lt(int m, int c, int k, const float* V, long ldv,
                  const float* T, long ldt, float* C, long ldc);

/* Right-looking blocked Householder QR of an n x n matrix with panel width
 * nb (nb <= 0: unblocked sgeqr2). In place; tau has n entries. */
void qro_geqrf(int n, float* A, long lda, float* tau, int nb);

/* Batched driver: H[b] = QR factors of A[b] (both contiguous batch x n x n). */
void qro_geqrf_batched(int batch, int n, const float* A, float* H, float* tau,
                       int nb);

/* Q (n x n, row-major) = H_0 H_1 ... H_{n-1} from (H, tau): LAPACK sorg2r. */
void qro_orgqr(int n, const float* H, const float* tau, float* Q);

#ifdef __cplusplus
}
#endif

#endif /* QR_ORACLE_H */
