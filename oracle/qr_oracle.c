/*
 * qr_oracle.c -- CPU restatement of the reference's batched compact-Householder
 * QR path, in plain fp32 C.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as a checker. The product
 * path (gpumode_qr_amd/) never calls it and has no CPU fallback.
 *
 * What each function restates (reference = jamesETsmith/gpumode_qr):
 *   qro_slarfg   per-column reflector of src/qrbench/triton_kernels.py:686-700
 *                (beta = -sign(alpha)*norm, tau = (beta-alpha)/beta,
 *                v = x * 1/(alpha-beta), sigma==0 -> tau=0, beta=alpha), with the
 *                LAPACK slarfg scaling rules the build contract asks for on top:
 *                scaled norm (snrm2), slapy2 and the |beta| < safmin rescale
 *                loop. The reference itself uses the unscaled sqrt(alpha^2+sigma).
 *   qro_geqr2    the per-column loop of triton_kernels.py:684-719 (apply H_j to
 *                the trailing columns, pack beta on the diagonal and the
 *                essential reflector below it, store tau_j).
 *   qro_larft    the in-kernel T build of triton_kernels.py:886-909 (forward
 *                LARFT: T[i,i] = tau_i, T[0:i,i] = -tau_i T[0:i,0:i] V[:,0:i]^T v_i).
 *   qro_larfb_lt the trailing update of src/qrbench/variants.py:800-804
 *                (C -= V (T^T (V^T C))).
 *   qro_geqrf    the right-looking blocked loop of variants.py:786-805.
 *   qro_orgqr    Q = H_0 ... H_{n-1}, i.e. what the reference's gates build with
 *                torch.linalg.householder_product (src/qrbench/checker.py:129).
 *
 * Parity pins (tests/test_oracle.py): MKL sgeqrf via torch.geqrf on CPU and the
 * committed fixtures in tests/golden/, the fp64 factor/orthogonality gates,
 * closed forms (1x1, 2x2, slarfg vs fp64 hypot), known answers (upper-
 * triangular input -> H == A and tau == 0; zero column -> tau == 0; last tau of
 * a square matrix == 0) and identities (I - V T V^T == householder_product;
 * larfb == (I - V T V^T)^T C in fp64).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include "qr_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* LAPACK slamch('S') / slamch('E') = 2^-126 / 2^-24. */
static const float QRO_SAFMIN = 0x1p-102f;
static const float QRO_RSAFMN = 0x1p102f;

float qro_snrm2(int n, const float* x, long incx)
{
    /* Classic LAPACK scaled sum of squares: scale * sqrt(ssq). */
    if (n < 1) return 0.0f;
    float scale = 0.0f, ssq = 1.0f;
    for (int i = 0; i < n; ++i) {
        const float v = x[(long)i * incx];
        if (v != 0.0f) {
            const float av = fabsf(v);
            if (scale < av) {
                const float r = scale / av;
                ssq = 1.0f + ssq * r * r;
                scale = av;
            } else {
                const float r = av / scale;
                ssq += r * r;
            }
        }
    }
    return scale * sqrtf(ssq);
}

float qro_slapy2(float x, float y)
{
    if (isnan(x)) return x;
    if (isnan(y)) return y;
    const float xa = fabsf(x), ya = fabsf(y);
    const float w = xa > ya ? xa : ya;
    const float z = xa < ya ? xa : ya;
    if (z == 0.0f || w > FLT_MAX) return w;
    const float q = z / w;
    return w * sqrtf(1.0f + q * q);
}

static void qro_sscal(int n, float a, float* x, long incx)
{
    for (int i = 0; i < n; ++i) x[(long)i * incx] *= a;
}

void qro_slarfg(int n, float* alpha, float* x, long incx, float* tau)
{
    if (n <= 1) {
        *tau = 0.0f;
        return;
    }
    float xnorm = qro_snrm2(n - 1, x, incx);
    if (xnorm == 0.0f) {
        /* H = I: tau = 0, beta = alpha, x untouched. */
        *tau = 0.0f;
        return;
    }
    float a = *alpha;
    float beta = -copysignf(qro_slapy2(a, xnorm), a);
    int knt = 0;
    if (fabsf(beta) < QRO_SAFMIN) {
        do {
            ++knt;
            qro_sscal(n - 1, QRO_RSAFMN, x, incx);
            beta *= QRO_RSAFMN;
            a *= QRO_RSAFMN;
        } while (fabsf(beta) < QRO_SAFMIN && knt < 20);
        xnorm = qro_snrm2(n - 1, x, incx);
        beta = -copysignf(qro_slapy2(a, xnorm), a);
    }
    *tau = (beta - a) / beta;
    qro_sscal(n - 1, 1.0f / (a - beta), x, incx);
    for (int j = 0; j < knt; ++j) beta *= QRO_SAFMIN;
    *alpha = beta;
}

/* C (m x c) -= tau * v * (v^T C), v of length m with v[0] == 1 implied. */
static void qro_larf_left(int m, int c, const float* v, long incv, float tau,
                          float* C, long ldc, float* work)
{
    if (tau == 0.0f) return;
    for (int k = 0; k < c; ++k) work[k] = C[k]; /* v[0] == 1 */
    for (int i = 1; i < m; ++i) {
        const float vi = v[(long)i * incv];
        const float* Ci = C + (long)i * ldc;
        for (int k = 0; k < c; ++k) work[k] += vi * Ci[k];
    }
    for (int k = 0; k < c; ++k) C[k] -= tau * work[k];
    for (int i = 1; i < m; ++i) {
        const float vi = v[(long)i * incv];
        float* Ci = C + (long)i * ldc;
        for (int k = 0; k < c; ++k) Ci[k] -= tau * vi * work[k];
    }
}

void qro_geqr2(int m, int n, float* A, long lda, float* tau)
{
    const int kmax = m < n ? m : n;
    float* work = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    for (int j = 0; j < kmax; ++j) {
        float* ajj = A + (long)j * lda + j;
        qro_slarfg(m - j, ajj, ajj + lda, lda, &tau[j]);
        if (j + 1 < n) qro_larf_left(m - j, n - j - 1, ajj, lda, tau[j], ajj + 1, lda, work);
    }
    free(work);
}

/* V[i][j] of a unit lower-trapezoidal reflector block stored in place. */
static inline float qro_vij(const float* V, long ldv, int i, int j)
{
    if (i < j) return 0.0f;
    if (i == j) return 1.0f;
    return V[(long)i * ldv + j];
}

void qro_larft(int m, int k, const float* V, long ldv, const float* tau,
               float* T, long ldt)
{
    for (int i = 0; i < k; ++i) {
        for (int p = 0; p < k; ++p) T[(long)p * ldt + i] = 0.0f;
        if (tau[i] == 0.0f) continue;
        /* T[0:i, i] = -tau_i * V[i:m, 0:i]^T v_i */
        for (int p = 0; p < i; ++p) {
            float s = 0.0f;
            for (int r = i; r < m; ++r) s += qro_vij(V, ldv, r, p) * qro_vij(V, ldv, r, i);
            T[(long)p * ldt + i] = -tau[i] * s;
        }
        /* T[0:i, i] = T[0:i, 0:i] * T[0:i, i]  (upper-triangular matvec, top-down) */
        for (int p = 0; p < i; ++p) {
            float s = 0.0f;
            for (int q = p; q < i; ++q) s += T[(long)p * ldt + q] * T[(long)q * ldt + i];
            T[(long)p * ldt + i] = s;
        }
        T[(long)i * ldt + i] = tau[i];
    }
}

void qro_larfb_lt(int m, int c, int k, const float* V, long ldv,
                  const float* T, long ldt, float* C, long ldc)
{
    float* W = (float*)calloc((size_t)k * (size_t)(c > 0 ? c : 1), sizeof(float));
    float* W2 = (float*)calloc((size_t)k * (size_t)(c > 0 ? c : 1), sizeof(float));
    /* W = V^T C */
    for (int p = 0; p < k; ++p)
        for (int r = p; r < m; ++r) {
            const float v = qro_vij(V, ldv, r, p);
            const float* Cr = C + (long)r * ldc;
            for (int q = 0; q < c; ++q) W[(long)p * c + q] += v * Cr[q];
        }
    /* W2 = T^T W  (T upper => T^T lower) */
    for (int p = 0; p < k; ++p)
        for (int q = 0; q <= p; ++q) {
            const float t = T[(long)q * ldt + p];
            for (int s = 0; s < c; ++s) W2[(long)p * c + s] += t * W[(long)q * c + s];
        }
    /* C -= V W2 */
    for (int r = 0; r < m; ++r) {
        float* Cr = C + (long)r * ldc;
        const int pmax = r < k - 1 ? r : k - 1;
        for (int p = 0; p <= pmax; ++p) {
            const float v = qro_vij(V, ldv, r, p);
            for (int s = 0; s < c; ++s) Cr[s] -= v * W2[(long)p * c + s];
        }
    }
    free(W);
    free(W2);
}

void qro_geqrf(int n, float* A, long lda, float* tau, int nb)
{
    if (nb <= 0 || nb >= n) {
        qro_geqr2(n, n, A, lda, tau);
        return;
    }
    float* T = (float*)malloc(sizeof(float) * (size_t)nb * (size_t)nb);
    for (int j0 = 0; j0 < n; j0 += nb) {
        const int w = (n - j0) < nb ? (n - j0) : nb;
        float* P = A + (long)j0 * lda + j0;
        qro_geqr2(n - j0, w, P, lda, tau + j0);
        const int c = n - j0 - w;
        if (c > 0) {
            qro_larft(n - j0, w, P, lda, tau + j0, T, nb);
            qro_larfb_lt(n - j0, c, w, P, lda, T, nb, P + w, lda);
        }
    }
    free(T);
}

void qro_geqrf_batched(int batch, int n, const float* A, float* H, float* tau, int nb)
{
    const size_t nn = (size_t)n * (size_t)n;
    for (int b = 0; b < batch; ++b) {
        float* Hb = H + (size_t)b * nn;
        if (Hb != A + (size_t)b * nn) memcpy(Hb, A + (size_t)b * nn, nn * sizeof(float));
        qro_geqrf(n, Hb, n, tau + (size_t)b * n, nb);
    }
}

void qro_orgqr(int n, const float* H, const float* tau, float* Q)
{
    /* Q = H_0 ... H_{n-1} I, applied right-to-left (LAPACK sorg2r order). */
    memset(Q, 0, sizeof(float) * (size_t)n * (size_t)n);
    for (int i = 0; i < n; ++i) Q[(long)i * n + i] = 1.0f;
    float* work = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    float* v = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    for (int j = n - 1; j >= 0; --j) {
        v[0] = 1.0f;
        for (int r = j + 1; r < n; ++r) v[r - j] = H[(long)r * n + j];
        /* Q[j:, j:] = H_j Q[j:, j:] */
        qro_larf_left(n - j, n - j, v, 1, tau[j], Q + (long)j * n + j, n, work);
    }
    free(work);
    free(v);
}
