// qr_cholqr.hip -- an outer block of 64 columns factored by CholeskyQR2 with
// Householder reconstruction, on FP32 MFMA, with the Householder panels as the
// per-matrix fallback.
//
// Reference: the blocked loop's panel step (hh_panel_qr, src/qrbench/
// triton_kernels.py:787-909, called from src/qrbench/variants.py:791-799)
// produces (V, tau, T) of each panel by sequential Householder column steps.
// Here the whole block A_b (r x 64) is factored at once:
//   pass 1  G1 = A_b^T A_b (row-chunk partials, MFMA); with D = diag(G1)^1/2,
//           D^-1 G1 D^-1 = R1s^T R1s (Cholesky), R1 = R1s D, M1 = R1^-1;
//   pass 2  X = A_b M1, G2 = X^T X (partials, MFMA); G2 = R2^T R2;
//           R_c = R2 R1, Rinv = M1 R2^-1, Q = A_b Rinv (orthonormal columns);
//   reconstruction (Ballard, Demmel, Grigori, Jacobsen, Knight, Nguyen,
//   "Reconstructing Householder vectors from Tall-Skinny QR", IPDPS 2014):
//           Q[0:64] - S = L1 U with the sign S_k = -sign(pivot) chosen during
//           the LU (no pivoting; |U_kk| >= 1), then
//           V = [L1; A_b[64:] Rinv U^-1], T = -U S L1^-T, R = S R_c.
// S_k = -sign(alpha_k) is exactly slarfg's beta = -sign(alpha) ||.||, so V,
// tau = diag(T) and R are LAPACK sgeqrf's (Householder QR of a block is unique
// given that sign rule). The trailing update only needs the 16 x 16 diagonal
// blocks of T: T_qq = -U_qq S_q L1_qq^-T, the T of panel q alone.
//
// Guard (per matrix and block): every diag(G1) in [1e-30, 1e30], every pivot of
// the scaled Cholesky >= 1e-5, max |G2 - I| <= 1e-2 (so Q is orthonormal to
// working accuracy after pass 2), finite LU pivots, and every column of the
// block nonzero somewhere below its top 64 rows. The last condition keeps out
// exact zeros below a diagonal (upper or block triangular input, a square
// block): slarfg gives tau = 0 (H = I) for such a column, while the
// reconstruction would give the equally valid tau = 2 with R's row negated.
// A matrix that fails any of them gets its flag set and none of its outputs
// written; the panel launches that follow factor exactly those matrices by
// Householder column steps and return at once for the others.
#include "qr_wy.hpp"

namespace qr {

constexpr int kCqB = 64;                 // columns of a block
constexpr int kCqLS = 68;                // LDS row stride of 64 x 64 matrices
constexpr int kCqTiles = 10;             // 16 x 16 tiles on and above the Gram's diagonal
constexpr int kCqPart = kCqTiles * 256;  // floats of a Gram partial's tiles
constexpr int kCqSlot = kCqPart + 4;     // partial slot: tiles, then a 64-bit column mask
constexpr int kCqMat = kCqB * kCqB;      // floats of a 64 x 64 matrix in the workspace
constexpr float kCqGramMin = 1e-30f;
constexpr float kCqGramMax = 1e30f;
constexpr float kCqPivMin = 1e-5f;
constexpr float kCqOrthTol = 1e-2f;
constexpr float kCqSingleMaxF2 = 144.0f;  // ||R1s^-1||_F^2 bound of the one-pass route
// Per-matrix flags of a block: the route with two passes, with one, or the
// Householder panels.
constexpr int kCqFlagTwo = 0;
constexpr int kCqFlagFallback = 1;
constexpr int kCqFlagSingle = 2;

__host__ __device__ constexpr int cq_tile(int I, int J) {
  return I * 4 - I * (I - 1) / 2 + (J - I);
}

// Max over the wave; NaN if any lane holds NaN.
__device__ __forceinline__ float wave_max64(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float u = __shfl_xor(v, o);
    v = (v != v || u != u) ? __builtin_nanf("") : fmaxf(v, u);
  }
  return v;
}

// ---------------------------------------------------------------------------
// Block rows times an upper-triangular 64 x 64 matrix M on MFMA.
//
// M as the B operand of v_mfma_f32_16x16x4_f32 (K step s covers rows 4s..4s+3):
// lane (j, kk) holds M[4s + kk][16J + j]; steps s > 4J + 3 of column tile J
// are zero and skipped (40 of 64). Index of (J, s): 2J(J+1) + s.
__device__ __forceinline__ void cq_load_mb(float (&mr)[40], const float* __restrict__ M,
                                           int lane) {
  const int j = lane & 15, kk = lane >> 4;
#pragma unroll
  for (int J = 0; J < 4; ++J)
#pragma unroll
    for (int s = 0; s <= 4 * J + 3; ++s) mr[2 * J * (J + 1) + s] = M[(4 * s + kk) * kCqB + 16 * J + j];
}

// x[J] = (rows row0..row0+15 of the block) * M, column tile J, in the MFMA
// accumulator layout: lane (k, g), register v holds X[row0 + 4g + v][16J + k].
// Rows >= r read as zero.
__device__ __forceinline__ void cq_tile_times_m(f32x4 (&x)[4], const float* __restrict__ S,
                                                int64_t lds, int row0, int r,
                                                const float (&mr)[40], int lane) {
  const int i = lane & 15, kk = lane >> 4;
  const int row = row0 + i;
  const float* p = S + (int64_t)row * lds + kk;
  float a[16];
#pragma unroll
  for (int s = 0; s < 16; ++s) a[s] = (row < r) ? p[4 * s] : 0.0f;
#pragma unroll
  for (int J = 0; J < 4; ++J) x[J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 16; ++s)
#pragma unroll
    for (int J = 0; J < 4; ++J)
      if (s <= 4 * J + 3)
        x[J] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], mr[2 * J * (J + 1) + s], x[J], 0, 0, 0);
}

// The 64 x 64 Gram of matrix b from its nchunk partials into G (row stride
// kCqLS), upper tiles mirrored. Every element has exactly one writer; the
// chunks are summed in order, 10 tiles x 4 chunks of loads in flight.
// Returns this thread's max |G - I| over its elements (NaN propagates).
__device__ __forceinline__ float cq_sum_gram(float* __restrict__ G, const float* __restrict__ part,
                                             int b, int nchunk) {
  const int e = threadIdx.x;  // 256 threads: element e of every tile
  const int ti = e >> 4, tj = e & 15;
  const float* src = part + (int64_t)b * nchunk * kCqSlot + e;
  float s[kCqTiles];
#pragma unroll
  for (int t = 0; t < kCqTiles; ++t) s[t] = 0.0f;
  for (int c0 = 0; c0 < nchunk; c0 += 4) {
    float v[4][kCqTiles];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int t = 0; t < kCqTiles; ++t)
        v[u][t] = (c0 + u < nchunk) ? src[(int64_t)(c0 + u) * kCqSlot + t * 256] : 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int t = 0; t < kCqTiles; ++t) s[t] += v[u][t];
  }
  float dev = 0.0f;
#pragma unroll
  for (int I = 0; I < 4; ++I)
#pragma unroll
    for (int J = I; J < 4; ++J) {
      const float sv = s[cq_tile(I, J)];
      G[(16 * I + ti) * kCqLS + 16 * J + tj] = sv;
      if (I != J) G[(16 * J + tj) * kCqLS + 16 * I + ti] = sv;
      const float d = fabsf(sv - ((I == J && ti == tj) ? 1.0f : 0.0f));
      dev = (d <= dev) ? dev : d;
    }
  return dev;
}

// ---------------------------------------------------------------------------
// 16 x 16 routines for one DPP row (16 lanes): lane c = lane & 15 holds column
// c of the block in x[0..15]. Every cross-lane value is a DPP row_newbcast of
// the row's own lane, so the four rows of a wave could run four blocks; the
// blocked 64 x 64 routines below use row 0's results.

// Upper Cholesky G = R^T R (only the upper triangle of G is read). On return
// x[i] = R[i][c] (zero below the diagonal), my_dinv = 1 / R[c][c] and my_piv =
// the pivot R[c][c]^2 (NaN or out of range if the factorisation broke down).
__device__ __forceinline__ void cq_chol16(float (&x)[16], float& my_dinv, float& my_piv, int c) {
  static_for<0, 16>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const float piv = row_bcast16<k>(x[k]);
    const float pv = (piv >= 1e-30f && piv <= 3.0e38f) ? piv : 1.0f;
    const float rs = __builtin_amdgcn_sqrtf(pv);  // 1 ulp
    const float ri = __builtin_amdgcn_rcpf(rs);   // 1 ulp
    const float rkc = (c > k) ? x[k] * ri : ((c == k) ? rs : 0.0f);
    x[k] = rkc;
    if (c == k) {
      my_dinv = ri;
      my_piv = piv;
    }
    const float nr = -rkc;
    static_for<k + 1, 16>([&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value;
      x[i] = fmaf(row_bcast16<i>(rkc), nr, x[i]);  // G[i][c] -= R[k][i] R[k][c]
    });
  });
}

// m = column c of R^-1 for upper R (x[i] = R[i][c], lane c holding my_dinv =
// 1 / R[c][c]); back substitution from the last row.
__device__ __forceinline__ void cq_inv16_upper(float (&m)[16], const float (&x)[16],
                                               float my_dinv, int c) {
  static_for<0, 16>([&](auto tc) __attribute__((always_inline)) {
    constexpr int i = 15 - decltype(tc)::value;
    float s = (c == i) ? 1.0f : 0.0f;
    static_for<i + 1, 16>([&](auto qc) __attribute__((always_inline)) {
      constexpr int q = decltype(qc)::value;
      s = fmaf(-row_bcast16<q>(x[i]), m[q], s);  // R[i][q] m[q]
    });
    m[i] = s * row_bcast16<i>(my_dinv);
  });
}

// y = column c of L^-1 for unit lower L (x[i] = L[i][c]); forward substitution.
__device__ __forceinline__ void cq_inv16_unit_lower(float (&y)[16], const float (&x)[16], int c) {
  static_for<0, 16>([&](auto ic) __attribute__((always_inline)) {
    constexpr int i = decltype(ic)::value;
    float s = (c == i) ? 1.0f : 0.0f;
    static_for<0, i>([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      s = fmaf(-row_bcast16<k>(x[i]), y[k], s);  // L[i][k] y[k]
    });
    y[i] = s;
  });
}

// A - S = L U without pivoting; S_k = -1 if the k-th pivot candidate is >= 0,
// else +1, so |U_kk| = |candidate| + 1 >= 1. On return x[i] = U[i][c] for
// i <= c and L[i][c] for i > c; my_sgn = S_c, my_pinv = 1 / U[c][c].
__device__ __forceinline__ void cq_lu16(float (&x)[16], float& my_sgn, float& my_pinv, int c) {
  static_for<0, 16>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const float q = row_bcast16<k>(x[k]);
    const float s = (q >= 0.0f) ? -1.0f : 1.0f;
    const float pv = q - s;
    const float pinv = __builtin_amdgcn_rcpf(pv);  // 1 ulp; |pv| >= 1
    if (c == k) {
      x[k] = pv;
      my_sgn = s;
      my_pinv = pinv;
    }
    // A[i][c] -= L[i][k] U[k][c], L[i][k] = A[i][k] / pv: column k is scaled
    // only at the end, so its lane keeps A[i][k] for the broadcasts.
    const float wc = (c > k) ? -(x[k] * pinv) : 0.0f;
    static_for<k + 1, 16>([&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value;
      x[i] = fmaf(row_bcast16<k>(x[i]), wc, x[i]);
    });
  });
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (i > c) x[i] *= my_pinv;
}

// ---------------------------------------------------------------------------
// 16 x 16 tiles of 64 x 64 LDS matrices (row stride kCqLS) on MFMA.

// acc += sx opX(X) opY(Y); kXT / kYT transpose the tile.
template <bool kXT, bool kYT>
__device__ __forceinline__ void cq_mm16(f32x4& acc, const float* __restrict__ X,
                                        const float* __restrict__ Y, float sx, int lane) {
  const int i = lane & 15, kk = lane >> 4;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int q = 4 * s + kk;
    const float a = (kXT ? X[q * kCqLS + i] : X[i * kCqLS + q]) * sx;
    const float b = kYT ? Y[i * kCqLS + q] : Y[q * kCqLS + i];
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
  }
}

__device__ __forceinline__ f32x4 cq_load_tile(const float* __restrict__ Z, int lane) {
  const int k = lane & 15, g = lane >> 4;
  f32x4 t;
#pragma unroll
  for (int v = 0; v < 4; ++v) t[v] = Z[(4 * g + v) * kCqLS + k];
  return t;
}

__device__ __forceinline__ void cq_store_tile(float* __restrict__ Z, const f32x4& t, int lane) {
  const int k = lane & 15, g = lane >> 4;
#pragma unroll
  for (int v = 0; v < 4; ++v) Z[(4 * g + v) * kCqLS + k] = t[v];
}

__device__ __forceinline__ float* cq_tile_ptr(float* M, int I, int J) {
  return M + 16 * I * kCqLS + 16 * J;
}

// Off-diagonal 16 x 16 blocks of Ri = U^-1 for block upper-triangular U (LDS)
// whose diagonal blocks' inverses are already in Ri: by distance d = J - K,
// Ri_KJ = -Ri_KK sum_{L=K+1..J} U_KL Ri_LJ. The sum's accumulator layout is the
// B operand of the last product with K order {v, v+4, v+8, v+12}. Lower blocks
// of Ri are set to zero. All threads; ends with a barrier.
__device__ __forceinline__ void cq_inv_offdiag(const float* __restrict__ U, float* __restrict__ Ri,
                                               int w, int lane) {
  const int i = lane & 15, kk = lane >> 4;
  for (int d = 1; d <= 3; ++d) {
    if (w < 4 - d) {
      const int K = w, J = w + d;
      f32x4 p = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int L = K + 1; L <= J; ++L)
        cq_mm16<false, false>(p, cq_tile_ptr(const_cast<float*>(U), K, L), cq_tile_ptr(Ri, L, J),
                              1.0f, lane);
      const float* D = cq_tile_ptr(Ri, K, K);
      f32x4 r = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int v = 0; v < 4; ++v)
        r = __builtin_amdgcn_mfma_f32_16x16x4f32(-D[i * kCqLS + 4 * kk + v], p[v], r, 0, 0, 0);
      cq_store_tile(cq_tile_ptr(Ri, K, J), r, lane);
    }
    __syncthreads();
  }
#pragma unroll
  for (int it = 0; it < 6; ++it) {
    const int e = threadIdx.x + 256 * it;  // tiles (I, J), I > J
    const int t = e >> 8, el = e & 255;
    const int I = t < 3 ? t + 1 : (t < 5 ? t - 1 : 3), J = t < 3 ? 0 : (t < 5 ? 1 : 2);
    Ri[(16 * I + (el >> 4)) * kCqLS + 16 * J + (el & 15)] = 0.0f;
  }
  __syncthreads();
}

// Blocked upper Cholesky of the 64 x 64 SPD matrix in G (upper triangle read),
// in place: G := R (zero below the diagonal), Ri := R^-1, piv[j] = the j-th
// pivot. All threads (four waves); ends with a barrier.
__device__ __forceinline__ void cq_chol_inv_blocked(float* __restrict__ G, float* __restrict__ Ri,
                                                    float* __restrict__ piv, int w, int lane) {
  const int c = lane & 15, g = lane >> 4;
  for (int K = 0; K < 4; ++K) {
    if (w == 0) {
      float* Gd = cq_tile_ptr(G, K, K);
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = Gd[i * kCqLS + c];
      float dv = 1.0f, pv = 0.0f;
      cq_chol16(x, dv, pv, c);
      float m[16];
      cq_inv16_upper(m, x, dv, c);
      if (g == 0) {
        float* Rd = cq_tile_ptr(Ri, K, K);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          Gd[i * kCqLS + c] = x[i];
          Rd[i * kCqLS + c] = m[i];
        }
        piv[16 * K + c] = pv;
      }
    }
    __syncthreads();
    if (w < 3 - K) {  // R_KJ = R_KK^-T G_KJ
      const int J = K + 1 + w;
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      cq_mm16<true, false>(acc, cq_tile_ptr(Ri, K, K), cq_tile_ptr(G, K, J), 1.0f, lane);
      cq_store_tile(cq_tile_ptr(G, K, J), acc, lane);
    }
    __syncthreads();
    int t = 0;  // G_IJ -= R_KI^T R_KJ, K < I <= J
    for (int I = K + 1; I < 4; ++I)
      for (int J = I; J < 4; ++J, ++t) {
        if ((t & 3) != w) continue;
        f32x4 acc = cq_load_tile(cq_tile_ptr(G, I, J), lane);
        cq_mm16<true, false>(acc, cq_tile_ptr(G, K, I), cq_tile_ptr(G, K, J), -1.0f, lane);
        cq_store_tile(cq_tile_ptr(G, I, J), acc, lane);
      }
    __syncthreads();
  }
#pragma unroll
  for (int it = 0; it < 6; ++it) {
    const int e = threadIdx.x + 256 * it;  // lower blocks of R
    const int t = e >> 8, el = e & 255;
    const int I = t < 3 ? t + 1 : (t < 5 ? t - 1 : 3), J = t < 3 ? 0 : (t < 5 ? 1 : 2);
    G[(16 * I + (el >> 4)) * kCqLS + 16 * J + (el & 15)] = 0.0f;
  }
  cq_inv_offdiag(G, Ri, w, lane);
}

// Blocked signed LU of the 64 x 64 matrix in A, in place: A := L\U (L unit
// lower strictly below the diagonal, U on and above it), Ui := U^-1, Li[K] :=
// L_KK^-1 (16 x 16 tiles, row stride kCqLS), sgn[j] = S_j, pinv[j] = 1 / U_jj.
// All threads (four waves); ends with a barrier.
__device__ __forceinline__ void cq_lu_blocked(float* __restrict__ A, float* __restrict__ Ui,
                                              float* __restrict__ Li, float* __restrict__ sgn,
                                              float* __restrict__ pinv, int w, int lane) {
  const int c = lane & 15, g = lane >> 4;
  for (int K = 0; K < 4; ++K) {
    float* Ad = cq_tile_ptr(A, K, K);
    if (w == 0) {
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = Ad[i * kCqLS + c];
      float sv = 1.0f, pi = 1.0f;
      cq_lu16(x, sv, pi, c);
      if (g == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) Ad[i * kCqLS + c] = x[i];
        sgn[16 * K + c] = sv;
        pinv[16 * K + c] = pi;
      }
    }
    __syncthreads();
    // The two triangular inverses of the diagonal block at once: U_KK^-1 in
    // wave 0, L_KK^-1 in wave 1.
    if (w < 2) {
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = Ad[i * kCqLS + c];
      float m[16];
      if (w == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = (i <= c) ? x[i] : 0.0f;
        cq_inv16_upper(m, x, pinv[16 * K + c], c);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = (i > c) ? x[i] : ((i == c) ? 1.0f : 0.0f);
        cq_inv16_unit_lower(m, x, c);
      }
      if (g == 0) {
        float* D = (w == 0) ? cq_tile_ptr(Ui, K, K) : Li + 16 * K * kCqLS;
#pragma unroll
        for (int i = 0; i < 16; ++i) D[i * kCqLS + c] = m[i];
      }
    }
    __syncthreads();
    // U_KJ = L_KK^-1 A_KJ (J > K) and L_IK = A_IK U_KK^-1 (I > K).
    for (int t = w; t < 2 * (3 - K); t += 4) {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      if (t < 3 - K) {
        const int J = K + 1 + t;
        cq_mm16<false, false>(acc, Li + 16 * K * kCqLS, cq_tile_ptr(A, K, J), 1.0f, lane);
        cq_store_tile(cq_tile_ptr(A, K, J), acc, lane);
      } else {
        const int I = K + 1 + t - (3 - K);
        cq_mm16<false, false>(acc, cq_tile_ptr(A, I, K), cq_tile_ptr(Ui, K, K), 1.0f, lane);
        cq_store_tile(cq_tile_ptr(A, I, K), acc, lane);
      }
    }
    __syncthreads();
    int t = 0;  // A_IJ -= L_IK U_KJ, I, J > K
    for (int I = K + 1; I < 4; ++I)
      for (int J = K + 1; J < 4; ++J, ++t) {
        if ((t & 3) != w) continue;
        f32x4 acc = cq_load_tile(cq_tile_ptr(A, I, J), lane);
        cq_mm16<false, false>(acc, cq_tile_ptr(A, I, K), cq_tile_ptr(A, K, J), -1.0f, lane);
        cq_store_tile(cq_tile_ptr(A, I, J), acc, lane);
      }
    __syncthreads();
  }
  cq_inv_offdiag(A, Ui, w, lane);
}

// Z rows 16w..16w+15 = X Y for 64 x 64 LDS matrices (row stride kCqLS), in the
// accumulator layout (lane (k, g), register v: Z[16w + 4g + v][16J + k]).
// kXUpper / kYUpper skip K steps whose operand block is known to be zero.
template <bool kXUpper, bool kYUpper>
__device__ __forceinline__ void cq_mm64(f32x4 (&acc)[4], const float* __restrict__ X,
                                        const float* __restrict__ Y, int w, int lane) {
  const int i = lane & 15, kk = lane >> 4;
#pragma unroll
  for (int J = 0; J < 4; ++J) acc[J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    if (kXUpper && 4 * s + 3 < 16 * w) continue;  // X[16w + i][4s + kk] == 0
    const float av = X[(16 * w + i) * kCqLS + 4 * s + kk];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      if (kYUpper && s > 4 * J + 3) continue;  // Y[4s + kk][16J + j] == 0
      const float bv = Y[(4 * s + kk) * kCqLS + 16 * J + i];
      acc[J] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[J], 0, 0, 0);
    }
  }
}

__device__ __forceinline__ void cq_store_rows(float* __restrict__ Z, int64_t ldz,
                                              const f32x4 (&acc)[4], int w, int lane) {
  const int k = lane & 15, g = lane >> 4;
#pragma unroll
  for (int J = 0; J < 4; ++J)
#pragma unroll
    for (int v = 0; v < 4; ++v) Z[(int64_t)(16 * w + 4 * g + v) * ldz + 16 * J + k] = acc[J][v];
}

// ---------------------------------------------------------------------------
// Pass 1 per matrix: scaled Cholesky of G1, guard, M1 = R1^-1 and R1 into the
// workspace (mats[b]: M1 at 0, R1 at kCqMat), flag[b] = kCqFlagTwo,
// kCqFlagSingle (one pass is enough; only with allow_single >= 1) or
// kCqFlagFallback (also, with allow_single = 2, a matrix that would need the
// second pass).
constexpr int kCqChol1Lds = 2 * kCqB * kCqLS + 4 * 64 + 16;  // floats
__device__ __forceinline__ void cq_chol1_body(float* __restrict__ smem, int b,
                                              const float* __restrict__ part, int nchunk,
                                              float* __restrict__ mats, int64_t sMb,
                                              int* __restrict__ flags, int allow_single) {
  float* const G = smem;
  float* const Ri = G + kCqB * kCqLS;
  float* const piv = Ri + kCqB * kCqLS;
  float* const dsc = piv + 64;   // d_j = sqrt(G1_jj)
  float* const rdsc = dsc + 64;  // 1 / d_j
  int* const dbad = reinterpret_cast<int*>(rdsc + 64);
  float* const ssw = rdsc + 68;  // per-wave sums of squares of R1s^-1
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  cq_sum_gram(G, part, b, nchunk);
  if (threadIdx.x == 0) *dbad = 0;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int j = threadIdx.x;
    const float gjj = G[j * kCqLS + j];
    const bool dok = gjj >= kCqGramMin && gjj <= kCqGramMax;
    const float dj = __builtin_amdgcn_sqrtf(dok ? gjj : 1.0f);
    dsc[j] = dj;
    rdsc[j] = __builtin_amdgcn_rcpf(dj);
    if (!dok) *dbad = 1;
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < kCqMat / 256; ++it) {
    const int e = threadIdx.x + 256 * it;  // D^-1 G1 D^-1
    const int i = e >> 6, c = e & 63;
    G[i * kCqLS + c] *= rdsc[i] * rdsc[c];
  }
  __syncthreads();
  cq_chol_inv_blocked(G, Ri, piv, w, lane);
  float* M1 = mats + (int64_t)b * sMb;
  float* R1 = M1 + kCqMat;
  // R1 = R1s D, M1 = R1^-1 = D^-1 R1s^-1.
  float ss = 0.0f;
#pragma unroll
  for (int it = 0; it < kCqMat / 256; ++it) {
    const int e = threadIdx.x + 256 * it;
    const int i = e >> 6, c = e & 63;
    const float ri = Ri[i * kCqLS + c];
    R1[e] = G[i * kCqLS + c] * dsc[c];
    M1[e] = ri * rdsc[i];
    ss = fmaf(ri, ri, ss);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) ss += __shfl_xor(ss, o);
  if (lane == 0) ssw[w] = ss;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int j = threadIdx.x;
    unsigned long long nzm = 0;
    for (int c = 0; c < nchunk; ++c)
      nzm |= *reinterpret_cast<const unsigned long long*>(
          part + ((int64_t)b * nchunk + c) * kCqSlot + kCqPart);
    const bool ok = __all(piv[j] >= kCqPivMin && piv[j] <= 3.0e38f) && *dbad == 0 &&
                    nzm == ~0ull;
    // One pass is enough when ||R1s^-1||_F^2 <= 144. With unit columns
    // sum(sigma_i^2) = ||R1s||_F^2 = 64, so sum(sigma_i^-2) <= 144 caps
    // kappa_2(R1s) at 34.0 (sigma_max^2 = 22.7, sigma_min^2 = 1/51, the other
    // 62 at 2/3). Q1 = A_b M1 is then orthonormal to about kappa^2 u, and the
    // (V, tau, R) built from it differ from LAPACK sgeqrf's by at most 8e-6 at
    // kappa = 37 and 4e-5 at kappa = 92 in a numpy model of these steps (r =
    // 128; 2.7e-6 and 1.3e-5 at r = 1024), under the parity tolerance 4 r eps32
    // (6.1e-5 at r = 128).
    const float ssum = (ssw[0] + ssw[1]) + (ssw[2] + ssw[3]);
    const bool single = allow_single != 0 && ssum <= kCqSingleMaxF2;
    const bool two_ok = allow_single != 2;
    if (j == 0)
      flags[b] = ok ? (single ? kCqFlagSingle : (two_ok ? kCqFlagTwo : kCqFlagFallback))
                    : kCqFlagFallback;
  }
}

// ---------------------------------------------------------------------------
// Pass 2 per matrix and the reconstruction: R2, Rinv = M1 R2^-1, R_c = R2 R1,
// Q_top = A_b[0:64] Rinv, the signed LU of Q_top, M = Rinv U^-1 (for the rows
// below, k_cq_form), T_qq, tau and the block's top 64 rows of H (R = S R_c on
// and above the diagonal, L1 below). Nothing is written for a matrix whose
// flag is or becomes set.
constexpr int kCqReconLds = 8 * kCqB * kCqLS + 4 * 64 + 8;  // floats (139 KB)
__device__ __forceinline__ void cq_recon_body(float* __restrict__ smem, int b,
                                              const float* __restrict__ part, int nchunk,
                                              float* __restrict__ mats, int64_t sMb,
                                              int* __restrict__ flags,
                                              const float* __restrict__ Src, int64_t sSb,
                                              int64_t lds, float* __restrict__ Hb, int64_t sHb,
                                              int64_t ldh, float* __restrict__ tau,
                                              int64_t sTaub, float* __restrict__ Tws,
                                              int64_t sTwb) {
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int kM = kCqB * kCqLS;
  float* const G2 = smem;         // G2, then R2
  float* const M1l = smem + kM;   // M1
  float* const R1l = smem + 2 * kM;  // R1
  float* const At = smem + 3 * kM;   // A_b[0:64], then Q_top, then L\U
  float* const R2i = smem + 4 * kM;  // R2^-1, then U^-1
  float* const Rinv = smem + 5 * kM;  // M1 R2^-1
  float* const Rc = smem + 6 * kM;    // R2 R1
  float* const Li = smem + 7 * kM;    // L_KK^-1 at rows 16K.., columns 0..15
  float* const piv = smem + 8 * kM;
  float* const sgn = piv + 64;
  float* const pinv = sgn + 64;
  float* const devw = pinv + 64;
  int* const okflagp = reinterpret_cast<int*>(devw + 4);
  int& okflag = *okflagp;
  const float* M1g = mats + (int64_t)b * sMb;
  const float* S = Src + (int64_t)b * sSb;
  const bool single = flags[b] == kCqFlagSingle;  // no second pass: R2 = I

  if (!single) {
    const float dev = wave_max64(cq_sum_gram(G2, part, b, nchunk));  // max |G2 - I|
    if (lane == 0) devw[w] = dev;
  }
#pragma unroll
  for (int it = 0; it < kCqMat / 256; ++it) {
    const int e = threadIdx.x + 256 * it;
    const int i = e >> 6, c = e & 63;
    M1l[i * kCqLS + c] = M1g[e];
    R1l[i * kCqLS + c] = M1g[kCqMat + e];
    At[i * kCqLS + c] = S[(int64_t)i * lds + c];
  }
  __syncthreads();
  if (single) {
    if (threadIdx.x == 0) okflag = 1;
  } else {
    cq_chol_inv_blocked(G2, R2i, piv, w, lane);
    if (threadIdx.x < 64) {
      // Every devw[u] <= tol (false for NaN).
      const bool dok = devw[0] <= kCqOrthTol && devw[1] <= kCqOrthTol &&
                       devw[2] <= kCqOrthTol && devw[3] <= kCqOrthTol;
      const bool ok = __all(piv[threadIdx.x] >= 0.25f && piv[threadIdx.x] <= 4.0f) && dok;
      if (threadIdx.x == 0) okflag = ok ? 1 : 0;
    }
  }
  __syncthreads();
  if (!okflag) {
    if (threadIdx.x == 0) flags[b] = kCqFlagFallback;
    return;
  }
  // With one pass R2 = I: Rinv = M1 and R_c = R1, already in LDS (and not
  // overwritten below).
  const float* const RinvP = single ? M1l : Rinv;
  const float* const RcP = single ? R1l : Rc;
  if (!single) {
    f32x4 acc[4];
    cq_mm64<true, true>(acc, M1l, R2i, w, lane);
    cq_store_rows(Rinv, kCqLS, acc, w, lane);
    cq_mm64<true, true>(acc, G2, R1l, w, lane);
    cq_store_rows(Rc, kCqLS, acc, w, lane);
    __syncthreads();
  }
  {
    f32x4 acc[4];
    cq_mm64<false, true>(acc, At, RinvP, w, lane);
    cq_store_rows(At, kCqLS, acc, w, lane);  // Q_top (each wave its own rows)
  }
  __syncthreads();
  cq_lu_blocked(At, R2i, Li, sgn, pinv, w, lane);
  if (threadIdx.x < 64) {
    const float p = pinv[threadIdx.x];
    const bool ok = __all(fabsf(p) <= 1.0f && fabsf(p) >= 1e-30f);
    if (threadIdx.x == 0) okflag = ok ? 1 : 0;
  }
  __syncthreads();
  if (!okflag) {
    if (threadIdx.x == 0) flags[b] = kCqFlagFallback;
    return;
  }
  // M = Rinv U^-1 for the rows below the top block.
  {
    f32x4 acc[4];
    cq_mm64<true, true>(acc, RinvP, R2i, w, lane);
    cq_store_rows(mats + (int64_t)b * sMb + 2 * kCqMat, kCqB, acc, w, lane);
  }
  // T_qq = -U_qq S_q (L_qq^-1)^T for panel q = w: A operand U[i][q'] S[q'] (upper
  // part of the packed diagonal block), B operand (L_qq^-1)^T.
  {
    const int q = w, i = lane & 15, kk = lane >> 4, k = lane & 15, g = lane >> 4;
    const float* Ad = cq_tile_ptr(At, q, q);
    const float* Ld = Li + 16 * q * kCqLS;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int qq = 4 * s + kk;
      const float a = (qq >= i) ? Ad[i * kCqLS + qq] * sgn[16 * q + qq] : 0.0f;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, Ld[i * kCqLS + qq], acc, 0, 0, 0);
    }
    float* Tq = Tws + (int64_t)b * sTwb + 256 * q;
#pragma unroll
    for (int v = 0; v < 4; ++v) Tq[(4 * g + v) * 16 + k] = -acc[v];
  }
  // H's top 64 rows of the block: R = S R_c on and above the diagonal, L1 below.
  float* Hm = Hb + (int64_t)b * sHb;
#pragma unroll
  for (int it = 0; it < kCqMat / 256; ++it) {
    const int e = threadIdx.x + 256 * it;
    const int i = e >> 6, c = e & 63;
    Hm[(int64_t)i * ldh + c] = (i <= c) ? sgn[i] * RcP[i * kCqLS + c] : At[i * kCqLS + c];
  }
  if (threadIdx.x < 64) {
    const int i = threadIdx.x;
    tau[(int64_t)b * sTaub + i] = -At[i * kCqLS + i] * sgn[i];
  }
}

// ---------------------------------------------------------------------------
// Gram partials, fused with the per-matrix step. Workgroup (b, c) sums X^T X
// over rows [c rc, (c+1) rc) of the block (X = A_b in pass 1, A_b M1 in pass
// 2) and writes the 10 upper 16 x 16 tiles, each row-major, to
// part[(b nchunk + c) kCqSlot]; pass 1 also writes, after the tiles, the mask
// of columns with a nonzero entry in rows >= 64 of the chunk. The last of
// matrix b's nchunk workgroups to finish (counted in cnt[b], which it resets
// to zero) then runs the per-matrix step: cq_chol1_body in pass 1,
// cq_recon_body in pass 2. Partials are summed in chunk order, so the result
// does not depend on which workgroup is last. kCqGramWaves(kFused) waves,
// rc / waves rows each (four when fused: the per-matrix bodies use 256 threads).
__host__ __device__ constexpr int kCqGramWaves(bool fused) { return fused ? 4 : 8; }
template <bool kPass2, bool kFused>
__global__ __launch_bounds__(64 * kCqGramWaves(kFused)) void k_cq_gram(const float* __restrict__ Src, int64_t sSb,
                                                 int64_t lds, int r, int rc, int nchunk,
                                                 float* __restrict__ mats, int64_t sMb,
                                                 float* __restrict__ part,
                                                 int* __restrict__ flags, int* __restrict__ cnt,
                                                 float* __restrict__ Hb, int64_t sHb, int64_t ldh,
                                                 float* __restrict__ tau, int64_t sTaub,
                                                 float* __restrict__ Tws, int64_t sTwb) {
  constexpr int kNW = kCqGramWaves(kFused);
  constexpr int kRed = kNW * kCqPart + 2 * kNW;
  constexpr int kLds = !kFused ? kRed
                               : (kPass2 ? kCqReconLds : (kCqChol1Lds > kRed ? kCqChol1Lds : kRed));
  __shared__ __attribute__((aligned(16))) float smem[kLds];
  float (*red)[kCqPart] = reinterpret_cast<float (*)[kCqPart]>(smem);
  unsigned long long* wmask = reinterpret_cast<unsigned long long*>(smem + kNW * kCqPart);
  __shared__ int last;
  const int b = blockIdx.x / nchunk;
  const int c = blockIdx.x - b * nchunk;
  if (kPass2 && flags[b] != kCqFlagTwo) return;  // fallback, or one pass is enough
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int k = lane & 15, g = lane >> 4;
  const float* S = Src + (int64_t)b * sSb;

  f32x4 acc[kCqTiles];
#pragma unroll
  for (int t = 0; t < kCqTiles; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float mr[40];
  if constexpr (kPass2) cq_load_mb(mr, mats + (int64_t)b * sMb, lane);

  const int rw = rc / kNW;
  const int rbeg = c * rc + w * rw;
  bool nz[4] = {false, false, false, false};  // pass 1: column 16I + k nonzero below row 64
  for (int t = 0; t < rw; t += 16) {
    const int row0 = rbeg + t;
    if (row0 >= r) break;
    f32x4 x[4];
    if constexpr (kPass2) {
      cq_tile_times_m(x, S, lds, row0, r, mr, lane);
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = row0 + 4 * g + v;
        const float* p = S + (int64_t)row * lds + k;
#pragma unroll
        for (int I = 0; I < 4; ++I) {
          x[I][v] = (row < r) ? p[16 * I] : 0.0f;
          nz[I] = nz[I] || (row >= kCqB && x[I][v] != 0.0f);
        }
      }
    }
    // G_IJ += X_I^T X_J: the accumulator layout with K order {v, v+4, v+8,
    // v+12} is the A and the B operand layout at once.
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int I = 0; I < 4; ++I)
#pragma unroll
        for (int J = I; J < 4; ++J)
          acc[cq_tile(I, J)] =
              __builtin_amdgcn_mfma_f32_16x16x4f32(x[I][v], x[J][v], acc[cq_tile(I, J)], 0, 0, 0);
  }
#pragma unroll
  for (int t = 0; t < kCqTiles; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[w][t * 256 + (4 * g + v) * 16 + k] = acc[t][v];
  if constexpr (!kPass2) {
    // Lane 16 g' + k of the ballot for tile I: column 16 I + k, rows 4 g' + v.
    unsigned long long m = 0;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      unsigned long long bl = __ballot(nz[I]);
      bl |= bl >> 32;
      bl |= bl >> 16;
      m |= (bl & 0xFFFFull) << (16 * I);
    }
    if (lane == 0) wmask[w] = m;
  }
  __syncthreads();
  float* dst = part + (int64_t)blockIdx.x * kCqSlot;
  for (int e = threadIdx.x; e < kCqPart; e += 64 * kNW) {
    float sum = (red[0][e] + red[1][e]) + (red[2][e] + red[3][e]);
    if constexpr (kNW == 8) sum += (red[4][e] + red[5][e]) + (red[6][e] + red[7][e]);
    dst[e] = sum;
  }
  if (!kPass2 && threadIdx.x == 0) {
    unsigned long long m = 0;
#pragma unroll
    for (int u = 0; u < kNW; ++u) m |= wmask[u];
    *reinterpret_cast<unsigned long long*>(dst + kCqPart) = m;
  }
  if constexpr (!kFused) return;
  // Publish the partial, count it; the last workgroup of matrix b goes on.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) last = (atomicAdd(&cnt[b], 1) == nchunk - 1) ? 1 : 0;
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (threadIdx.x == 0) cnt[b] = 0;
  if constexpr (kPass2)
    cq_recon_body(smem, b, part, nchunk, mats, sMb, flags, Src, sSb, lds, Hb, sHb, ldh, tau,
                  sTaub, Tws, sTwb);
  else
    cq_chol1_body(smem, b, part, nchunk, mats, sMb, flags, 0);  // two passes
}

// The per-matrix steps as kernels of their own (one workgroup per matrix),
// after Gram kernels launched without kFused.
__global__ __launch_bounds__(256) void k_cq_chol1(const float* __restrict__ part, int nchunk,
                                                  float* __restrict__ mats, int64_t sMb,
                                                  int* __restrict__ flags, int allow_single) {
  __shared__ __attribute__((aligned(16))) float smem[kCqChol1Lds + 8];
  cq_chol1_body(smem, blockIdx.x, part, nchunk, mats, sMb, flags, allow_single);
}

__global__ __launch_bounds__(256) void k_cq_recon(const float* __restrict__ part, int nchunk,
                                                  float* __restrict__ mats, int64_t sMb,
                                                  int* __restrict__ flags,
                                                  const float* __restrict__ Src, int64_t sSb,
                                                  int64_t lds, float* __restrict__ Hb,
                                                  int64_t sHb, int64_t ldh,
                                                  float* __restrict__ tau, int64_t sTaub,
                                                  float* __restrict__ Tws, int64_t sTwb) {
  __shared__ __attribute__((aligned(16))) float smem[kCqReconLds];
  if (flags[blockIdx.x] == kCqFlagFallback) return;
  cq_recon_body(smem, blockIdx.x, part, nchunk, mats, sMb, flags, Src, sSb, lds, Hb, sHb, ldh,
                tau, sTaub, Tws, sTwb);
}

// ---------------------------------------------------------------------------
// V below the top block: H rows 64 + [c rc, (c+1) rc) of the block = A_b M.
__global__ __launch_bounds__(256) void k_cq_form(const float* __restrict__ Src, int64_t sSb,
                                                 int64_t lds, float* __restrict__ Hb,
                                                 int64_t sHb, int64_t ldh, int r, int rc,
                                                 int nchunk, const float* __restrict__ mats,
                                                 int64_t sMb, const int* __restrict__ flags) {
  const int b = blockIdx.x / nchunk;
  const int c = blockIdx.x - b * nchunk;
  if (flags[b] == kCqFlagFallback) return;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int k = lane & 15, g = lane >> 4;
  const float* S = Src + (int64_t)b * sSb;
  float* Hm = Hb + (int64_t)b * sHb;
  float mr[40];
  cq_load_mb(mr, mats + (int64_t)b * sMb + 2 * kCqMat, lane);
  const int rw = rc >> 2;
  const int rbeg = kCqB + c * rc + w * rw;
  for (int t = 0; t < rw; t += 16) {
    const int row0 = rbeg + t;
    if (row0 >= r) break;
    f32x4 x[4];
    cq_tile_times_m(x, S, lds, row0, r, mr, lane);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = row0 + 4 * g + v;
      if (row < r) {
        float* dst = Hm + (int64_t)row * ldh + k;
#pragma unroll
        for (int J = 0; J < 4; ++J) dst[16 * J] = x[J][v];
      }
    }
  }
}

// Rows per chunk (a multiple of unit) and chunk count for `rows` rows: about
// 256 workgroups over the batch, at most max_chunks per matrix.
void cq_chunks(int rows, int batch, int max_chunks, int unit, int* rc, int* nchunk) {
  int nc = (256 + batch - 1) / batch;
  if (nc > max_chunks) nc = max_chunks;
  if (nc < 1) nc = 1;
  int c = ((rows + nc - 1) / nc + unit - 1) / unit * unit;
  if (c < unit) c = unit;
  *rc = c;
  *nchunk = (rows + c - 1) / c;
}

constexpr int kCqMaxChunks = 16;

// Fused Gram + per-matrix kernels (the last workgroup of a matrix finishes it)
// save two launches per block but measured slower at every shape tried (b2
// n4096 9.48 vs 9.19 ms, b16 n2048 7.07 vs 5.69 ms): the fused pass-2 kernel's
// 137 KB of LDS per workgroup keeps its workgroups off the CUs that the
// concurrent trailing update holds. The caller selects them (`fused`); the
// default options do not.

// Workspace floats of the CholeskyQR2 route for `batch` matrices: Gram
// partials, three 64 x 64 matrices per matrix, flags.
size_t cq_workspace_floats(int batch) {
  int nc = (256 + batch - 1) / batch;
  if (nc > kCqMaxChunks) nc = kCqMaxChunks;
  return (size_t)batch * nc * kCqSlot + (size_t)batch * 3 * kCqMat + 2 * (size_t)batch;
}

// The launches of one block: Gram 1, pass 1, Gram 2, pass 2 (each pair one
// launch when fused), then V. Src / Hb point at the block's top-left
// element of matrix 0; ws holds cq_workspace_floats(batch) floats.
hipError_t launch_cq_block(const float* Src, int64_t sSb, int64_t lds, float* Hb, int64_t sHb,
                           int64_t ldh, int r, float* tau, int64_t sTaub, float* Tws,
                           int64_t sTwb, float* ws, int batch, bool fused, int one_pass,
                           hipStream_t stream) {
  if (r <= kCqB || r > kMaxStripRows || batch < 1) return hipErrorInvalidValue;
  const int gw = kCqGramWaves(fused);
  int rc = 0, nc = 0;
  cq_chunks(r, batch, kCqMaxChunks, 16 * gw, &rc, &nc);
  int ncw = (256 + batch - 1) / batch;
  if (ncw > kCqMaxChunks) ncw = kCqMaxChunks;
  if (nc > ncw) return hipErrorInvalidValue;  // partials sized for ncw chunks
  float* part = ws;
  float* mats = part + (size_t)batch * ncw * kCqSlot;
  int* flags = reinterpret_cast<int*>(mats + (size_t)batch * 3 * kCqMat);
  int* cnt = flags + batch;
  const int64_t sMb = 3 * kCqMat;
  const unsigned g1 = (unsigned)(nc * batch);
  if (fused) {
    hipLaunchKernelGGL((k_cq_gram<false, true>), dim3(g1), dim3(256), 0, stream, Src, sSb, lds, r,
                       rc, nc, mats, sMb, part, flags, cnt, Hb, sHb, ldh, tau, sTaub, Tws, sTwb);
    hipLaunchKernelGGL((k_cq_gram<true, true>), dim3(g1), dim3(256), 0, stream, Src, sSb, lds, r,
                       rc, nc, mats, sMb, part, flags, cnt, Hb, sHb, ldh, tau, sTaub, Tws, sTwb);
  } else {
    hipLaunchKernelGGL((k_cq_gram<false, false>), dim3(g1), dim3(64 * gw), 0, stream, Src, sSb, lds,
                       r, rc, nc, mats, sMb, part, flags, cnt, Hb, sHb, ldh, tau, sTaub, Tws,
                       sTwb);
    hipLaunchKernelGGL(k_cq_chol1, dim3(batch), dim3(256), 0, stream, (const float*)part, nc,
                       mats, sMb, flags, one_pass);
    // one_pass = 2: no matrix takes the second pass, so its Gram launch (which
    // would return at once for every matrix) is not made.
    if (one_pass != 2)
      hipLaunchKernelGGL((k_cq_gram<true, false>), dim3(g1), dim3(64 * gw), 0, stream, Src, sSb,
                         lds, r, rc, nc, mats, sMb, part, flags, cnt, Hb, sHb, ldh, tau, sTaub,
                         Tws, sTwb);
    hipLaunchKernelGGL(k_cq_recon, dim3(batch), dim3(256), 0, stream, (const float*)part, nc, mats,
                       sMb, flags, Src, sSb, lds, Hb, sHb, ldh, tau, sTaub, Tws, sTwb);
  }
  {
    int rc3 = 0, nc3 = 0;
    cq_chunks(r - kCqB, batch, 64, 64, &rc3, &nc3);
    hipLaunchKernelGGL(k_cq_form, dim3((unsigned)(nc3 * batch)), dim3(256), 0, stream, Src, sSb,
                       lds, Hb, sHb, ldh, r, rc3, nc3, (const float*)mats, sMb,
                       (const int*)flags);
  }
  return hipGetLastError();
}

__global__ void k_cq_zero(int* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Zero the per-matrix arrival counters of the workspace (once per call, before
// its first launch_cq_block: the workspace arrives uninitialised; every use
// leaves them at zero again).
hipError_t launch_cq_reset(float* ws, int batch, hipStream_t stream) {
  int ncw = (256 + batch - 1) / batch;
  if (ncw > kCqMaxChunks) ncw = kCqMaxChunks;
  int* cnt = reinterpret_cast<int*>(ws + (size_t)batch * ncw * kCqSlot +
                                    (size_t)batch * 3 * kCqMat) + batch;
  hipLaunchKernelGGL(k_cq_zero, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, stream, cnt,
                     batch);
  return hipGetLastError();
}

// Offset (floats) of the per-matrix flags in the route's workspace.
size_t cq_flags_offset_floats(int batch) {
  int ncw = (256 + batch - 1) / batch;
  if (ncw > kCqMaxChunks) ncw = kCqMaxChunks;
  return (size_t)batch * ncw * kCqSlot + (size_t)batch * 3 * kCqMat;
}

// Flags of the last launch_cq_block (for the fallback panels).
const int* cq_flags(float* ws, int batch) {
  return reinterpret_cast<const int*>(ws + cq_flags_offset_floats(batch));
}

}  // namespace qr
