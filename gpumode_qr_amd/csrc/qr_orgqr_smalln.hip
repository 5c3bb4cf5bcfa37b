// qr_orgqr_smalln.hip -- Q of factored n x n matrices, n <= 64, one wavefront
// per matrix (the orgqr counterpart of the fused small-n factorisation).
//
// Reference: torch.linalg.householder_product(H, tau) as the reference's gates
// call it (src/qrbench/checker.py:129; LAPACK sorgqr), Q = H_0 H_1 ... H_{n-1}
// with H_j = I - tau_j v_j v_j^T.
//
// gfx950 layout: the small-n kernel's strip layout, Q in VGPRs,
//   c[s][4 t + v] = Q[16 t + 4 g + v][16 s + k]   (lane l: k = l & 15, g = l >> 4),
// padded to 16 S x 16 S with the identity. Q starts as I and takes the panels'
// block reflectors B_p = I - V_p T_p V_p^T last to first (backward
// accumulation, as sorgqr): B_p only touches rows and columns >= 16 p, since
// the columns left of panel p are still unit vectors that are zero there. Per
// panel: V_p is read from H into the strip layout, its Gram V_p^T V_p is one
// MFMA chain (the register is both V^T's A-operand entry and V's B-operand
// entry), T_p follows from the forward recurrence with row k of T in lane k,
// and C -= V (T (V^T C)) runs on MFMA for the strips right of the panel.
#include "qr_device.hpp"

namespace qr {

constexpr int kOqWaves = 4;     // matrices (one per wave) per workgroup
constexpr int kOqVStride = 20;  // row stride of the row-major V staging (floats)

template <int S>
struct OrgqrShared {
  float vt[S * 16 * kOqVStride];  // V of the current panel, row-major from its diagonal tile
  float gm[16][17];               // its Gram V^T V
  float tb[16][17];               // its T
};

__device__ __forceinline__ void oq_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Two waves per SIMD at most 256 VGPRs each (as the small-n factorisation).
template <int S>
__global__ __launch_bounds__(64 * kOqWaves, 2)
__attribute__((amdgpu_waves_per_eu(2, 2))) void k_orgqr_smalln(
    const float* __restrict__ H, int64_t sHb, int64_t ldh, const float* __restrict__ tau,
    int64_t sTaub, float* __restrict__ Q, int64_t sQb, int64_t ldq, int batch, int n) {
  __shared__ __align__(16) OrgqrShared<S> shm[kOqWaves];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.x * kOqWaves + w;
  if (b >= batch) return;  // whole wave: no workgroup barrier below
  OrgqrShared<S>& sh = shm[w];
  const int lane = threadIdx.x & 63, k = lane & 15, g = lane >> 4;
  const float* Hb = H + (int64_t)b * sHb;
  const float* taub = tau + (int64_t)b * sTaub;

  float c[S][4 * S];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int t = 0; t < S; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        c[s][4 * t + v] = (16 * t + 4 * g + v == 16 * s + k) ? 1.0f : 0.0f;

  static_for<0, S>([&](auto PI) {
    constexpr int p = S - 1 - decltype(PI)::value;
    constexpr int NT = S - p;  // row tiles from the panel's diagonal tile
    const int kw = min(16, n - 16 * p);
    const int col = 16 * p + k;
    // V_p (unit lower-trapezoidal) in the strip layout; branch-free loads from
    // a clamped valid address for rows and columns outside the panel.
    float vm[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * (p + t) + 4 * g + v;
        const bool in = row < n && k < kw;
        const float x = Hb[(in ? (int64_t)row * ldh + col : 0)];
        vm[t][v] = in ? ((row > col) ? x : (row == col ? 1.0f : 0.0f)) : 0.0f;
      }
    // Gram and T.
    f32x4 gacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        gacc = __builtin_amdgcn_mfma_f32_16x16x4f32(vm[t][v], vm[t][v], gacc, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 4; ++v) sh.gm[4 * g + v][k] = gacc[v];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) sh.vt[(16 * t + 4 * g + v) * kOqVStride + k] = vm[t][v];
    oq_wave_sync();
    // T[k][i] = tau_i (k == i), -tau_i sum_{q < i} T[k][q] G[q][i] (k < i), 0
    // below the diagonal; tau_i == 0 gives a zero column.
    float trow[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float ti = (i < kw) ? taub[16 * p + i] : 0.0f;
      float sacc = 0.0f;
#pragma unroll
      for (int q = 0; q < i; ++q) sacc = fmaf(trow[q], sh.gm[q][i], sacc);
      trow[i] = (k == i) ? ti : ((k > i || ti == 0.0f) ? 0.0f : -ti * sacc);
    }
    if (g == 0) {
#pragma unroll
      for (int q = 0; q < 16; ++q) sh.tb[k][q] = trow[q];
    }
    oq_wave_sync();
    // C -= V (T (V^T C)) for the strips p .. S-1, rows from 16 p.
    // W = V^T C: A = V[16 t + 4 g + v][k], B = C[16 t + 4 g + v][k].
    // W2 = T W:  A = T[k][4 g + v], B = W[4 g + v][k].
    // C -= V W2: A = V[16 t + k][4 g + v], B = W2[4 g + v][k].
    constexpr int NS = S - p;
    f32x4 treg, va[NT];
#pragma unroll
    for (int v = 0; v < 4; ++v) treg[v] = sh.tb[k][4 * g + v];
#pragma unroll
    for (int t = 0; t < NT; ++t)
      va[t] = *reinterpret_cast<const f32x4*>(&sh.vt[(16 * t + k) * kOqVStride + 4 * g]);
    f32x4 wacc[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) wacc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int i = 0; i < NS; ++i)
          wacc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(vm[t][v], c[p + i][4 * (p + t) + v],
                                                         wacc[i], 0, 0, 0);
    f32x4 w2[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) w2[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int i = 0; i < NS; ++i)
        w2[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(treg[v], wacc[i][v], w2[i], 0, 0, 0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 acc[NS];
#pragma unroll
      for (int i = 0; i < NS; ++i)
        acc[i] = f32x4{c[p + i][4 * (p + t)], c[p + i][4 * (p + t) + 1],
                       c[p + i][4 * (p + t) + 2], c[p + i][4 * (p + t) + 3]};
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int i = 0; i < NS; ++i)
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(-va[t][v], w2[i][v], acc[i], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < NS; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) c[p + i][4 * (p + t) + v] = acc[i][v];
    }
    oq_wave_sync();  // sh is rewritten by the next panel
  });

  float* Qb = Q + (int64_t)b * sQb;
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int t = 0; t < S; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * t + 4 * g + v, col = 16 * s + k;
        if (row < n && col < n) Qb[(int64_t)row * ldq + col] = c[s][4 * t + v];
      }
}

// Q (batch, n, n) at strides (sQb, ldq, 1) from H at (sHb, ldh, 1) and tau at
// (sTaub, 1); 1 <= n <= 64. H and Q must not overlap.
hipError_t launch_orgqr_smalln(const float* H, int64_t sHb, int64_t ldh, const float* tau,
                               int64_t sTaub, float* Q, int64_t sQb, int64_t ldq, int batch,
                               int n, hipStream_t stream) {
  if (n < 1 || n > 64 || batch < 1) return hipErrorInvalidValue;
  const dim3 grid((batch + kOqWaves - 1) / kOqWaves), block(64 * kOqWaves);
#define QR_ORGQR_CASE(SV)                                                                  \
  case SV:                                                                                 \
    hipLaunchKernelGGL((k_orgqr_smalln<SV>), grid, block, 0, stream, H, sHb, ldh, tau, sTaub, \
                       Q, sQb, ldq, batch, n);                                             \
    break;
  switch ((n + 15) / 16) {
    QR_ORGQR_CASE(1)
    QR_ORGQR_CASE(2)
    QR_ORGQR_CASE(3)
    QR_ORGQR_CASE(4)
    default:
      return hipErrorInvalidValue;
  }
#undef QR_ORGQR_CASE
  return hipGetLastError();
}

}  // namespace qr
