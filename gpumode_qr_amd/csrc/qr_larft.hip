// qr_larft.hip -- kernel (c): compact-WY factor T of k <= 64 reflectors.
//
// Reference: the forward LARFT recurrence of src/qrbench/triton_kernels.py:886-909
//   T[i,i] = tau_i,  T[0:i, i] = -tau_i * T[0:i, 0:i] @ (V[:, 0:i]^T v_i),
// with V unit lower-trapezoidal (stored below the diagonal of the factored panel,
// triton_kernels.py:874-884). tau_i == 0 gives a zero column (LAPACK slarft).
//
// One workgroup per matrix: the Gram block S = V^T V is accumulated from
// 64-row chunks staged in LDS, then the k-step recurrence runs on LDS-resident T.
// The 16-column panel kernel builds its own T from the dot products it already
// has; this kernel serves wider blocks and stands alone for testing.
// k_larft_panels (orgqr / ormqr) rebuilds the 16 x 16 T of every panel of a
// factored matrix with the Gram on MFMA.
#include "qr_device.hpp"

namespace qr {

constexpr int kLarftMaxK = 64;

struct LarftShared {
  float vs[64][kLarftMaxK + 1];
  float S[kLarftMaxK][kLarftMaxK + 1];
  float Ts[kLarftMaxK][kLarftMaxK + 1];
  float taus[kLarftMaxK];
};

// T (k x k, row stride ldt) of the k reflectors stored below the diagonal of
// the m x k block Vb, with coefficients taub[0..k-1]. One workgroup of 256.
__device__ void larft_block(const float* __restrict__ Vb, int64_t ldv, int m, int k,
                            const float* __restrict__ taub, float* __restrict__ Tb, int64_t ldt,
                            LarftShared& sh) {
  auto& vs = sh.vs;
  auto& S = sh.S;
  auto& Ts = sh.Ts;
  auto& taus = sh.taus;
  const int tid = threadIdx.x;
  const int npairs = k * (k - 1) / 2;  // strictly upper (p < q)
  constexpr int kMaxPer = (kLarftMaxK * (kLarftMaxK - 1) / 2 + 255) / 256;
  float acc[kMaxPer];
#pragma unroll
  for (int s = 0; s < kMaxPer; ++s) acc[s] = 0.0f;

  for (int r0 = 0; r0 < m; r0 += 64) {
    for (int idx = tid; idx < 64 * k; idx += 256) {
      const int rr = idx / k, cc = idx - rr * k;
      const int row = r0 + rr;
      float v = 0.0f;
      if (row < m) v = (row > cc) ? Vb[(int64_t)row * ldv + cc] : ((row == cc) ? 1.0f : 0.0f);
      vs[rr][cc] = v;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kMaxPer; ++s) {
      const int pi = tid + 256 * s;
      if (pi < npairs) {
        // decode pair index -> (p, q), p < q, column-major over q
        int q = 1, base = 0;
        while (base + q <= pi) {
          base += q;
          ++q;
        }
        const int p = pi - base;
        float sum = acc[s];
        for (int rr = 0; rr < 64; ++rr) sum = fmaf(vs[rr][p], vs[rr][q], sum);
        acc[s] = sum;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int s = 0; s < kMaxPer; ++s) {
    const int pi = tid + 256 * s;
    if (pi < npairs) {
      int q = 1, base = 0;
      while (base + q <= pi) {
        base += q;
        ++q;
      }
      S[pi - base][q] = acc[s];
    }
  }
  if (tid < k) taus[tid] = taub[tid];
  for (int idx = tid; idx < k * k; idx += 256) Ts[idx / k][idx % k] = 0.0f;
  __syncthreads();

  for (int i = 0; i < k; ++i) {
    float s = 0.0f;
    if (tid < i) {
      for (int q = tid; q < i; ++q) s = fmaf(Ts[tid][q], S[q][i], s);
    }
    __syncthreads();
    const float ti = taus[i];
    if (tid < i) Ts[tid][i] = (ti == 0.0f) ? 0.0f : -ti * s;
    if (tid == i) Ts[i][i] = ti;
    __syncthreads();
  }
  for (int idx = tid; idx < k * k; idx += 256) {
    const int p = idx / k, q = idx - (idx / k) * k;
    Tb[(int64_t)p * ldt + q] = Ts[p][q];
  }
}

__global__ __launch_bounds__(256) void k_larft(const float* __restrict__ V, int64_t sVb,
                                               int64_t ldv, int m, int k,
                                               const float* __restrict__ tau, int64_t sTaub,
                                               float* __restrict__ T, int64_t sTb, int64_t ldt) {
  __shared__ LarftShared sh;
  const int b = blockIdx.x;
  larft_block(V + (int64_t)b * sVb, ldv, m, k, tau + (int64_t)b * sTaub, T + (int64_t)b * sTb, ldt,
              sh);
}

// T of every 16-wide panel of factored n x n matrices: one wave per (panel p,
// matrix b) builds the 16 x 16 T of panel p (kw = min(16, n - 16 p)
// reflectors, zero-padded to 16 x 16) at T + b sTb + 256 p.
// The Gram S = V^T V comes from v_mfma_f32_16x16x4f32 with V in the strip
// layout (lane l: column k = l & 15, rows 4 (l >> 4) + v of each 16-row tile):
// that one register is both V^T's A-operand entry and V's B-operand entry, so
// the panel is read once from HBM straight into the MFMA, with no LDS staging.
// T's recurrence then runs with row k of T in lane k (16 serial steps over S
// from LDS).
constexpr int kLpWaves = 4;
__global__ __launch_bounds__(64 * kLpWaves) void k_larft_panels(
    const float* __restrict__ H, int64_t sHb, int64_t ldh, int n, const float* __restrict__ tau,
    int64_t sTaub, float* __restrict__ T, int64_t sTb, int npan, int batch) {
  __shared__ float Sg[kLpWaves][16][17];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int item = blockIdx.x * kLpWaves + w;
  if (item >= npan * batch) return;  // whole wave: no workgroup barrier below
  const int b = item / npan, p = item - b * npan;
  const int lane = threadIdx.x & 63, k = lane & 15, g = lane >> 4;
  const int j0 = 16 * p, r = n - j0, kw = min(16, r);
  const float* Vb = H + (int64_t)b * sHb + (int64_t)j0 * ldh + j0;
  // Branch-free loads: rows outside the panel and columns beyond kw read a
  // valid address (row 0, column 0) and are replaced by zero.
  const int64_t coff = (k < kw) ? k : 0;
  f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  for (int t0 = 0; t0 < r; t0 += 32) {  // two 16-row tiles per round
    float x[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = t0 + 16 * h + 4 * g + v;
        x[h][v] = Vb[((row < r) ? (int64_t)row * ldh : 0) + coff];
      }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = t0 + 16 * h + 4 * g + v;
        // Unit lower-trapezoidal: zero above the diagonal, one on it.
        const float val = (row < r && k < kw) ? ((row > k) ? x[h][v] : (row == k ? 1.0f : 0.0f))
                                              : 0.0f;
        acc[h] = __builtin_amdgcn_mfma_f32_16x16x4f32(val, val, acc[h], 0, 0, 0);
      }
  }
  const f32x4 S = acc[0] + acc[1];  // S[4 g + v][k]
#pragma unroll
  for (int v = 0; v < 4; ++v) Sg[w][4 * g + v][k] = S[v];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // T[k][i] = tau_i (k == i), -tau_i sum_{q < i} T[k][q] S[q][i] (k < i), 0
  // below the diagonal (row k's entries T[k][q < k] are zero, so the sum is
  // zero there); tau_i == 0 gives a zero column, as LAPACK's slarft.
  const float* taub = tau + (int64_t)b * sTaub + j0;
  float trow[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float ti = (i < kw) ? taub[i] : 0.0f;
    float sacc = 0.0f;
#pragma unroll
    for (int q = 0; q < i; ++q) sacc = fmaf(trow[q], Sg[w][q][i], sacc);
    trow[i] = (k == i) ? ti : ((k > i || ti == 0.0f) ? 0.0f : -ti * sacc);
  }
  if (g == 0) {
    float* Tb = T + (int64_t)b * sTb + 256 * p + 16 * k;
#pragma unroll
    for (int i = 0; i < 16; i += 4)
      *reinterpret_cast<f32x4*>(&Tb[i]) = f32x4{trow[i], trow[i + 1], trow[i + 2], trow[i + 3]};
  }
}

hipError_t launch_larft(const float* V, int64_t sVb, int64_t ldv, int m, int k, const float* tau,
                        int64_t sTaub, float* T, int64_t sTb, int64_t ldt, int batch,
                        hipStream_t stream) {
  if (k < 1 || k > kLarftMaxK || m < k) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_larft, dim3(batch), dim3(256), 0, stream, V, sVb, ldv, m, k, tau, sTaub, T,
                     sTb, ldt);
  return hipGetLastError();
}

hipError_t launch_larft_panels(const float* H, int64_t sHb, int64_t ldh, int n, const float* tau,
                               int64_t sTaub, float* T, int64_t sTb, int batch,
                               hipStream_t stream) {
  if (n < 1 || batch < 1) return hipErrorInvalidValue;
  const int npan = (n + 15) / 16;
  const int64_t waves = (int64_t)npan * batch;
  hipLaunchKernelGGL(k_larft_panels, dim3((unsigned)((waves + kLpWaves - 1) / kLpWaves)),
                     dim3(64 * kLpWaves), 0, stream, H, sHb, ldh, n, tau, sTaub, T, sTb, npan,
                     batch);
  return hipGetLastError();
}

}  // namespace qr
