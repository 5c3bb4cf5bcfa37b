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

// T of every 16-wide panel of factored n x n matrices: workgroup (p, b) builds
// the 16 x 16 T of panel p of matrix b (kw = min(16, n - 16 p) reflectors,
// zero-padded to 16 x 16) at T + b sTb + 256 p.
__global__ __launch_bounds__(256) void k_larft_panels(const float* __restrict__ H, int64_t sHb,
                                                      int64_t ldh, int n,
                                                      const float* __restrict__ tau,
                                                      int64_t sTaub, float* __restrict__ T,
                                                      int64_t sTb) {
  __shared__ LarftShared sh;
  const int p = blockIdx.x, b = blockIdx.y;
  const int j0 = 16 * p, kw = min(16, n - j0);
  float* Tb = T + (int64_t)b * sTb + 256 * p;
  for (int idx = threadIdx.x; idx < 256; idx += 256) Tb[idx] = 0.0f;
  __syncthreads();
  larft_block(H + (int64_t)b * sHb + (int64_t)j0 * ldh + j0, ldh, n - j0, kw,
              tau + (int64_t)b * sTaub + j0, Tb, 16, sh);
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
  hipLaunchKernelGGL(k_larft_panels, dim3((n + 15) / 16, batch), dim3(256), 0, stream, H, sHb, ldh,
                     n, tau, sTaub, T, sTb);
  return hipGetLastError();
}

}  // namespace qr
