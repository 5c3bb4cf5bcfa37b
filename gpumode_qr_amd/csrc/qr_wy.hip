// qr_wy.hip -- kernel (d): trailing compact-WY update C -= V T^T V^T C with
// true-fp32 MFMA (v_mfma_f32_16x16x4_f32), plus the strided A -> H copy.
//
// Reference: the three batched GEMMs of src/qrbench/variants.py:800-804
//   W1 = V^T C,  W2 = T^T W1,  C += -V W2   (rocBLAS SGEMM through torch.bmm).
// Here W1 and W2 are fused in one kernel (T^T is applied in the epilogue while
// W1 is still in LDS), and the rank-16 update is a second kernel whose MFMA
// accumulators are initialised with C, so C is read once and written once.
//
// MFMA 16x16x4 f32 operand layout (lane l = 0..63):
//   A (16 x 4): A[l % 16][l / 16]     B (4 x 16): B[l / 16][l % 16]
//   D (16 x 16): D[4 * (l / 16) + v][l % 16], v = 0..3
#include "qr_device.hpp"

namespace qr {

// V is the unit lower-trapezoidal reflector block stored in place in the panel.
__device__ __forceinline__ float load_v(const float* P, int64_t ldh, int row, int col, int r) {
  if (row >= r || row < col) return 0.0f;
  if (row == col) return 1.0f;
  return P[(int64_t)row * ldh + col];
}

// W2[b] (16 x c) = T^T (V^T C) for one 64-column tile of C. Grid (ceil(c/64), batch),
// 4 waves split the r rows (K dimension) and are summed through LDS.
__global__ __launch_bounds__(256) void k_wy_w2_16(const float* __restrict__ H, int64_t sHb,
                                                  int64_t ldh, int j0, int r, int c,
                                                  const float* __restrict__ T, int64_t sTb,
                                                  float* __restrict__ W2, int64_t sWb) {
  __shared__ float part[4][16][65];
  __shared__ float wsum[16][65];
  __shared__ float Ts[16][16];

  const int b = blockIdx.y;
  const int col0 = blockIdx.x * 64;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int ii = lane & 15, kk = lane >> 4;
  const float* P = H + (int64_t)b * sHb + (int64_t)j0 * ldh + j0;
  const float* C = P + 16;

  f32x4 acc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) acc[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int nsteps = (r + 3) / 4;
#pragma unroll 4
  for (int t = w; t < nsteps; t += 4) {
    const int row = 4 * t + kk;
    const float av = load_v(P, ldh, row, ii, r);
    float bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = col0 + 16 * q + ii;
      bv[q] = (row < r && col < c) ? C[(int64_t)row * ldh + col] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[q], acc[q], 0, 0, 0);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[w][4 * kk + v][16 * q + ii] = acc[q][v];
  if (threadIdx.x < 256) {
    const float* Tb = T + (int64_t)b * sTb;
    Ts[threadIdx.x >> 4][threadIdx.x & 15] = Tb[threadIdx.x];
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int idx = threadIdx.x + 256 * s;
    const int p = idx >> 6, col = idx & 63;
    wsum[p][col] = part[0][p][col] + part[1][p][col] + part[2][p][col] + part[3][p][col];
  }
  __syncthreads();
  float* Wb = W2 + (int64_t)b * sWb;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int idx = threadIdx.x + 256 * s;
    const int p = idx >> 6, col = idx & 63;
    float acc2 = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q)
      if (q <= p) acc2 = fmaf(Ts[q][p], wsum[q][col], acc2);
    if (col0 + col < c) Wb[(int64_t)p * c + col0 + col] = acc2;
  }
}

// C[b] -= V W2 on a 64 x 64 tile. Grid (ceil(r/64), ceil(c/64), batch); wave w
// owns rows 16w..16w+15 of the tile, K = 16 (four MFMA steps).
__global__ __launch_bounds__(256) void k_wy_apply_16(float* __restrict__ H, int64_t sHb,
                                                     int64_t ldh, int j0, int r, int c,
                                                     const float* __restrict__ W2, int64_t sWb) {
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int ii = lane & 15, kk = lane >> 4;
  const int row0 = blockIdx.x * 64 + 16 * w;
  const int col0 = blockIdx.y * 64;
  float* P = H + (int64_t)b * sHb + (int64_t)j0 * ldh + j0;
  float* C = P + 16;
  const float* Wb = W2 + (int64_t)b * sWb;

  f32x4 acc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int col = col0 + 16 * q + ii;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = row0 + 4 * kk + v;
      acc[q][v] = (row < r && col < c) ? C[(int64_t)row * ldh + col] : 0.0f;
    }
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float av = -load_v(P, ldh, row0 + ii, 4 * s + kk, r);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = col0 + 16 * q + ii;
      const float bv = (col < c) ? Wb[(int64_t)(4 * s + kk) * c + col] : 0.0f;
      acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[q], 0, 0, 0);
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int col = col0 + 16 * q + ii;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = row0 + 4 * kk + v;
      if (row < r && col < c) C[(int64_t)row * ldh + col] = acc[q][v];
    }
  }
}

hipError_t launch_wy_w2_16(const float* H, int64_t sHb, int64_t ldh, int j0, int r, int c,
                           const float* T, int64_t sTb, float* W2, int64_t sWb, int batch,
                           hipStream_t stream) {
  hipLaunchKernelGGL(k_wy_w2_16, dim3((c + 63) / 64, batch), dim3(256), 0, stream, H, sHb, ldh,
                     j0, r, c, T, sTb, W2, sWb);
  return hipGetLastError();
}

hipError_t launch_wy_apply_16(float* H, int64_t sHb, int64_t ldh, int j0, int r, int c,
                              const float* W2, int64_t sWb, int batch, hipStream_t stream) {
  hipLaunchKernelGGL(k_wy_apply_16, dim3((r + 63) / 64, (c + 63) / 64, batch), dim3(256), 0,
                     stream, H, sHb, ldh, j0, r, c, W2, sWb);
  return hipGetLastError();
}

// H[b] (contiguous n x n) = A[b] with arbitrary element strides.
__global__ __launch_bounds__(256) void k_copy_in(const float* __restrict__ A, int64_t sAb,
                                                 int64_t sAr, int64_t sAc, float* __restrict__ H,
                                                 int64_t sHb, int n, int64_t total) {
  const int64_t nn = (int64_t)n * n;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * 256) {
    const int64_t b = idx / nn;
    const int64_t rem = idx - b * nn;
    const int64_t i = rem / n, j = rem - i * n;
    H[b * sHb + rem] = A[b * sAb + i * sAr + j * sAc];
  }
}

hipError_t launch_copy_in(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                          int64_t sHb, int batch, int n, hipStream_t stream) {
  const int64_t total = (int64_t)batch * n * n;
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_copy_in, dim3((unsigned)blocks), dim3(256), 0, stream, A, sAb, sAr, sAc, H,
                     sHb, n, total);
  return hipGetLastError();
}

}  // namespace qr
