// qr_copy.hip -- strided A -> contiguous H copy that starts the blocked route
// (the reference's H = A.contiguous().clone(), src/qrbench/variants.py:787),
// and the identity that orgqr starts from.
#include "qr_device.hpp"

namespace qr {

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

// Q[b] (n x n, row stride ldq) = I.
__global__ __launch_bounds__(256) void k_eye(float* __restrict__ Q, int64_t sQb, int64_t ldq,
                                             int n, int64_t total) {
  const int64_t nn = (int64_t)n * n;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * 256) {
    const int64_t b = idx / nn;
    const int64_t rem = idx - b * nn;
    const int64_t i = rem / n, j = rem - i * n;
    Q[b * sQb + i * ldq + j] = (i == j) ? 1.0f : 0.0f;
  }
}

hipError_t launch_eye(float* Q, int64_t sQb, int64_t ldq, int batch, int n, hipStream_t stream) {
  const int64_t total = (int64_t)batch * n * n;
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_eye, dim3((unsigned)blocks), dim3(256), 0, stream, Q, sQb, ldq, n, total);
  return hipGetLastError();
}

}  // namespace qr
