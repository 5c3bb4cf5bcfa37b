// qr_smalln.hip -- kernel (a): fused Householder QR of a whole n x n matrix
// (n <= 64) per wavefront, geqrf packing.
//
// Reference: the fused small-n Triton kernel, src/qrbench/triton_kernels.py:641-755
// (one program per matrix, per-column reflector + rank-1 trailing update, pack
// beta on the diagonal and the essential reflector below it).
//
// gfx950 layout: one 64-lane wave per matrix, lane k owns column k in VGPRs
// (a[NP], NP = n rounded up to 8). Column j is published to LDS by lane j; every
// lane then forms its dot product with it from its own registers, so the per-step
// reductions need no cross-lane traffic at all. sigma = x^T x is lane j's own dot
// and alpha is lane j's row-j entry; both are read back with v_readlane, so the
// reflector scalars are wave-uniform. Row indices are compile-time (the outer
// chunk loop is unrolled), so rows above the current chunk are skipped.
#include "qr_device.hpp"

namespace qr {

template <int NP, int CH>
__global__ __launch_bounds__(64) void k_geqrf_smalln(
    const float* __restrict__ A, int64_t sAb, int64_t sAr, int64_t sAc,
    float* __restrict__ H, int64_t sHb, float* __restrict__ tau, int64_t sTb, int n) {
  static_assert(NP % CH == 0 && NP <= 64, "tile");
  __shared__ __align__(16) float xs[2][NP];

  const int b = blockIdx.x;
  const int k = threadIdx.x;  // column owned by this lane
  const float* Ab = A + (int64_t)b * sAb;

  float a[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i)
    a[i] = (i < n && k < n) ? Ab[(int64_t)i * sAr + (int64_t)k * sAc] : 0.0f;

  float my_beta = 0.0f, my_gamma = 1.0f, my_pre = 1.0f, my_tau = 0.0f;

  static_for<0, NP / CH>([&](auto CI) {
    constexpr int jc = decltype(CI)::value * CH;  // first row/column of this chunk
    if (jc < n) {
      for (int jj = 0; jj < CH; ++jj) {
        const int j = jc + jj;
        if (j >= n) break;
        float* x = xs[j & 1];
        // Lane j publishes x = its column below the diagonal (rows <= j masked).
        if (k == j) {
#pragma unroll
          for (int i = jc; i < NP; ++i) x[i] = (i > j) ? a[i] : 0.0f;
        }
        __syncthreads();
        float d = 0.0f;  // x^T a_k over rows > j
#pragma unroll
        for (int i = jc; i < NP; ++i) d = fmaf(x[i], a[i], d);
        float e = 0.0f;  // a_k[j]
#pragma unroll
        for (int i = jc; i < jc + CH; ++i) e = (i == j) ? a[i] : e;
        const float sigma = readlane_f(d, j);
        const float alpha = readlane_f(e, j);

        Reflector R;
        bool fast = true;
        if (j == n - 1) {
          R = reflector_identity(alpha);
        } else if (reflector_fast_ok(alpha, sigma)) {
          R = reflector_fast(alpha, sigma);
        } else {
          // Scaled norm of x from the LDS copy (identical in every lane).
          float xmax = 0.0f;
#pragma unroll
          for (int i = jc; i < NP; ++i) xmax = fmaxf(xmax, fabsf(x[i]));
          float ssq = 0.0f;
          if (xmax > 0.0f) {
#pragma unroll
            for (int i = jc; i < NP; ++i) {
              const float t = x[i] / xmax;
              ssq = fmaf(t, t, ssq);
            }
          }
          R = reflector_scaled(alpha, xmax, ssq);
          fast = false;
        }

        if (k > j) {
          // v^T a_k = a_k[j] + sum_{i>j} v_i a_k[i];  a_k -= tau (v^T a_k) v.
          if (fast) {
            const float c = R.tau * fmaf(R.gamma, d, e);
            const float cg = c * R.gamma;
#pragma unroll
            for (int i = jc; i < NP; ++i) a[i] = fmaf(-cg, x[i], a[i]);
#pragma unroll
            for (int i = jc; i < jc + CH; ++i) a[i] = (i == j) ? a[i] - c : a[i];
          } else if (R.tau != 0.0f) {
            const float c = R.tau * fmaf(R.gamma, R.pre * d, e);
#pragma unroll
            for (int i = jc; i < NP; ++i) a[i] = fmaf(-c, (x[i] * R.pre) * R.gamma, a[i]);
#pragma unroll
            for (int i = jc; i < jc + CH; ++i) a[i] = (i == j) ? a[i] - c : a[i];
          }
        }
        if (k == j) {
          my_beta = R.beta;
          my_gamma = R.gamma;
          my_pre = R.pre;
          my_tau = R.tau;
        }
      }
    }
  });

  if (k < n) {
    float* Hb = H + (int64_t)b * sHb;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      if (i < n) {
        const float v = (i < k) ? a[i] : ((i == k) ? my_beta : (a[i] * my_pre) * my_gamma);
        Hb[(int64_t)i * n + k] = v;
      }
    }
    tau[(int64_t)b * sTb + k] = my_tau;
  }
}

// Host-side dispatch over the padded size.
hipError_t launch_geqrf_smalln(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                               int64_t sHb, float* tau, int64_t sTb, int batch, int n,
                               hipStream_t stream) {
  const int np = (n + 7) & ~7;
  const dim3 grid(batch), block(64);
#define QR_SMALLN_CASE(NPV)                                                                   \
  case NPV:                                                                                   \
    hipLaunchKernelGGL((k_geqrf_smalln<NPV, 8>), grid, block, 0, stream, A, sAb, sAr, sAc, H, \
                       sHb, tau, sTb, n);                                                     \
    break;
  switch (np) {
    QR_SMALLN_CASE(8)
    QR_SMALLN_CASE(16)
    QR_SMALLN_CASE(24)
    QR_SMALLN_CASE(32)
    QR_SMALLN_CASE(40)
    QR_SMALLN_CASE(48)
    QR_SMALLN_CASE(56)
    QR_SMALLN_CASE(64)
    default:
      return hipErrorInvalidValue;
  }
#undef QR_SMALLN_CASE
  return hipGetLastError();
}

}  // namespace qr
