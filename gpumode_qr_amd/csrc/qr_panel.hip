// qr_panel.hip -- kernel (b): Householder factorisation of a tall r x 16 panel
// in place, plus its 16 x 16 compact-WY factor T (the larft of this panel).
//
// Reference: _hh_panel_kernel, src/qrbench/triton_kernels.py:787-909 (per-column
// reflector + in-panel update :839-863, geqrf packing :866-871, forward LARFT
// T recurrence :888-909) and its host call at src/qrbench/variants.py:793-796.
//
// gfx950 layout: a workgroup of NW waves per matrix. Lane l of wave w owns
// column k = l & 15 of the panel for the rows i = (m*NW + w)*4 + (l >> 4),
// m < RL, in VGPRs. Each 16-lane DPP row therefore holds 16 columns of one panel
// row, so the current column j reaches every lane of the row with one
// v_mov_dpp row_newbcast:j (no LDS). Each lane forms the dot of column j with
// its own column over its rows; that single set of dots gives
//   * sigma = x^T x           (lane j),
//   * v_j^T a_k for k > j      (the trailing update of the panel), and
//   * V_k^T v_j for k < j      (the column of T, for free).
// One LDS round (NW partials per column, one barrier) completes each step.
#include "qr_device.hpp"

namespace qr {

template <int NW, int RL>
__global__ __launch_bounds__(64 * NW) void k_panel16(
    float* __restrict__ H, int64_t sHb, int64_t ldh, int j0, int r, int kw,
    float* __restrict__ tau, int64_t sTaub, float* __restrict__ Tout, int64_t sTb) {
  static_assert(NW >= 4, "rows 0..15 must sit in register 0 of waves 0..3");
  __shared__ float red[2][NW][16];
  __shared__ float erow[2][16];
  __shared__ float zbuf[16][16];
  __shared__ float scr[2][NW];

  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int k = lane & 15;
  const int g = lane >> 4;
  float* P = H + (int64_t)b * sHb + (int64_t)j0 * ldh + j0;
  const int row0 = w * 4 + g;  // panel row held in register 0

  float a[RL];
#pragma unroll
  for (int m = 0; m < RL; ++m) {
    const int i = (m * NW + w) * 4 + g;
    a[m] = (i < r && k < kw) ? P[(int64_t)i * ldh + k] : 0.0f;
  }

  float my_beta = 0.0f, my_gamma = 1.0f, my_pre = 1.0f, my_tau = 0.0f;

  static_for<0, 16>([&](auto JC) {
    constexpr int J = decltype(JC)::value;
    if (J < kw) {
      // x = column J below the diagonal, re-broadcast from lane J at each use
      // (lane J's registers do not change during step J). Rows <= J can only
      // be in register 0, so only x0 needs the mask.
      const float x0 = (row0 > J) ? row_bcast16<J>(a[0]) : 0.0f;
      float d = x0 * a[0];
#pragma unroll
      for (int m = 1; m < RL; ++m)
        d = fmaf(row_bcast16_nocse<J>(a[m]), a[m], d);
      d = sum_over_rows16(d);
      if (g == 0) red[J & 1][w][k] = d;
      if (w == J / 4 && g == J % 4) erow[J & 1][k] = a[0];
      __syncthreads();
      float ds = 0.0f;
#pragma unroll
      for (int q = 0; q < NW; ++q) ds += red[J & 1][q][k];
      const float e = erow[J & 1][k];
      const float sigma = readlane_f(ds, J);
      const float alpha = readlane_f(e, J);

      Reflector R;
      bool fast = true;
      if (J >= r - 1) {
        R = reflector_identity(alpha);
      } else if (reflector_fast_ok(alpha, sigma)) {
        R = reflector_fast(alpha, sigma);
      } else {
        // Scaled norm of column J below the diagonal: two workgroup reductions.
        float xm = fabsf(x0);
#pragma unroll
        for (int m = 1; m < RL; ++m)
          xm = fmaxf(xm, fabsf(row_bcast16<J>(a[m])));
        xm = max_over_rows16(xm);
        if (lane == 0) scr[0][w] = xm;
        __syncthreads();
        float xmax = 0.0f;
#pragma unroll
        for (int q = 0; q < NW; ++q) xmax = fmaxf(xmax, scr[0][q]);
        float s = 0.0f;
        if (xmax > 0.0f) {
          const float t0 = x0 / xmax;
          s = t0 * t0;
#pragma unroll
          for (int m = 1; m < RL; ++m) {
            const float t = row_bcast16<J>(a[m]) / xmax;
            s = fmaf(t, t, s);
          }
        }
        s = sum_over_rows16(s);
        if (lane == 0) scr[1][w] = s;
        __syncthreads();
        float ssq = 0.0f;
#pragma unroll
        for (int q = 0; q < NW; ++q) ssq += scr[1][q];
        R = reflector_scaled(alpha, xmax, ssq);
        fast = false;
      }

      // Trailing update of the panel (lanes k > J); every lane executes the
      // FMAs (coefficient 0 where nothing changes) so the DPP sources stay live.
      const bool upd = (k > J) && (k < kw);
      const bool own_row = (w == J / 4) && (g == J % 4);
      if (fast) {
        const float c = R.tau * fmaf(R.gamma, ds, e);
        const float cg = upd ? c * R.gamma : 0.0f;
        a[0] = fmaf(-cg, x0, a[0]);
#pragma unroll
        for (int m = 1; m < RL; ++m)
          a[m] = fmaf(-cg, row_bcast16_nocse<J>(a[m]), a[m]);
        if (upd && own_row) a[0] -= c;
      } else if (R.tau != 0.0f) {
        const float c = R.tau * fmaf(R.gamma, R.pre * ds, e);
        const float cs = upd ? c : 0.0f;
        a[0] = fmaf(-cs, (x0 * R.pre) * R.gamma, a[0]);
#pragma unroll
        for (int m = 1; m < RL; ++m)
          a[m] = fmaf(-cs, (row_bcast16<J>(a[m]) * R.pre) * R.gamma, a[m]);
        if (upd && own_row) a[0] -= c;
      }
      // Column J of T needs z_k = V_k^T v_J for k < J.
      if (w == 0 && g == 0 && k < J)
        zbuf[J][k] = (my_pre * my_gamma) * fmaf(R.pre * R.gamma, ds, e);
      if (k == J) {
        my_beta = R.beta;
        my_gamma = R.gamma;
        my_pre = R.pre;
        my_tau = R.tau;
      }
    }
  });
  __syncthreads();

  // T (16 x 16, upper): T[J][J] = tau_J, T[0:J, J] = -tau_J T[0:J, 0:J] z_J.
  if (w == 0 && g == 0) {
    float trow[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) trow[q] = 0.0f;
    static_for<0, 16>([&](auto JC) {
      constexpr int J = decltype(JC)::value;
      if (J < kw) {
        const float tj = readlane_f(my_tau, J);
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < J; ++q) s = fmaf(trow[q], zbuf[J][q], s);
        trow[J] = (k < J) ? -tj * s : ((k == J) ? tj : 0.0f);
      }
    });
    float* Tb = Tout + (int64_t)b * sTb;
#pragma unroll
    for (int q = 0; q < 16; ++q) Tb[k * 16 + q] = trow[q];
    if (k < kw) tau[(int64_t)b * sTaub + j0 + k] = my_tau;
  }

#pragma unroll
  for (int m = 0; m < RL; ++m) {
    const int i = (m * NW + w) * 4 + g;
    if (i < r && k < kw) {
      const float v = (i < k) ? a[m] : ((i == k) ? my_beta : (a[m] * my_pre) * my_gamma);
      P[(int64_t)i * ldh + k] = v;
    }
  }
}

static inline int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

hipError_t launch_panel16(float* H, int64_t sHb, int64_t ldh, int j0, int r, int kw, float* tau,
                          int64_t sTaub, float* T, int64_t sTb, int batch, hipStream_t stream) {
  if (kw < 1 || kw > 16 || r < kw) return hipErrorInvalidValue;
  const dim3 grid(batch);
#define QR_PANEL_CASE(NWV, RLV)                                                                \
  hipLaunchKernelGGL((k_panel16<NWV, RLV>), grid, dim3(64 * NWV), 0, stream, H, sHb, ldh, j0, \
                     r, kw, tau, sTaub, T, sTb)
  if (r <= 256) {
    const int rl = next_pow2((r + 15) / 16);
    switch (rl) {
      case 1: QR_PANEL_CASE(4, 1); break;
      case 2: QR_PANEL_CASE(4, 2); break;
      case 4: QR_PANEL_CASE(4, 4); break;
      case 8: QR_PANEL_CASE(4, 8); break;
      default: QR_PANEL_CASE(4, 16); break;
    }
  } else if (r <= 2048) {
    const int rl = next_pow2((r + 31) / 32);
    switch (rl) {
      case 16: QR_PANEL_CASE(8, 16); break;
      case 32: QR_PANEL_CASE(8, 32); break;
      default: QR_PANEL_CASE(8, 64); break;
    }
  } else if (r <= 4096) {
    QR_PANEL_CASE(16, 64);
  } else {
    return hipErrorInvalidValue;
  }
#undef QR_PANEL_CASE
  return hipGetLastError();
}

}  // namespace qr
