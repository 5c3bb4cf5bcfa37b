// qr_midn.hip -- fused Householder QR of a whole n x n matrix, 64 < n <= 16 NR,
// one workgroup per matrix: the mid-size counterpart of kernel (a).
//
// Reference: the fused route of make_hh_fused_smalln (src/qrbench/variants.py:
// 739-758, n <= 128) over _hh_fused_qr_kernel (src/qrbench/triton_kernels.py:
// 641-755): one program per matrix, per-column reflectors with beta on the
// diagonal and the essential reflector below it (packing rules :684-719).
//
// gfx950 layout: NR = ceil(n / 16) waves, wave w holding strip w (columns
// 16 w .. 16 w + 15, every row) in VGPRs in the MFMA strip layout of the
// small-n kernel: lane l has k = l & 15 and g = l >> 4, and
//   cs[4 t + v] = A[16 t + 4 g + v][16 w + k]     (zeros outside n x n),
// the accumulator layout of v_mfma_f32_16x16x4f32 for row tile t. The matrix
// never leaves the registers between its load and its store.
//
// Phase P = 0 .. NR-1 (two workgroup barriers per phase):
//   wave P applies panel P-1 to its strip, C -= V T^T V^T C on MFMA, with V
//     and T read from LDS (W = V^T C, W2 = T^T W, C -= V W2), alone;
//   wave P then factors its strip's rows >= 16 P column by column with the
//     small-n kernel's column steps (DPP row broadcasts fused into v_fmac,
//     permlane row-group sums, T built one column behind), packs and stores
//     the strip, and leaves V and T in LDS, while the waves w > P apply panel
//     P-1 to their strips (those on wave P's SIMD one phase later).
// The critical path of a phase is one strip's update and one panel.
#include "qr_colstep.hpp"

namespace qr {

constexpr int kMnVStride = 20;  // row stride of the staged V (floats): conflict-free reads
constexpr int kMnMinStrips = 5;   // n > 64
constexpr int kMnMaxStrips = 12;  // n <= 192

template <int NR>
struct MidnShared {
  // V of the last three panels from their diagonal tiles, twice: row-major
  // (the A operand of C -= V W2) and in the strip layout, lane-linear (W =
  // V^T C). Panel q lives in slot q % 3 from the end of phase q to the end of
  // phase q + 2.
  float vt[3][NR * 16 * kMnVStride];
  float vl[3][NR * 64 * 4];
  float tb[3][16][17];                // T of the last three panels
  int simd[16];                       // SIMD of each wave
  float zb[16][16];                   // z_j = V[:, 0:j]^T v_j of the panel being factored
  float refl[16][2];                  // -beta and tau of its columns
  float save[NR * 4 * 64];            // its registers, for the safe re-run
};

// C -= V T^T V^T C for the strip's row tiles Q .. NR-1, panel Q's V staged
// from its diagonal tile (vt row-major, vl in the strip layout) and its T (tb,
// row-major).
// W = V^T C: lane (k, g) supplies V[16 t + 4 g + v][k] (A) and its own
// C[16 t + 4 g + v][k] (B) for K slice (t, v). W2 = T^T W: T[4 g + v][k] and
// W[4 g + v][k]. C -= V W2: V[16 t + k][4 g + v] and W2[4 g + v][k].
template <int NR, int Q>
__device__ __forceinline__ void midn_apply(float (&cs)[4 * NR], const float* vt,
                                           const float* vl, const float (*tb)[17], int k, int g,
                                           int lane) {
  constexpr int NT = NR - Q;
  f32x4 treg;
#pragma unroll
  for (int v = 0; v < 4; ++v) treg[v] = tb[4 * g + v][k];
  // Two accumulators (even and odd tiles): consecutive MFMAs are independent,
  // so a lone wave issues them back to back instead of waiting on each result.
  f32x4 wacc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const f32x4 vw = *reinterpret_cast<const f32x4*>(&vl[(t * 64 + lane) * 4]);
#pragma unroll
    for (int v = 0; v < 4; ++v)
      wacc[t & 1] =
          __builtin_amdgcn_mfma_f32_16x16x4f32(vw[v], cs[4 * (Q + t) + v], wacc[t & 1], 0, 0, 0);
  }
  const f32x4 wsum = wacc[0] + wacc[1];
  f32x4 w2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int v = 0; v < 4; ++v) w2 = __builtin_amdgcn_mfma_f32_16x16x4f32(treg[v], wsum[v], w2, 0, 0, 0);
  // Tiles in pairs, K slice v outer: two independent accumulations at a time
  // with few extra registers.
#pragma unroll
  for (int t0 = 0; t0 < NT; t0 += 2) {
    const int nt = (t0 + 1 < NT) ? 2 : 1;
    f32x4 va[2], acc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (i >= nt) break;
      const int t = t0 + i;
      va[i] = *reinterpret_cast<const f32x4*>(&vt[(16 * t + k) * kMnVStride + 4 * g]);
      acc[i] = f32x4{cs[4 * (Q + t)], cs[4 * (Q + t) + 1], cs[4 * (Q + t) + 2], cs[4 * (Q + t) + 3]};
    }
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (i < nt) acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(-va[i][v], w2[v], acc[i], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (i >= nt) break;
#pragma unroll
      for (int v = 0; v < 4; ++v) cs[4 * (Q + t0 + i) + v] = acc[i][v];
    }
  }
}

// SIMD of the calling wave within its CU (HW_ID bits 5:4).
__device__ __forceinline__ int simd_id() {
  int v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID, 4, 2)" : "=s"(v));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;  // the same in every lane: each butterfly pair adds the same two values
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// Rare path of a panel (a column with sigma outside [2^-100, 2^100], |alpha|
// above 2^50, or a zero, tiny or huge column): the panel, restored to its state
// before the steps in `pan` (lane-linear strip layout: row r, column c at
// ((r / 16) 64 + ((r / 4) % 4) 16 + c) 4 + r % 4, rows from the diagonal tile),
// is factored there column by column with slarfg's general branches (the
// power-of-two scaled norm, as in the steps' safe pass), left packed (R, beta,
// essential reflectors), with tau to taub and refl, and T (when tbo is given)
// from the Gram of the reflectors. Rolled loops: one copy of the code for
// every panel of the kernel.
__device__ __noinline__ void midn_panel_safe(float* pan, float (*zb)[16], float (*refl)[2],
                                             float (*tbo)[17], float* taub, int P, int n, int kw,
                                             int lane) {
  const int rows = n - 16 * P;
  auto at = [pan](int r, int c) -> float& {
    return pan[(((r >> 4) * 64 + ((r >> 2) & 3) * 16 + c) << 2) + (r & 3)];
  };
  for (int jj = 0; jj < kw; ++jj) {
    const float alpha = at(jj, jj);
    float xm = 0.0f, s2 = 0.0f;
    for (int r = jj + 1 + lane; r < rows; r += 64) {
      const float x = at(r, jj);
      xm = fmaxf(xm, fabsf(x));
      s2 = fmaf(x, x, s2);
    }
    xm = wave_max(xm);
    s2 = wave_sum(s2);
    Reflector R;
    if (16 * P + jj >= n - 1) {
      R = reflector_identity(alpha);
    } else if (reflector_fast_ok(alpha, s2)) {
      R = reflector_fast(alpha, s2);
    } else {
      float scale = 0.0f, ssq = 0.0f;
      if (xm > 0.0f) {
        const int ex = __builtin_amdgcn_frexp_expf(xm);
        float sq = 0.0f;
        for (int r = jj + 1 + lane; r < rows; r += 64) {
          const float q = __builtin_amdgcn_ldexpf(at(r, jj), -ex);
          sq = fmaf(q, q, sq);
        }
        ssq = wave_sum(sq);
        scale = __builtin_amdgcn_ldexpf(1.0f, ex);
      }
      R = reflector_scaled(alpha, scale, ssq);
    }
    // v = (x pre) gamma below the diagonal (pre gamma can overflow: never formed).
    for (int r = jj + 1 + lane; r < rows; r += 64) at(r, jj) = (at(r, jj) * R.pre) * R.gamma;
    wave_lds_sync();
    for (int c = jj + 1; c < kw; ++c) {
      float d = 0.0f;
      for (int r = jj + 1 + lane; r < rows; r += 64) d = fmaf(at(r, jj), at(r, c), d);
      const float tw = R.tau * (at(jj, c) + wave_sum(d));  // tau v^T c, v_jj = 1
      for (int r = jj + 1 + lane; r < rows; r += 64) at(r, c) = fmaf(-tw, at(r, jj), at(r, c));
      wave_lds_sync();
      if (lane == 0) at(jj, c) -= tw;
      wave_lds_sync();
    }
    if (lane == 0) {
      at(jj, jj) = R.beta;
      refl[jj][0] = -R.beta;
      refl[jj][1] = R.tau;
      taub[16 * P + jj] = R.tau;
    }
    wave_lds_sync();
  }
  if (!tbo) return;
  // z[q][j] = v_q^T v_j (q < j < kw): v_j is 1 at row j and zero above.
  for (int e = lane; e < 256; e += 64) {
    const int q = e >> 4, j = e & 15;
    if (q < j && j < kw) {
      float z = at(j, q);
      for (int r = j + 1; r < rows; ++r) z = fmaf(at(r, q), at(r, j), z);
      zb[q][j] = z;
    }
  }
  wave_lds_sync();
  // Row i of T in lane i: T[i][i] = tau_i, T[i][j] = -tau_j sum_{i <= q < j}
  // T[i][q] z[q][j] (upper triangular, zero from column kw on).
  if (lane < 16) {
    const int i = lane;
    for (int j = 0; j < 16; ++j) {
      float val = 0.0f;
      if (j < kw && i <= j) {
        if (i == j) {
          val = refl[j][1];
        } else {
          float sacc = 0.0f;
          for (int q = i; q < j; ++q) sacc = fmaf(tbo[i][q], zb[q][j], sacc);
          val = -refl[j][1] * sacc;
        }
      }
      tbo[i][j] = val;
    }
  }
  wave_lds_sync();
}

// Panel P on its own wave: the column steps over row tiles P .. NR-1, then the
// geqrf packing, the strip's store to H (rows above the panel hold R, final
// since phase P's update) and, for a later panel, V and T into LDS.
template <int NR, int P>
__device__ __forceinline__ void midn_panel(float (&cs)[4 * NR], MidnShared<NR>& sh, float* Hb,
                                           int64_t ldh, float* taub, int n, int k, int g,
                                           int lane) {
  constexpr int NT = NR - P;
  const int kw = min(16, n - 16 * P);  // >= 1: NR = ceil(n / 16)
  const uint64_t kin_mask = __builtin_amdgcn_ballot_w64(k < kw);
  float* zrow = &sh.zb[0][k];
  // Every MFMA result of the strip is read here first (what the steps' wait
  // states assume), and kept for the safe path.
#pragma unroll
  for (int t = 0; t < NT; ++t)
    *reinterpret_cast<f32x4*>(&sh.save[(t * 64 + lane) * 4]) =
        f32x4{cs[4 * (P + t)], cs[4 * (P + t) + 1], cs[4 * (P + t) + 2], cs[4 * (P + t) + 3]};
  SmallnCol col;
  int bad = 0;
  static_for<0, 16>([&](auto JI) {
    constexpr int jj = decltype(JI)::value;
    if (jj < kw) smalln_step<NR, P, jj, false>(cs, sh, zrow, n, kin_mask, bad, col);
  });
  const int kd = 16 * P + k;
  if (__builtin_amdgcn_readfirstlane(bad)) [[unlikely]] {
    wave_lds_sync();
    midn_panel_safe(sh.save, sh.zb, sh.refl, (P + 1 < NR) ? sh.tb[P % 3] : nullptr, taub, P, n,
                    kw, lane);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const f32x4 sv = *reinterpret_cast<const f32x4*>(&sh.save[(t * 64 + lane) * 4]);
#pragma unroll
      for (int v = 0; v < 4; ++v) cs[4 * (P + t) + v] = sv[v];
    }
  } else {
    // The last column of T (the steps compute each column one step late).
    static_for<0, 16>([&](auto JI) {
      constexpr int jq = decltype(JI)::value;
      if (jq == kw - 1) smalln_t_column<jq>(col, sh);
    });
    const float2 rf = *reinterpret_cast<const float2*>(&sh.refl[k][0]);
    const bool kin = k < kw;
    const float my_beta = kin ? -rf.x : 0.0f, my_tau = kin ? rf.y : 0.0f;
    const float my_gamma = col.gamma, my_pre = col.pre;
    if (g == 0 && kin) taub[16 * P + k] = my_tau;
    // R above the diagonal, beta on it, the essential reflector (x pre) gamma below.
#pragma unroll
    for (int t = P; t < NR; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * t + 4 * g + v;
        const float x = cs[4 * t + v];
        cs[4 * t + v] = (row < kd) ? x : ((row == kd) ? my_beta : (x * my_pre) * my_gamma);
      }
    if constexpr (P + 1 < NR) {
      if (g == 0) {
#pragma unroll
        for (int q = 0; q < 16; ++q) sh.tb[P % 3][k][q] = col.trow[q];
      }
    }
  }
  if (kd < n) {
#pragma unroll
    for (int t = 0; t < NR; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (16 * t + 4 * g + v < n) Hb[(16 * t + v) * ldh + 16 * P] = cs[4 * t + v];
  }
  if constexpr (P + 1 < NR) {
    // V, unit lower-trapezoidal from the diagonal tile: zero above row kd, one on it.
    float* vt = sh.vt[P % 3];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 vm;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * (P + t) + 4 * g + v;
        const float x = cs[4 * (P + t) + v];
        vm[v] = (row < kd) ? 0.0f : ((row == kd) ? 1.0f : x);
        vt[(16 * t + 4 * g + v) * kMnVStride + k] = vm[v];
      }
      *reinterpret_cast<f32x4*>(&sh.vl[P % 3][(t * 64 + lane) * 4]) = vm;
    }
  }
}

// A and H may be the same memory (the blocked route's last columns, factored
// in place): every element of a matrix is loaded before the first barrier,
// and nothing is stored before it.
template <int NR>
__global__ __launch_bounds__(64 * NR) void k_geqrf_midn(const float* A, int64_t sAb, int64_t sAr,
                                                       int64_t sAc, float* H, int64_t sHb,
                                                       int64_t ldh, float* __restrict__ tau,
                                                       int64_t sTaub, int n) {
  __shared__ __align__(16) MidnShared<NR> sh;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int k = lane & 15, g = lane >> 4;

  // Branch-free loads of strip w, all issued before the first is used:
  // out-of-range rows or columns read a clamped (valid) address and are
  // replaced by zero.
  float cs[4 * NR];
  {
    const float* base = A + (int64_t)b * sAb + (int64_t)(4 * g) * sAr + (int64_t)k * sAc;
    const int col = 16 * w + k;
    const int64_t coff = (col < n) ? (int64_t)(16 * w) * sAc : -(int64_t)k * sAc;
#pragma unroll
    for (int t = 0; t < NR; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * t + 4 * g + v;
        const int64_t roff = (row < n) ? (int64_t)(16 * t + v) * sAr : -(int64_t)(4 * g) * sAr;
        cs[4 * t + v] = base[roff + coff];
      }
#pragma unroll
    for (int t = 0; t < NR; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * t + 4 * g + v;
        asm volatile("" : "+v"(cs[4 * t + v]));  // keep the load unconditional
        cs[4 * t + v] = (row < n && col < n) ? cs[4 * t + v] : 0.0f;
      }
  }
  float* Hb = H + (int64_t)b * sHb + (int64_t)(4 * g) * ldh + k;
  float* taub = tau + (int64_t)b * sTaub;

  if (lane == 0) sh.simd[w] = simd_id();
  __syncthreads();
  const int my_simd = __builtin_amdgcn_readfirstlane(sh.simd[w]);
  auto apply = [&](auto QI) {
    constexpr int Q = decltype(QI)::value;
    midn_apply<NR, Q>(cs, sh.vt[Q % 3], sh.vl[Q % 3], sh.tb[Q % 3], k, g, lane);
  };
  // Phase P: wave P applies the panels still pending on its strip alone (no
  // other wave's MFMAs compete with it), then factors panel P while the waves
  // right of it apply panel P-1 to their strips. A wave on wave P's SIMD
  // defers that by one phase: its MFMAs would slow the column steps. Panel
  // P-2, deferred in phase P-1, is applied now in any case (its slot is
  // reused at the end of phase P+1).
  bool deferred = false;  // wave-uniform: panel P-2 still to apply
  static_for<0, NR>([&](auto PI) {
    constexpr int P = decltype(PI)::value;
    if constexpr (P > 0) {
      if (w == P) {
        if constexpr (P > 1) {
          if (deferred) apply(std::integral_constant<int, P - 2>{});
        }
        apply(std::integral_constant<int, P - 1>{});
      }
      __syncthreads();
    }
    if (w == P) {
      midn_panel<NR, P>(cs, sh, Hb, ldh, taub, n, k, g, lane);
    } else if constexpr (P > 0) {
      if (w > P) {
        if constexpr (P > 1) {
          if (deferred) apply(std::integral_constant<int, P - 2>{});
        }
        deferred = my_simd == __builtin_amdgcn_readfirstlane(sh.simd[P]);
        if (!deferred) apply(std::integral_constant<int, P - 1>{});
      }
    }
    if constexpr (P + 1 < NR) __syncthreads();
  });
}

int midn_max_n() { return 16 * kMnMaxStrips; }

// 64 < n <= 192. H: element (i, j) of matrix b at H[b sHb + i ldh + j]; tau:
// tau[b sTaub + j]. A and H may be the same memory.
hipError_t launch_geqrf_midn(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                             int64_t sHb, int64_t ldh, float* tau, int64_t sTaub, int batch,
                             int n, hipStream_t stream) {
  const int nr = (n + 15) / 16;
  if (nr < kMnMinStrips || nr > kMnMaxStrips || batch < 1) return hipErrorInvalidValue;
  const dim3 grid(batch), block(64 * nr);
#define QR_MIDN_CASE(NRV)                                                                  \
  case NRV:                                                                                \
    hipLaunchKernelGGL((k_geqrf_midn<NRV>), grid, block, 0, stream, A, sAb, sAr, sAc, H, sHb, \
                       ldh, tau, sTaub, n);                                                \
    break;
  switch (nr) {
    QR_MIDN_CASE(5)
    QR_MIDN_CASE(6)
    QR_MIDN_CASE(7)
    QR_MIDN_CASE(8)
    QR_MIDN_CASE(9)
    QR_MIDN_CASE(10)
    QR_MIDN_CASE(11)
    QR_MIDN_CASE(12)
    default:
      return hipErrorInvalidValue;
  }
#undef QR_MIDN_CASE
  return hipGetLastError();
}

}  // namespace qr
