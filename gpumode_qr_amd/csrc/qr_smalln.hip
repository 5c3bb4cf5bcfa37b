// qr_smalln.hip -- kernel (a): fused Householder QR of a whole n x n matrix
// (n <= 64) per wavefront, geqrf packing, with the trailing updates on MFMA.
//
// Reference: the fused small-n Triton kernel, src/qrbench/triton_kernels.py:641-755
// (one program per matrix, per-column reflectors, beta on the diagonal and the
// essential reflector below it) and its packing/sign rules (:684-719).
//
// gfx950 layout: one 64-lane wave holds the whole matrix in VGPRs, padded to
// NP = 16 S rows and columns (S = ceil(n / 16), zeros outside n x n). Lane l has
// k = l & 15 (column within a 16-column strip) and g = l >> 4 (row group);
//   c[s][4 t + v] = A[16 t + 4 g + v][16 s + k],
// which is the accumulator layout of v_mfma_f32_16x16x4f32 for the 16 x 16 tile
// (t, s), and also its B-operand layout.
//
// Panel p = strip p is factored column by column entirely inside the wave:
// column j is broadcast to every lane of its 16-lane row with DPP row_newbcast,
// each lane forms the partial dot of its column over its rows, and the gfx950
// permlane swaps sum the four row groups. sigma and alpha come back through
// v_readlane, so the reflector scalars are wave-uniform. The strips right of
// the panel are then updated as a compact-WY block, C -= V T^T V^T C, with
// three MFMA chains (W = V^T C, W2 = T^T W, C -= V W2). The only LDS traffic is
// a wave-private 16 x 16 transpose of V per tile and the T recurrence. No
// workgroup barrier is used, so waves of a workgroup are independent. The
// column steps (qr_colstep.hpp) assume what holds here: no VALU instruction
// writes EXEC, and a panel's MFMA results are first read by the panel's save
// stores, before any step.
#include "qr_colstep.hpp"

namespace qr {

constexpr int kSnWaves = 4;     // matrices (one per wave) per workgroup
constexpr int kSnVStride = 20;  // row stride of the V transpose buffer (floats)

template <int S>
struct SmallnShared {
  float vt[S * 16 * kSnVStride];  // V tiles of the current panel, row-major
  float zb[16][16];               // z_j = V[:, 0:j]^T v_j of the current panel
  float tb[16][17];               // T of the current panel
  float refl[16][2];              // -beta and tau of the panel's columns
  // The panel's registers for the safe re-run; also the 16 x (16 S + 4) staging
  // tile of the vectorised load.
  float save[(S * 4 * 64) > 16 * (16 * S + 4) ? (S * 4 * 64) : 16 * (16 * S + 4)];
};

// kStrided: H and tau at the strides given (the blocked route's last columns,
// in place); otherwise H is (batch, n, n) and tau (batch, n), contiguous, and
// the strides are not read. kWhole: n = 16 S (implied by kVec).
template <int S, bool kVec, bool kStrided, bool kWhole>
// At least two waves per SIMD (<= 256 VGPRs): 2048 matrices fill every SIMD
// twice, and the second wave hides the first one's per-column latency.
__global__ __launch_bounds__(64 * kSnWaves, 2)
__attribute__((amdgpu_waves_per_eu(2, 2))) void k_geqrf_smalln(
    const float* __restrict__ A, int64_t sAb, int64_t sAr, int64_t sAc, float* __restrict__ H,
    int64_t sHb, int64_t ldh, float* __restrict__ tau, int64_t sTaub, int batch, int n) {
  __shared__ __align__(16) SmallnShared<S> shm[kSnWaves];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int b = blockIdx.x * kSnWaves + w;
  if (b >= batch) return;  // whole wave: no workgroup barrier below
  SmallnShared<S>& sh = shm[w];
  const int lane = threadIdx.x & 63;
  const int k0 = lane & 15, g0 = lane >> 4;
  const int k = k0, g = g0;
  const float* Ab = A + (int64_t)b * sAb;
  float* zrow = &sh.zb[0][k0];

  float c[S][4 * S];
  // kVec: n = 16 S, unit column stride, 16-byte aligned rows. Each load
  // instruction reads 16 rows of one strip (lane l: row 16 rb + l / 4, columns
  // 16 s + 4 (l % 4) .. +3; 1 KB), strip 0 first; a strip is transposed to the
  // strip layout through a per-wave LDS tile (row pitch kSnVStride:
  // conflict-free reads). Strip 0 is transposed at once; strips 1 .. S-1 only
  // after panel 0's column steps, which so overlap their loads.
  static_assert(!kVec || S == 4, "vectorised load is laid out for 64 x 64");
  f32x4 q[kVec ? S : 1][4];
  auto transpose_strip = [&](auto SI) {
    constexpr int s = decltype(SI)::value;
    const int lr = lane >> 2, lc = 4 * (lane & 3);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
      *reinterpret_cast<f32x4*>(&sh.vt[(16 * rb + lr) * kSnVStride + lc]) = q[s][rb];
    wave_lds_sync();
#pragma unroll
    for (int t = 0; t < S; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) c[s][4 * t + v] = sh.vt[(16 * t + 4 * g + v) * kSnVStride + k];
    wave_lds_sync();
  };
  if constexpr (kVec) {
    const int lr = lane >> 2, lc = 4 * (lane & 3);
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
        q[s][rb] = *reinterpret_cast<const f32x4*>(Ab + (int64_t)(16 * rb + lr) * sAr + 16 * s +
                                                   lc);
    transpose_strip(std::integral_constant<int, 0>{});
  } else {
  // Branch-free loads: out-of-range rows/columns read a clamped (valid)
  // address and are replaced by zero, so the 16 S^2 loads issue back to back,
  // all before the first is used.
  const float* base = Ab + (int64_t)(4 * g) * sAr + (int64_t)k * sAc;
  static_for<0, S>([&](auto SI) {
    constexpr int s = decltype(SI)::value;
    const int col = 16 * s + k;
    const int64_t coff = (col < n) ? (int64_t)(16 * s) * sAc : -(int64_t)k * sAc;
#pragma unroll
    for (int t = 0; t < S; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * t + 4 * g + v;
        const int64_t roff = (row < n) ? (int64_t)(16 * t + v) * sAr : -(int64_t)(4 * g) * sAr;
        c[s][4 * t + v] = base[roff + coff];
      }
  });
  static_for<0, S>([&](auto SI) {
    constexpr int s = decltype(SI)::value;
    const int col = 16 * s + k;
#pragma unroll
    for (int t = 0; t < S; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * t + 4 * g + v;
        asm volatile("" : "+v"(c[s][4 * t + v]));  // keep the load unconditional
        c[s][4 * t + v] = (row < n && col < n) ? c[s][4 * t + v] : 0.0f;
      }
  });
  }

  // Strip s of H, stored as soon as its panel is packed (no later step
  // touches it), so the stores of strips 0 .. S-2 overlap the later panels.
  if constexpr (!kStrided) {
    sHb = (int64_t)n * n;
    ldh = n;
    sTaub = n;
  }
  float* Hb = H + (int64_t)b * sHb + (int64_t)(4 * g) * ldh + k;
  auto store_strip = [&](auto SI) {
    constexpr int s = decltype(SI)::value;
    if (n == 16 * S) {
#pragma unroll
      for (int t = 0; t < S; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) Hb[(16 * t + v) * ldh + 16 * s] = c[s][4 * t + v];
    } else {
      int kk = k0, gg = g0;
      asm volatile("" : "+v"(kk), "+v"(gg));
#pragma unroll
      for (int t = 0; t < S; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (16 * t + 4 * gg + v < n && 16 * s + kk < n)
            Hb[(16 * t + v) * ldh + 16 * s] = c[s][4 * t + v];
    }
  };

  static_for<0, S>([&](auto PI) {
    constexpr int p = decltype(PI)::value;
    constexpr int NT = S - p;  // row tiles at or below the panel's diagonal tile
    // S = ceil(n / 16): every panel but the last has all 16 columns and none of
    // them is column n - 1, so only the last panel of a ragged n tests them.
    constexpr bool kFull = kVec || kWhole || p + 1 < S;
    const int kw = kFull ? 16 : min(16, n - 16 * p);  // >= 1
    // Lanes whose column exists (wave-uniform mask).
    const uint64_t kin_mask = kFull ? ~uint64_t(0) : __builtin_amdgcn_ballot_w64(k0 < kw);

    // The steps only modify the panel's own rows >= 16 p: keep a copy for the
    // safe re-run (conflict-free b128 stores, lane-consecutive).
#pragma unroll
    for (int t = 0; t < NT; ++t)
      *reinterpret_cast<f32x4*>(&sh.save[(t * 64 + lane) * 4]) =
          f32x4{c[p][4 * (p + t)], c[p][4 * (p + t) + 1], c[p][4 * (p + t) + 2],
                c[p][4 * (p + t) + 3]};
    SmallnCol col;
    int bad = 0;
    static_for<0, 16>([&](auto JI) {
      constexpr int jj = decltype(JI)::value;
      if (kFull || jj < kw)
        smalln_step<S, p, jj, false, kFull>(c[p], sh, zrow, n, kin_mask, bad, col);
    });
    if (__builtin_amdgcn_readfirstlane(bad)) [[unlikely]] {
      wave_lds_sync();
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const f32x4 sv = *reinterpret_cast<const f32x4*>(&sh.save[(t * 64 + lane) * 4]);
#pragma unroll
        for (int v = 0; v < 4; ++v) c[p][4 * (p + t) + v] = sv[v];
      }
      col = SmallnCol();
      int unused = 0;
      static_for<0, 16>([&](auto JI) {
        constexpr int jj = decltype(JI)::value;
        if (jj < kw) smalln_step<S, p, jj, true>(c[p], sh, zrow, n, kin_mask, unused, col);
      });
    }
    // The last column of T (the steps compute each column one step late).
    static_for<0, 16>([&](auto JI) {
      constexpr int jq = decltype(JI)::value;
      if (jq == kw - 1) smalln_t_column<jq>(col, sh);
    });
    const float2 rf = *reinterpret_cast<const float2*>(&sh.refl[k][0]);
    const bool kin = k < kw;
    const float my_beta = kin ? -rf.x : 0.0f, my_tau = kin ? rf.y : 0.0f;
    const float my_gamma = col.gamma, my_pre = col.pre;

    if (g == 0 && kin) tau[(int64_t)b * sTaub + 16 * p + k] = my_tau;

    // Final packing of the panel: R above the diagonal, beta on it, the
    // essential reflector v = (x pre) gamma below it.
    const int kd = 16 * p + k;
#pragma unroll
    for (int t = p; t < S; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 16 * t + 4 * g + v;
        const float x = c[p][4 * t + v];
        c[p][4 * t + v] = (row < kd) ? x : ((row == kd) ? my_beta : (x * my_pre) * my_gamma);
      }

    store_strip(PI);
    if constexpr (kVec && p == 0)
      static_for<1, S>([&](auto SI) { transpose_strip(SI); });

    if constexpr (p + 1 < S) {
      // T (16 x 16, upper), row k in lane k: to the accumulator layout via LDS.
      wave_lds_sync();
      if (g == 0) {
#pragma unroll
        for (int q = 0; q < 16; ++q) sh.tb[k][q] = col.trow[q];
      }

      // V of the panel, unit lower-trapezoidal: kept in registers for the
      // A operand of W = V^T C, and staged row-major for the A operand of V W2.
      float vm[NT][4];
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * (p + t) + 4 * g + v;
          const float x = c[p][4 * (p + t) + v];
          vm[t][v] = (row < kd) ? 0.0f : ((row == kd) ? 1.0f : x);
          sh.vt[(16 * t + 4 * g + v) * kSnVStride + k] = vm[t][v];
        }
      wave_lds_sync();
      f32x4 treg, va[NT];
#pragma unroll
      for (int v = 0; v < 4; ++v) treg[v] = sh.tb[4 * g + v][k];
#pragma unroll
      for (int t = 0; t < NT; ++t)
        va[t] = *reinterpret_cast<const f32x4*>(&sh.vt[(16 * t + k) * kSnVStride + 4 * g]);

      // The trailing strips s = p+1 .. S-1 are independent: each phase runs
      // their MFMA chains interleaved, so consecutive MFMAs do not wait on
      // each other's accumulators.
      constexpr int NS = S - 1 - p;
      // W_s = V^T C_s (16 reflectors x 16 columns), accumulator layout.
      f32x4 wacc[NS];
#pragma unroll
      for (int i = 0; i < NS; ++i) wacc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int i = 0; i < NS; ++i)
            wacc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(vm[t][v], c[p + 1 + i][4 * (p + t) + v],
                                                           wacc[i], 0, 0, 0);
      // W2_s = T^T W_s: K slice v pairs T[4g + v][:] with W[4g + v][:].
      f32x4 w2[NS];
#pragma unroll
      for (int i = 0; i < NS; ++i) w2[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int i = 0; i < NS; ++i)
          w2[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(treg[v], wacc[i][v], w2[i], 0, 0, 0);
      // C_s -= V W2_s: lane (k, g) supplies V[16 t + k][4 g + v] and W2[4 g + v][k].
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4 acc[NS];
#pragma unroll
        for (int i = 0; i < NS; ++i)
          acc[i] = f32x4{c[p + 1 + i][4 * (p + t)], c[p + 1 + i][4 * (p + t) + 1],
                         c[p + 1 + i][4 * (p + t) + 2], c[p + 1 + i][4 * (p + t) + 3]};
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int i = 0; i < NS; ++i)
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(-va[t][v], w2[i][v], acc[i], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < NS; ++i)
#pragma unroll
          for (int v = 0; v < 4; ++v) c[p + 1 + i][4 * (p + t) + v] = acc[i][v];
      }
      wave_lds_sync();  // sh is rewritten by the next panel
    }
  });

}

// Host-side dispatch over the number of 16-column strips. H: element (i, j) of
// matrix b at H[b sHb + i ldh + j]; tau: tau[b sTaub + j]. A may be H itself
// (the blocked route's last columns, factored in place): every value a wave
// stores is computed from what it loaded from that same address, so no store
// can overtake the load it overwrites (the restrict qualifiers allow no
// reordering that matters here).
hipError_t launch_geqrf_smalln(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                               int64_t sHb, int64_t ldh, float* tau, int64_t sTaub, int batch,
                               int n, hipStream_t stream) {
  if (n < 1 || n > 64 || batch < 1) return hipErrorInvalidValue;
  const dim3 grid((batch + kSnWaves - 1) / kSnWaves), block(64 * kSnWaves);
  const bool vec = n == 64 && sAc == 1 && (sAr % 4) == 0 && (sAb % 4) == 0 &&
                   (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  const bool strided = !(sHb == (int64_t)n * n && ldh == n && sTaub == n);
  const bool whole = n % 16 == 0;
#define QR_SMALLN_LAUNCH(SV, VEC, STR, WH)                                                  \
  hipLaunchKernelGGL((k_geqrf_smalln<SV, VEC, STR, WH>), grid, block, 0, stream, A, sAb, sAr, \
                     sAc, H, sHb, ldh, tau, sTaub, batch, n)
  if (vec) {
    if (strided)
      QR_SMALLN_LAUNCH(4, true, true, true);
    else
      QR_SMALLN_LAUNCH(4, true, false, true);
    return hipGetLastError();
  }
#define QR_SMALLN_CASE(SV)                        \
  case SV:                                        \
    if (strided) {                                \
      if (whole)                                  \
        QR_SMALLN_LAUNCH(SV, false, true, true);  \
      else                                        \
        QR_SMALLN_LAUNCH(SV, false, true, false); \
    } else {                                      \
      if (whole)                                  \
        QR_SMALLN_LAUNCH(SV, false, false, true); \
      else                                        \
        QR_SMALLN_LAUNCH(SV, false, false, false); \
    }                                             \
    break;
  switch ((n + 15) / 16) {
    QR_SMALLN_CASE(1)
    QR_SMALLN_CASE(2)
    QR_SMALLN_CASE(3)
    QR_SMALLN_CASE(4)
    default:
      return hipErrorInvalidValue;
  }
#undef QR_SMALLN_CASE
#undef QR_SMALLN_LAUNCH
  return hipGetLastError();
}

}  // namespace qr
