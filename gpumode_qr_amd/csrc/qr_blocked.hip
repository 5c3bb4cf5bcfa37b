// qr_blocked.hip -- kernels (b) panel and (d) trailing update of the blocked
// factorisation, both built on one register layout and one MFMA routine.
//
// Reference: the right-looking blocked loop of src/qrbench/variants.py:786-805,
// the fused panel kernel _hh_panel_kernel (src/qrbench/triton_kernels.py:787-909)
// and the trailing GEMMs C -= V (T^T (V^T C)) at variants.py:800-804.
//
// Two-level blocking. The matrix is processed in outer blocks of P 16-wide
// panels (NB = 16 P columns). Inside an outer block, panel p is factored by
// k_panel, which first applies panels 0..p-1 of the same outer block to its 16
// columns (left-looking, so no extra launches), then factors them and writes
// V_p (in place), tau_p and the 16 x 16 compact-WY factor T_p. The columns right
// of the outer block are then updated by k_trail: each workgroup holds a 16-wide
// strip of C (all r rows) in VGPRs and applies the P block reflectors one after
// the other, so C crosses HBM once per outer block instead of once per panel.
//
// Both kernels keep their columns in the strip layout of qr_wy.hpp and apply
// block reflectors with its apply_wy16p.
#include "qr_wy.hpp"

namespace qr {

// Lanes of column j (is_j) write column j below the diagonal row dj (this
// wave's rows, strip order) into the wave's slab; rows <= dj lie in tile 0.
template <int NW, int RL>
__device__ __forceinline__ void publish_x(float* __restrict__ xw, const float (&c)[RL], int dj,
                                          bool is_j, int w, int g) {
  using S = Strip<NW, RL>;
  if (is_j) {
    f32x4 xv;
#pragma unroll
    for (int v = 0; v < 4; ++v) xv[v] = (S::row(0, v, w, g) > dj) ? c[v] : 0.0f;
    *reinterpret_cast<f32x4*>(&xw[4 * g]) = xv;
#pragma unroll
    for (int t = 1; t < S::kTiles; ++t) {  // rows >= r hold zeros
      const f32x4 cv = {c[4 * t], c[4 * t + 1], c[4 * t + 2], c[4 * t + 3]};
      *reinterpret_cast<f32x4*>(&xw[16 * t + 4 * g]) = cv;
    }
  }
}

// Shared memory of k_panel.
template <int NW, int RL>
struct PanelShared {
  WyPipeShared<NW, RL> wy;
  alignas(16) float xs[NW][4 * RL];  // per-wave x slab of the general pass
  // Row stride 4 NW + 4: the b128 reads of 16 columns land on distinct banks.
  alignas(16) float red[2][16][4 * NW + 4];
  float erow[2][16];
  alignas(16) float zbuf[16][16];
  float taus[16];
  float scr[2][NW];
};

// What lane k keeps of column k's own step.
struct PanelCol {
  float beta = 0.0f, gamma = 1.0f, pre = 1.0f, tau = 0.0f;
};

// x^T c_k summed over the 4 NW partials (wave w, row group g) at rp.
template <int NW>
__device__ __forceinline__ float panel_dot_sum(const float* __restrict__ rp) {
  f32x4 a4 = *reinterpret_cast<const f32x4*>(rp);
#pragma unroll
  for (int u = 1; u < NW; ++u) {
    const f32x4 q4 = *reinterpret_cast<const f32x4*>(rp + 4 * u);
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) a4[e4] += q4[e4];
  }
  return (a4[0] + a4[1]) + (a4[2] + a4[3]);
}

// Sum of the NW per-wave partials at rp, in a fixed pairwise order (the same
// in every lane of a column).
template <int NW>
__device__ __forceinline__ float panel_wave_sum(const float* __restrict__ rp) {
  static_assert(NW % 4 == 0, "b128 reads of the partials");
  f32x4 a4 = *reinterpret_cast<const f32x4*>(rp);
#pragma unroll
  for (int u = 1; u < NW / 4; ++u) {
    const f32x4 q4 = *reinterpret_cast<const f32x4*>(rp + 4 * u);
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) a4[e4] += q4[e4];
  }
  return (a4[0] + a4[1]) + (a4[2] + a4[3]);
}

// Fast pass over the kw column steps of the panel whose diagonal rows
// 16p..16p+15 are tile 0 of wave p. The steps are unrolled, and x (column J
// below the diagonal) is read straight from the registers of lane J of each
// 16-lane row by DPP row_newbcast, folded into the v_fmac of the dot and of
// the update: no LDS traffic for x and one workgroup barrier per step. Each
// wave sums its four row groups with permlane swaps first, so the barrier
// exchanges one partial per wave and column. Lane conditions are
// compile-time lane masks (lanes_*), combined with wave-uniform ones: selects
// on them read an SGPR pair instead of comparing per lane.
// Returns false, with c and st meaningless, if some column was outside the
// fast reflector's range (zero, tiny or huge norm); the result is then to be
// recomputed by panel_general_pass.
template <int NW, int RL>
__device__ __forceinline__ bool panel_fast_pass(float (&c)[RL], PanelShared<NW, RL>& sh, int p,
                                                int r, int kw, int w, int lane, PanelCol& st) {
  const int k = lane & 15;
  const int d0 = 16 * p;
  // Lanes whose column exists; tile 0 of wave w lies wholly below the panel's
  // diagonal rows (w > p), above them (w < p), or is the diagonal tile (w = p).
  const uint64_t kin = __builtin_amdgcn_ballot_w64(k < kw);
  const bool diag = w == p;
  const uint64_t tile0_rows = w > p ? ~uint64_t(0) : uint64_t(0);
  int bad = 0;  // wave-uniform integer flag (a bool becomes a per-lane 0/1 here)
  static_for<0, 16>([&](auto jc) __attribute__((always_inline)) {
    constexpr int J = decltype(jc)::value;
    if (J >= kw) return;
    const int dj = d0 + J;
    constexpr uint64_t row_j = lanes_g_eq(J >> 2);  // row group of row dj in tile 0
    if (lane_in(diag ? row_j : 0)) sh.erow[J & 1][k] = c[J & 3];
    // Tile 0's broadcast with its rows <= dj zeroed, kept for the update.
    float xb0[4], dv[4];
    static_for<0, 4>([&](auto vc) __attribute__((always_inline)) {
      constexpr int v = decltype(vc)::value;
      constexpr uint64_t below = lanes_g_ge((J - v + 4) / 4);  // 4 g + v > J
      xb0[v] = lane_in(diag ? below : tile0_rows) ? row_bcast16<J>(c[v]) : 0.0f;
      dv[v] = xb0[v] * c[v];
    });
#pragma unroll
    for (int t = 1; t < RL / 4; ++t)
      dot4_bcast16<J>(dv[0], dv[1], dv[2], dv[3], c[4 * t], c[4 * t + 1], c[4 * t + 2],
                      c[4 * t + 3]);
    const float dw = rows16_sum((dv[0] + dv[1]) + (dv[2] + dv[3]));
    if (lane_in(lanes_g_eq(0))) sh.red[J & 1][k][w] = dw;
    __syncthreads();
    const float ds = panel_wave_sum<NW>(&sh.red[J & 1][k][0]);
    const float e = sh.erow[J & 1][k];
    const float sigma = readlane_f(ds, J);
    const float alpha = readlane_f(e, J);
    const bool ident = dj >= r - 1;  // no rows below the diagonal
    bad |= (ident || reflector_fast_ok_bits(alpha, sigma)) ? 0 : 1;
    Reflector R = reflector_fast_rcp(alpha, sigma);
    if (ident) R = reflector_identity(alpha);
    const float wk = fmaf(R.gamma, ds, e);  // v_J^T c_k
    const float cc = R.tau * wk;
    const float ncx = lane_in(lanes_k_gt(J) & kin) ? -(cc * R.gamma) : 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) c[v] = fmaf(ncx, xb0[v], c[v]);
#pragma unroll
    for (int t = 1; t < RL / 4; ++t)
      axpy4_bcast16<J>(c[4 * t], c[4 * t + 1], c[4 * t + 2], c[4 * t + 3], ncx);
    // v_J[dj] = 1
    const float cj = c[J & 3] - cc;
    c[J & 3] = lane_in(diag ? lanes_k_gt(J) & kin & row_j : 0) ? cj : c[J & 3];
    // Column J of T needs z_k = V_k^T v_J = (c_k[dj] + gamma x^T c_k) gamma_k, k < J.
    if (lane_in(w == 0 ? lanes_g_eq(0) & lanes_k_lt(J) : 0)) sh.zbuf[J][k] = wk * st.gamma;
    const bool own = lane_in(lanes_k_eq(J));
    st.beta = own ? R.beta : st.beta;
    st.gamma = own ? R.gamma : st.gamma;
    st.tau = own ? R.tau : st.tau;
  });
  st.pre = 1.0f;
  return __builtin_amdgcn_readfirstlane(bad) == 0;
}

// General pass: the same steps for any column (slarfg's zero-norm and
// rescaled branches included), a runtime loop with x published by the lanes of
// column j into the wave's LDS slab.
template <int NW, int RL>
__device__ __forceinline__ void panel_general_pass(float (&c)[RL], PanelShared<NW, RL>& sh, int p,
                                                   int r, int kw, int w, int lane,
                                                   PanelCol& st) {
  using S = Strip<NW, RL>;
  const int k = lane & 15, g = lane >> 4;
  const int d0 = 16 * p;
  float* xw = sh.xs[w];
  // Small strips keep x in registers between the dot and the update.
  constexpr bool kKeepX = RL <= 32;
  constexpr int RX = kKeepX ? RL : 1;

  // x for step 0; later steps are published by the lanes of column j+1 right
  // after their update of step j, so the write is off the critical path.
  publish_x<NW, RL>(xw, c, d0, k == 0, w, g);
  for (int j = 0; j < kw; ++j) {
    const int dj = d0 + j;
    if (w == p && g == (j >> 2)) {
      // Opaque copies: a select between loads of c[0..3] would be folded into
      // one load at a computed index, and c would no longer fit in registers.
      float t0 = c[0], t1 = c[1], t2 = c[2], t3 = c[3];
      asm("" : "+v"(t0), "+v"(t1), "+v"(t2), "+v"(t3));
      const int v = j & 3;
      sh.erow[j & 1][k] = (v == 0) ? t0 : (v == 1) ? t1 : (v == 2) ? t2 : t3;
    }
    wave_sync();
    float x[RX];
    float dv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < S::kTiles; ++t) {
      const f32x4 xv = *reinterpret_cast<const f32x4*>(&xw[16 * t + 4 * g]);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if constexpr (kKeepX) x[4 * t + v] = xv[v];
        dv[v] = fmaf(xv[v], c[4 * t + v], dv[v]);
      }
    }
    // Partial dot of (wave w, row group g) for column k, summed after the barrier.
    sh.red[j & 1][k][4 * w + g] = (dv[0] + dv[1]) + (dv[2] + dv[3]);
    __syncthreads();
    const float ds = panel_dot_sum<NW>(sh.red[j & 1][k]);
    const float e = sh.erow[j & 1][k];
    const float sigma = readlane_f(ds, j);
    const float alpha = readlane_f(e, j);

    Reflector R;
    bool fast = true;
    if (dj >= r - 1) {
      R = reflector_identity(alpha);
    } else if (reflector_fast_ok(alpha, sigma)) {
      R = reflector_fast(alpha, sigma);
    } else {
      // Zero, tiny or huge column: scaled norm of x from the slab, two
      // workgroup reductions.
      float xm = 0.0f;
      for (int idx = lane; idx < 4 * RL; idx += 64) xm = fmaxf(xm, fabsf(xw[idx]));
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) xm = fmaxf(xm, __shfl_xor(xm, o));
      if (lane == 0) sh.scr[0][w] = xm;
      __syncthreads();
      float xmax = 0.0f;
#pragma unroll
      for (int u = 0; u < NW; ++u) xmax = fmaxf(xmax, sh.scr[0][u]);
      float sq = 0.0f;
      if (xmax > 0.0f) {
        for (int idx = lane; idx < 4 * RL; idx += 64) {
          const float tq = xw[idx] / xmax;
          sq = fmaf(tq, tq, sq);
        }
      }
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) sq += __shfl_xor(sq, o);
      if (lane == 0) sh.scr[1][w] = sq;
      __syncthreads();
      float ssq = 0.0f;
#pragma unroll
      for (int u = 0; u < NW; ++u) ssq += sh.scr[1][u];
      R = reflector_scaled(alpha, xmax, ssq);
      fast = false;
    }

    const bool upd = (k > j) && (k < kw);
    const bool own_row = (w == p) && (g == (j >> 2));
    if (fast || R.tau != 0.0f) {
      const float wk = fast ? fmaf(R.gamma, ds, e) : fmaf(R.gamma, R.pre * ds, e);
      const float cc = R.tau * wk;
      // fast: c -= (cc gamma) x;  slow: c -= cc ((x pre) gamma)
      const float cx = upd ? (fast ? cc * R.gamma : cc) : 0.0f;
      if (fast && kKeepX) {
#pragma unroll
        for (int m = 0; m < RX; ++m) c[m] = fmaf(-cx, x[m], c[m]);
      } else {
#pragma unroll
        for (int t = 0; t < S::kTiles; ++t) {
          const f32x4 xv = *reinterpret_cast<const f32x4*>(&xw[16 * t + 4 * g]);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float xe = fast ? xv[v] : (xv[v] * R.pre) * R.gamma;
            c[4 * t + v] = fmaf(-cx, xe, c[4 * t + v]);
          }
        }
      }
      // v_j[dj] = 1 (unconditional stores at fixed indices, for the same reason)
#pragma unroll
      for (int v = 0; v < 4; ++v) c[v] -= (upd && own_row && v == (j & 3)) ? cc : 0.0f;
    }
    // Column j of T needs z_k = V_k^T v_j = ((c_k[j] + (x^T c_k pre) gamma) pre_k)
    // gamma_k for k < j; pre gamma itself can overflow for tiny columns.
    if (w == 0 && g == 0 && k < j)
      sh.zbuf[j][k] = (fmaf(R.gamma, R.pre * ds, e) * st.pre) * st.gamma;
    if (k == j) {
      st.beta = R.beta;
      st.gamma = R.gamma;
      st.pre = R.pre;
      st.tau = R.tau;
    }
    // x for step j+1 (every lane of this wave has finished reading the slab).
    if (j + 1 < kw) publish_x<NW, RL>(xw, c, dj + 1, k == j + 1, w, g);
  }
}

// c := panel p (kw columns at Src + 16 p, row stride lds, r rows, strip
// layout) after the left-looking update with panels 0..p-1 of the outer block
// at Blk (V and R in place, row stride ldh).
template <int NW, int RL>
__device__ __forceinline__ void panel_load_apply(float (&c)[1][RL], const float* __restrict__ Blk,
                                                 int64_t ldh, const float* Src, int64_t lds,
                                                 int p, int r, int kw,
                                                 const float* __restrict__ Tb,
                                                 WyPipeShared<NW, RL>& wy, int w, int lane) {
  auto block = [&](int q) { return VBlock{Blk + (int64_t)(16 * q) * ldh + 16 * q, 16 * q, 16}; };
  VChunk<NW, RL> ck;
  if (p > 0) load_v_chunk<NW, RL>(ck, block(0), ldh, r, 0, w, lane);
  load_strip<NW, RL>(c[0], Src + 16 * p, lds, r, kw, w, lane);
  for (int q = 0; q < p; ++q)
    apply_wy16p<NW, RL, 1>(c, ck, block(q), Tb + 256 * q, block(q + 1 < p ? q + 1 : q), q + 1 < p,
                           ldh, r, wy, w, lane);
}

// The fast pass can be switched off (every panel then takes the general pass).
#ifndef QR_PANEL_FAST
#define QR_PANEL_FAST 1
#endif
constexpr bool kPanelFastPass = QR_PANEL_FAST != 0;

// Body of the panel kernels: factor panel p of matrix b (see k_panel).
template <int NW, int RL>
__device__ __forceinline__ void panel_factor(PanelShared<NW, RL>& sh, int b, float* __restrict__ H,
                                             int64_t sHb, int64_t ldh, int J0, int p, int r,
                                             int kw, float* __restrict__ tau, int64_t sTaub,
                                             float* __restrict__ Tws, int64_t sTwb,
                                             const float* A, int64_t sAb, int64_t lda) {
  using S = Strip<NW, RL>;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int k = lane & 15, g = lane >> 4;
  float* Blk = H + (int64_t)b * sHb + (int64_t)J0 * ldh + J0;
  float* P = Blk + 16 * p;
  float* Tb = Tws + (int64_t)b * sTwb;
  const float* Src = A ? A + (int64_t)b * sAb + (int64_t)J0 * lda + J0 : Blk;
  const int64_t lds = A ? lda : ldh;

  // The panel after the left-looking update with panels 0..p-1; the panel in
  // HBM is not written before the end, so the general pass can start over.
  float cs[1][RL];
  float (&c)[RL] = cs[0];
  panel_load_apply<NW, RL>(cs, Blk, ldh, Src, lds, p, r, kw, Tb, sh.wy, w, lane);

  PanelCol st;
  bool ok = false;
  if constexpr (kPanelFastPass) ok = panel_fast_pass<NW, RL>(c, sh, p, r, kw, w, lane, st);
  if (!ok) [[unlikely]] {
    if constexpr (kPanelFastPass) {
      __syncthreads();  // every wave is past its last read of erow / red
      panel_load_apply<NW, RL>(cs, Blk, ldh, Src, lds, p, r, kw, Tb, sh.wy, w, lane);
      st = PanelCol{};
    }
    panel_general_pass<NW, RL>(c, sh, p, r, kw, w, lane, st);
  }
  const int d0 = 16 * p;

  // Write back first: R above the diagonal, beta on it, v = (x pre) gamma
  // below. The stores drain while wave 0 forms T.
  const int kd = d0 + k;
#pragma unroll
  for (int t = 0; t < S::kTiles; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = S::row(t, v, w, g);
      c[4 * t + v] =
          (row < kd) ? c[4 * t + v] : ((row == kd) ? st.beta : (c[4 * t + v] * st.pre) * st.gamma);
    }
  store_strip<NW, RL>(c, P, ldh, r, kw, w, lane);

  // T_p (16 x 16, upper): T[j][j] = tau_j, T[0:j, j] = -tau_j T[0:j, 0:j] z_j.
  // Lane k of wave 0 holds row k of T in registers; z_j rows are b128 reads.
  // Only wave 0 wrote zbuf and writes taus, so a wave-level sync suffices.
  if (w != 0) return;  // the caller synchronises the workgroup before reusing sh
  if (g == 0) sh.taus[k] = (k < kw) ? st.tau : 0.0f;
  wave_sync();
  if (g == 0) {
    float trow[16];
    const float tk = sh.taus[k];
#pragma unroll
    for (int q = 0; q < 16; ++q) trow[q] = (q == k) ? tk : 0.0f;
#pragma unroll
    for (int j = 1; j < 16; ++j) {
      float z[16];
#pragma unroll
      for (int q4 = 0; q4 < (j + 3) / 4; ++q4) {
        const f32x4 zz = *reinterpret_cast<const f32x4*>(&sh.zbuf[j][4 * q4]);
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) z[4 * q4 + e4] = zz[e4];
      }
      float sa = 0.0f, sb = 0.0f;
#pragma unroll
      for (int q = 0; q < j; ++q) {  // trow[q] = 0 for q < k
        if (q & 1) sb = fmaf(trow[q], z[q], sb);
        else sa = fmaf(trow[q], z[q], sa);
      }
      const float tj = sh.taus[j];
      // zbuf rows j >= kw are not written by this launch: never read them.
      trow[j] = (j < kw && k < j) ? -tj * (sa + sb) : trow[j];
    }
    float* Tp = Tb + 256 * p;
#pragma unroll
    for (int q = 0; q < 16; ++q) Tp[k * 16 + q] = trow[q];
    if (k < kw) tau[(int64_t)b * sTaub + J0 + d0 + k] = st.tau;
  }
}

// Factor panel p (columns 16p..16p+kw-1 of the outer block whose top-left is
// Blk, r rows) after applying panels 0..p-1 of the block (their T's at Tb).
// Writes V_p / R in place, tau_p, and T_p at Tb + 256 p. The panel's columns are
// read from H, or from A (row stride lda, unit column stride) when A is not
// null: the first outer block reads the caller's matrix directly. When `only`
// is not null, only matrices b with only[b] == 1 are factored (the others
// return at once).
// Panels of 4 or 8 waves and up to 16 strip registers run at most 80 VGPRs
// (six waves per SIMD), so that three 8-wave or six 4-wave workgroups share a
// CU: at b640 n512 the 640 panels of a launch run in one round instead of two.
// Wider strips keep their registers.
template <int NW, int RL>
constexpr int kPanelWavesPerEu = (NW <= 8 && RL <= 16) ? 6 : 1;

template <int NW, int RL>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(kPanelWavesPerEu<NW, RL>))) void k_panel(float* __restrict__ H, int64_t sHb,
                                                   int64_t ldh, int J0, int p, int r, int kw,
                                                   float* __restrict__ tau, int64_t sTaub,
                                                   float* __restrict__ Tws, int64_t sTwb,
                                                   const float* A, int64_t sAb, int64_t lda,
                                                   const int* __restrict__ only) {
  __shared__ PanelShared<NW, RL> sh;
  const int b = blockIdx.x;
  if (only && only[b] != 1) return;  // this matrix's block was factored elsewhere
  panel_factor<NW, RL>(sh, b, H, sHb, ldh, J0, p, r, kw, tau, sTaub, Tws, sTwb, A, sAb, lda);
}

// Panels 0..nblk-1 of the outer block, one after the other in one workgroup
// per matrix, for the matrices b with only[b] == 1 (the others return at
// once). Panel p + 1 reads V_p, T_p from global memory after the workgroup
// barrier that ends panel p.
template <int NW, int RL>
__global__ __launch_bounds__(64 * NW) void k_panel_seq(float* __restrict__ H, int64_t sHb,
                                                       int64_t ldh, int J0, int nblk, int r,
                                                       float* __restrict__ tau, int64_t sTaub,
                                                       float* __restrict__ Tws, int64_t sTwb,
                                                       const float* A, int64_t sAb, int64_t lda,
                                                       const int* __restrict__ only) {
  __shared__ PanelShared<NW, RL> sh;
  const int b = blockIdx.x;
  if (only[b] != 1) return;
  for (int p = 0; p < nblk; ++p) {
    const int kw = (r - 16 * p) < 16 ? (r - 16 * p) : 16;
    panel_factor<NW, RL>(sh, b, H, sHb, ldh, J0, p, r, kw, tau, sTaub, Tws, sTwb, A, sAb, lda);
    __syncthreads();
  }
}

// Columns c0.. c0+ncols-1 (relative to the outer block at J0, r rows) :=
// Q^T C with the nblk 16-wide reflector blocks of the outer block, applied
// in order 0..nblk-1. C is read from H, or from A (row stride lda, unit column
// stride) when A is not null, and written to H. Each workgroup updates KS adjacent 16-column strips;
// 1-D grid of ngroups * batch workgroups, ngroups = ceil(ncols / (16 KS)),
// group-major within a matrix after the XCD renumbering.
template <int NW, int RL, int KS>
__global__ __launch_bounds__(64 * NW) void k_trail(float* __restrict__ H, int64_t sHb,
                                                   int64_t ldh, int J0, int nblk, int r, int c0,
                                                   int ncols, const float* __restrict__ Tws,
                                                   int64_t sTwb, const float* A, int64_t sAb,
                                                   int64_t lda) {
  __shared__ WyPipeShared<NW, RL, KS> wy;
  const int ngroups = (ncols + 16 * KS - 1) / (16 * KS);
  const int id = xcd_logical_id(blockIdx.x, gridDim.x);
  const int b = id / ngroups;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  float* Blk = H + (int64_t)b * sHb + (int64_t)J0 * ldh + J0;
  const int s0 = 16 * KS * (id - b * ngroups);
  float* P = Blk + c0 + s0;
  const float* Ps = (A ? A + (int64_t)b * sAb + (int64_t)J0 * lda + J0 : Blk) + c0 + s0;
  const int64_t lds = A ? lda : ldh;
  const float* Tb = Tws + (int64_t)b * sTwb;
  auto block = [&](int q) { return VBlock{Blk + (int64_t)(16 * q) * ldh + 16 * q, 16 * q, 16}; };
  // Columns of strip st inside the matrix (<= 0: strip past the last column).
  auto ncol = [&](int st) {
    const int left = ncols - s0 - 16 * st;
    return left < 16 ? left : 16;
  };

  float c[KS][RL];
  VChunk<NW, RL> ck;
#pragma unroll
  for (int st = 0; st < KS; ++st) load_strip<NW, RL>(c[st], Ps + 16 * st, lds, r, ncol(st), w, lane);
  // The strip's loads are issued (and their 64-bit addresses dead) before the
  // first V chunk's: the compiler would otherwise keep every address live at
  // once and spill.
  asm volatile("" ::: "memory");
  load_v_chunk<NW, RL>(ck, block(0), ldh, r, 0, w, lane);
  for (int q = 0; q < nblk; ++q)
    apply_wy16p<NW, RL, KS>(c, ck, block(q), Tb + 256 * q, block(q + 1 < nblk ? q + 1 : q),
                            q + 1 < nblk, ldh, r, wy, w, lane);
#pragma unroll
  for (int st = 0; st < KS; ++st)
    store_strip<NW, RL>(c[st], P + 16 * st, ldh, r, ncol(st), w, lane);
}

hipError_t launch_panel(float* H, int64_t sHb, int64_t ldh, int J0, int p, int r, int kw,
                        float* tau, int64_t sTaub, float* Tws, int64_t sTwb, const float* A,
                        int64_t sAb, int64_t lda, int batch, hipStream_t stream,
                        const int* only) {
  if (kw < 1 || kw > 16 || p < 0 || p >= kMaxBlocks || r > kMaxStripRows || r < 16 * p + kw)
    return hipErrorInvalidValue;
#define QR_PANEL_CASE(NWV, RLV)                                                             \
  hipLaunchKernelGGL((k_panel<NWV, RLV>), dim3(batch), dim3(64 * NWV), 0, stream, H, sHb, ldh, \
                     J0, p, r, kw, tau, sTaub, Tws, sTwb, A, sAb, lda, only)
  // More matrices than CUs (a throughput-bound call): panels of up to 256 rows
  // run 4 waves, so that more of them share a CU. Only for p < 4: panel p's
  // diagonal tile is tile 0 of wave p. With few matrices the 8-wave panel's
  // shorter per-wave work wins.
  if (p < 4 && r <= 256 && batch > device_cu_count()) {
    if (r <= 128)
      QR_PANEL_CASE(4, 8);
    else
      QR_PANEL_CASE(4, 16);
    return hipGetLastError();
  }
  QR_STRIP_DISPATCH(r, QR_PANEL_CASE)
#undef QR_PANEL_CASE
  return hipGetLastError();
}

hipError_t launch_panel_seq(float* H, int64_t sHb, int64_t ldh, int J0, int nblk, int r,
                            float* tau, int64_t sTaub, float* Tws, int64_t sTwb, const float* A,
                            int64_t sAb, int64_t lda, int batch, hipStream_t stream,
                            const int* only) {
  if (!only || nblk < 1 || nblk > kMaxBlocks || r > kMaxStripRows || r < 16 * (nblk - 1) + 1)
    return hipErrorInvalidValue;
#define QR_PANEL_SEQ_CASE(NWV, RLV)                                                            \
  hipLaunchKernelGGL((k_panel_seq<NWV, RLV>), dim3(batch), dim3(64 * NWV), 0, stream, H, sHb, \
                     ldh, J0, nblk, r, tau, sTaub, Tws, sTwb, A, sAb, lda, only)
  QR_STRIP_DISPATCH(r, QR_PANEL_SEQ_CASE)
#undef QR_PANEL_SEQ_CASE
  return hipGetLastError();
}

hipError_t launch_trail(float* H, int64_t sHb, int64_t ldh, int J0, int nblk, int r, int c0,
                        int ncols, const float* Tws, int64_t sTwb, const float* A, int64_t sAb,
                        int64_t lda, int batch, hipStream_t stream) {
  if (ncols <= 0) return hipSuccess;
  if (nblk < 1 || nblk > kMaxBlocks || r > kMaxStripRows || r < 16 * (nblk - 1) + 1)
    return hipErrorInvalidValue;
  if ((int64_t)((ncols + 15) / 16) * batch > INT32_MAX) return hipErrorInvalidValue;
#define QR_TRAIL_CASE(NWV, RLV)                                                                 \
  do {                                                                                          \
    constexpr int KS = TrailKS<NWV, RLV>::value;                                                \
    const dim3 grid((unsigned)((ncols + 16 * KS - 1) / (16 * KS) * (int64_t)batch));           \
    hipLaunchKernelGGL((k_trail<NWV, RLV, KS>), grid, dim3(64 * NWV), 0, stream, H, sHb, ldh,  \
                       J0, nblk, r, c0, ncols, Tws, sTwb, A, sAb, lda);                         \
  } while (0)
#if QR_TRAIL_WIDE
  // 16 waves for strips of more than 256 rows: one wave's V staging latency is
  // covered by the other waves' MFMAs (up to 1024 rows with two strips per
  // workgroup, two workgroups per CU at 257-512 rows).
  if (r > kTrailWideMinRows && r <= 512) {
    QR_TRAIL_CASE(16, 8);
  } else if (r > 512 && r <= 1024) {
    QR_TRAIL_CASE(16, 16);
  } else if (r > 1024 && r <= 2048) {
    QR_TRAIL_CASE(16, 32);
  } else {
    QR_STRIP_DISPATCH(r, QR_TRAIL_CASE)
  }
#else
  QR_STRIP_DISPATCH(r, QR_TRAIL_CASE)
#endif
#undef QR_TRAIL_CASE
  return hipGetLastError();
}

// Workgroups launch_trail would launch for (r, ncols, batch), and how many of
// them the device holds at once (occupancy of that kernel instance times the
// CU count; cached per instance).
hipError_t trail_grid(int r, int ncols, int batch, int64_t* wgs, int64_t* resident) {
  *wgs = 0;
  *resident = 1;
  if (ncols <= 0 || r > kMaxStripRows) return hipSuccess;
  static std::atomic<int> per_cu[16];
  int slot = 0;
  hipError_t e = hipSuccess;
#define QR_TRAIL_GRID_CASE(NWV, RLV)                                                         \
  do {                                                                                       \
    constexpr int KS = TrailKS<NWV, RLV>::value;                                             \
    *wgs = (int64_t)((ncols + 16 * KS - 1) / (16 * KS)) * batch;                            \
    int v = per_cu[slot].load(std::memory_order_relaxed);                                    \
    if (v <= 0) {                                                                            \
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(                                      \
          &v, reinterpret_cast<const void*>(&k_trail<NWV, RLV, KS>), 64 * NWV, 0);           \
      if (e != hipSuccess) return e;                                                         \
      if (v < 1) v = 1;                                                                      \
      per_cu[slot].store(v, std::memory_order_relaxed);                                      \
    }                                                                                        \
    *resident = (int64_t)v * device_cu_count();                                              \
  } while (0)
#if QR_TRAIL_WIDE
  if (r > kTrailWideMinRows && r <= 512) {
    slot = 1;
    QR_TRAIL_GRID_CASE(16, 8);
  } else if (r > 512 && r <= 1024) {
    slot = 2;
    QR_TRAIL_GRID_CASE(16, 16);
  } else if (r > 1024 && r <= 2048) {
    slot = 3;
    QR_TRAIL_GRID_CASE(16, 32);
  } else
#endif
  {
#define QR_TRAIL_GRID_CASE2(NWV, RLV)                                             \
  do {                                                                            \
    slot = 4 + (RLV >= 8) + (RLV >= 16) + (RLV >= 32) + (RLV >= 64) + (NWV == 16 ? 5 : 0); \
    QR_TRAIL_GRID_CASE(NWV, RLV);                                                 \
  } while (0)
    QR_STRIP_DISPATCH(r, QR_TRAIL_GRID_CASE2)
#undef QR_TRAIL_GRID_CASE2
  }
#undef QR_TRAIL_GRID_CASE
  return e;
}

}  // namespace qr
