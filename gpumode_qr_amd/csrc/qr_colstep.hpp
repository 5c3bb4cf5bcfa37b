// qr_colstep.hpp -- the column steps of a 16-column panel held in one wave's
// registers, in the MFMA strip layout: shared by the fused small-n kernel (one
// wave per matrix) and the fused mid-n kernel (one wave per 16-column strip).
//
// Layout: lane l has k = l & 15 (column within the strip) and g = l >> 4 (row
// group); cp[4 t + v] = A[16 t + 4 g + v][16 P + k] for the strip's row tiles t.
// Reference for the per-column rules: src/qrbench/triton_kernels.py:684-719.
#pragma once

#include "qr_device.hpp"

namespace qr {

// Wait states before each fused-DPP asm block of the steps: 1 (two wait
// states) is what a DPP source written by the previous VALU instruction needs.
// A kernel that calls the steps writes EXEC with no VALU instruction, and
// reads every MFMA result in the strip with a compiler-visible instruction (a
// store) before the first step reads it.
constexpr int kStepNop = 1;

// Rare path (zero, tiny or huge column, sigma outside [2^-100, 2^100]): the
// exact power-of-two scaled norm ||x|| = 2^ex sqrt(sum (x 2^-ex)^2), with 2^ex >
// max |x| from frexp (no term can overflow or lose its significant bits), then
// slarfg's branches. x0..x15 are this lane's broadcast copies of the pivot
// column's rows (zeros where the panel has fewer row tiles), so the row-group
// reductions give the same value in every lane. Out of line: the code exists
// once instead of once per unrolled column step. Called with all lanes active.
static __device__ __noinline__ Reflector smalln_slow_reflector(
    float alpha, float x0, float x1, float x2, float x3, float x4, float x5, float x6, float x7,
    float x8, float x9, float x10, float x11, float x12, float x13, float x14, float x15) {
  const float x[16] = {x0, x1, x2, x3, x4, x5, x6, x7, x8, x9, x10, x11, x12, x13, x14, x15};
  float xm = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) xm = fmaxf(xm, fabsf(x[i]));
  xm = readlane_f(rows16_max(xm), 0);
  float scale = 0.0f, ssq = 0.0f;
  if (xm > 0.0f) {
    const int ex = __builtin_amdgcn_frexp_expf(xm);
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float q = __builtin_amdgcn_ldexpf(x[i], -ex);
      sq = fmaf(q, q, sq);
    }
    ssq = readlane_f(rows16_sum(sq), 0);
    scale = __builtin_amdgcn_ldexpf(1.0f, ex);
  }
  return reflector_scaled(alpha, scale, ssq);
}

// The same reflector for a taller panel (more than four row tiles): the max
// and the scaled sum of squares over this lane's copies of the pivot column,
// reduced over the row groups, then slarfg's branches out of line.
static __device__ __noinline__ Reflector reflector_scaled_ool(float alpha, float xmax, float ssq) {
  return reflector_scaled(alpha, xmax, ssq);
}

template <int NX>
__device__ __forceinline__ Reflector slow_reflector_tiles(float alpha, const float (&xb)[NX][4]) {
  float xm = 0.0f;
#pragma unroll
  for (int t = 0; t < NX; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) xm = fmaxf(xm, fabsf(xb[t][v]));
  xm = readlane_f(rows16_max(xm), 0);
  float scale = 0.0f, ssq = 0.0f;
  if (xm > 0.0f) {
    const int ex = __builtin_amdgcn_frexp_expf(xm);
    float sq = 0.0f;
#pragma unroll
    for (int t = 0; t < NX; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float q = __builtin_amdgcn_ldexpf(xb[t][v], -ex);
        sq = fmaf(q, q, sq);
      }
    ssq = readlane_f(rows16_sum(sq), 0);
    scale = __builtin_amdgcn_ldexpf(1.0f, ex);
  }
  return reflector_scaled_ool(alpha, scale, ssq);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-panel reflector state of this lane's column (column 16 P + k), and row k
// of the panel's compact-WY factor T (16 x 16, upper triangular). beta and tau,
// needed only when the panel is packed, wait in SmallnShared::refl.
struct SmallnCol {
  float gamma = 1.0f, pre = 1.0f;
  float prev_tau = 0.0f;  // tau of the previous column step
  float trow[16] = {};
};

// Column JQ of T: T[k][JQ] = -tau_JQ sum_{q < JQ} T[k][q] z_q for k < JQ, with
// z_q = V_q^T v_JQ stored in zb[JQ] by the lanes q during column step JQ. Run
// one step later, off that step's critical path, in two parts: the LDS reads
// at the start of step JQ + 1 (LDS operations of one wave are performed in
// program order, so the stores are visible) and the products at its end, so
// that the reads' latency hides behind the step instead of stalling it.
// Exactly the JQ values z_0 .. z_{JQ-1} are read (b128, b64, b32 pieces): a
// register loaded but never used would be reallocated at once, and its write
// would make the wave wait for the read there.
template <int JQ>
struct SmalnTz {
  float z[JQ > 0 ? JQ : 1];
};

template <int JQ, class Sh>
__device__ __forceinline__ void smalln_t_load(SmalnTz<JQ>& tz, const Sh& sh) {
  if constexpr (JQ > 0) {
#pragma unroll
    for (int q4 = 0; q4 < JQ / 4; ++q4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&sh.zb[JQ][4 * q4]);
#pragma unroll
      for (int e = 0; e < 4; ++e) tz.z[4 * q4 + e] = v[e];
    }
    constexpr int q0 = JQ & ~3;
    if constexpr ((JQ & 3) >= 2) {
      const float2 v = *reinterpret_cast<const float2*>(&sh.zb[JQ][q0]);
      tz.z[q0] = v.x;
      tz.z[q0 + 1] = v.y;
    }
    if constexpr (JQ & 1) tz.z[JQ - 1] = sh.zb[JQ][JQ - 1];
  }
}

// Lanes k >= JQ need no select: their entries T[k][q < JQ] are still zero
// (row k of T is upper triangular, and |z_q| <= 64 since no reflector entry
// exceeds 1 in magnitude), so their sum
// is exactly zero and the fma leaves T[k][JQ] (0, or tau_JQ on the diagonal)
// as it was. Lanes k < JQ hold T[k][JQ] = 0 before: the fma is the product.
template <int JQ>
__device__ __forceinline__ void smalln_t_finish(SmallnCol& col, const SmalnTz<JQ>& tz) {
  if constexpr (JQ > 0) {
    float sa = 0.0f, sb = 0.0f;
#pragma unroll
    for (int q = 0; q < JQ; ++q) {
      if (q & 1) sb = fmaf(col.trow[q], tz.z[q], sb);
      else sa = fmaf(col.trow[q], tz.z[q], sa);
    }
    col.trow[JQ] = fmaf(-col.prev_tau, sa + sb, col.trow[JQ]);
  }
}

template <int JQ, class Sh>
__device__ __forceinline__ void smalln_t_column(SmallnCol& col, const Sh& sh) {
  SmalnTz<JQ> tz;
  smalln_t_load<JQ>(tz, sh);
  smalln_t_finish<JQ>(col, tz);
}

// Column step JJ of panel P (column j = 16 P + JJ): reflector of column j and
// its application to the panel's columns j+1.. (lanes k > JJ).
//
// kSafe = false is the hot path: straight-line code, the fast reflector only
// (sigma = sum x^2 in [2^-100, 2^100], |alpha| <= 2^50) plus the identity of a
// column with no rows below the diagonal. A column outside that range clears
// `ok` and leaves garbage; the caller then restores the panel and re-runs it
// with kSafe = true, which takes slarfg's general path (zero, tiny, huge) for
// such columns: v = (x pre) gamma with the power-of-two prescale `pre`.
//
// Lane conditions are compile-time masks (lanes_*), ANDed with kin_mask (the
// lanes whose column exists): selects on them take an SGPR pair, no compare.
// zrow = &sh.zb[0][k] of this lane.
template <int S, int P, int JJ, bool kSafe, bool kFullN = false, class Sh>
__device__ __forceinline__ void smalln_step(float (&cp)[4 * S], Sh& sh, float* zrow, int n,
                                            uint64_t kin_mask, int& bad, SmallnCol& col) {
  constexpr int NT = S - P;  // row tiles at or below the panel's diagonal tile
  constexpr int gj = JJ >> 2, vj = JJ & 3;
  const int j = 16 * P + JJ;
  const bool upd = lane_in(lanes_k_gt(JJ) & kin_mask);
  const bool upd_row_j = lane_in(lanes_k_gt(JJ) & lanes_g_eq(gj) & kin_mask);
  const bool is_jj = lane_in(lanes_k_eq(JJ));
  constexpr int JT = JJ > 0 ? JJ - 1 : 0;  // column of T finished in this step
  SmalnTz<JT> tz;
  if constexpr (JJ > 0) smalln_t_load<JT>(tz, sh);

  // x = column j below the diagonal (rows <= j masked), broadcast from lane JJ
  // of every 16-lane row; partial dot with this lane's column. Rows <= j all
  // lie in tile 0: its masked broadcast is kept for the update. The fast pass
  // reads tiles 1.. straight from lane JJ's registers with the broadcast fused
  // into v_fmac (dot4_bcast16 / axpy4_bcast16); the safe pass keeps them all.
  // Fast pass: tile 0's rows at or above row JJ are left out by the DPP row
  // mask of the fused broadcast (dot4_bcast16_below), not by selects.
  constexpr int NX = kSafe ? NT : 1;
  float xb[NX][4];
  float dv[4];
  if constexpr (!kSafe) {
    // Tiles 1.. first (the first one writes dv, so no zeroing), then tile 0,
    // whose masked rows keep the sum of the others.
    if constexpr (NT >= 2) {
      dot4_bcast16_first<JJ, kStepNop>(dv[0], dv[1], dv[2], dv[3], cp[4 * (P + 1)],
                             cp[4 * (P + 1) + 1], cp[4 * (P + 1) + 2],
                             cp[4 * (P + 1) + 3]);
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) dv[v] = 0.0f;
    }
#pragma unroll
    for (int t = 2; t < NT; ++t)
      dot4_bcast16<JJ, kStepNop>(dv[0], dv[1], dv[2], dv[3], cp[4 * (P + t)],
                               cp[4 * (P + t) + 1], cp[4 * (P + t) + 2],
                               cp[4 * (P + t) + 3]);
    dot4_bcast16_below<JJ, kStepNop>(dv[0], dv[1], dv[2], dv[3], cp[4 * P], cp[4 * P + 1],
                                   cp[4 * P + 2], cp[4 * P + 3]);
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v) dv[v] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if constexpr (!kSafe) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float own = cp[4 * (P + t) + v];
      if (t == 0) own = lane_in(lanes_g_ge((JJ - v + 4) / 4)) ? own : 0.0f;  // 4 g + v > JJ
      xb[t < NX ? t : 0][v] = row_bcast16<JJ>(own);
      dv[v] = fmaf(xb[t < NX ? t : 0][v], cp[4 * (P + t) + v], dv[v]);
    }
  }
  // sigma and alpha, on the per-column critical path, come straight from the
  // four partial dots of lane JJ's row groups and from the lane that holds row
  // j; the per-lane sums over the row groups (needed by every column's update)
  // run beside them.
  const float dsum = (dv[0] + dv[1]) + (dv[2] + dv[3]);
  const float alpha = readlane_f(cp[4 * P + vj], JJ + 16 * gj);
  // ds = x^T c_k summed over the row groups, e = row j of this column.
  float ds, e, dpart;
  rows16_sum_bcast<gj>(dsum, cp[4 * P + vj], ds, e, dpart);
  const float sigma = readlane_f(dpart, JJ);  // lane JJ's dot is x^T x
  // No rows below the diagonal (the last column): tau = 0. When the caller
  // knows the panel is full (kFullN: n = 16 S, or any panel before the last,
  // whose columns all lie before column n - 1 since S = ceil(n / 16)), that
  // is a compile-time fact, which saves the selects of a runtime test in
  // every step (cfg 2: 44.8 -> 43.0 us).
  const bool identity = kFullN ? (16 * P + JJ == 16 * S - 1) : (j >= n - 1);

  Reflector R;
  float wk;
  if constexpr (!kSafe) {
    // Wave-uniform integer flag (a scalar register; a bool here ends up as a
    // per-lane 0/1 value moved back and forth every step).
    bad |= (identity || reflector_fast_ok_bits(alpha, sigma)) ? 0 : 1;
    R = reflector_fast_rcp(alpha, identity ? 1.0f : sigma);
    if (identity) R = reflector_identity(alpha);
    // v^T c_k = c_k[j] + gamma x^T c_k;  c_k -= tau (v^T c_k) v.
    wk = fmaf(R.gamma, ds, e);
    const float cc = R.tau * wk;
    const float ncx = upd ? -(cc * R.gamma) : 0.0f;
    // Tile 0 below row JJ, then tiles 1..: lane JJ (ncx = 0) is never changed,
    // so each broadcast still reads column j's x.
    axpy4_bcast16_below<JJ, kStepNop>(cp[4 * P], cp[4 * P + 1], cp[4 * P + 2],
                                    cp[4 * P + 3], ncx);
#pragma unroll
    for (int t = 1; t < NT; ++t)
      axpy4_bcast16<JJ, kStepNop>(cp[4 * (P + t)], cp[4 * (P + t) + 1],
                                cp[4 * (P + t) + 2], cp[4 * (P + t) + 3], ncx);
    cp[4 * P + vj] = upd_row_j ? cp[4 * P + vj] - cc : cp[4 * P + vj];
  } else {
    bool fast = true;
    if (identity) {
      R = reflector_identity(alpha);
    } else if (reflector_fast_ok(alpha, sigma)) {
      R = reflector_fast(alpha, sigma);
    } else {
      if constexpr (NT <= 4) {
        float xa[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) xa[i] = (i < 4 * NT) ? xb[i / 4][i % 4] : 0.0f;
        R = smalln_slow_reflector(alpha, xa[0], xa[1], xa[2], xa[3], xa[4], xa[5], xa[6], xa[7],
                                  xa[8], xa[9], xa[10], xa[11], xa[12], xa[13], xa[14], xa[15]);
      } else {
        R = slow_reflector_tiles<NT>(alpha, xb);
      }
      fast = false;
    }
    // v^T c_k = c_k[j] + ((x^T c_k) pre) gamma;  c_k -= tau (v^T c_k) v with
    // v = (x pre) gamma. The product pre gamma can overflow (tiny x: pre =
    // 2^102), so it is never formed.
    wk = fmaf(R.gamma, R.pre * ds, e);
    const float cc = R.tau * wk;
    if (fast) {
      const float cx = upd ? cc * R.gamma : 0.0f;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          cp[4 * (P + t) + v] = fmaf(-cx, xb[t][v], cp[4 * (P + t) + v]);
    } else {
      const float cx = upd ? cc : 0.0f;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          cp[4 * (P + t) + v] = fmaf(-cx, (xb[t][v] * R.pre) * R.gamma, cp[4 * (P + t) + v]);
    }
    cp[4 * P + vj] = upd_row_j ? cp[4 * P + vj] - cc : cp[4 * P + vj];
  }
  if constexpr (JJ > 0) {
    // Keep the products here, after the step's own work: hoisted next to
    // their LDS reads, they would make the step wait for those reads first.
    __builtin_amdgcn_sched_barrier(0);
    smalln_t_finish<JT>(col, tz);
  }
  // Column j of T needs z_q = V_q^T v_j = ((c_q[j] + (x^T c_q pre) gamma) pre_q)
  // gamma_q for the panel's q < j (c_q still holds the raw x_q). Every row
  // group stores the same value.
  // (Entries k >= JJ are never read.)
  zrow[16 * JJ] = (wk * col.pre) * col.gamma;
  // -beta and tau are wave-uniform: every lane stores the same pair.
  *reinterpret_cast<float2*>(&sh.refl[JJ][0]) = float2{-R.beta, R.tau};
  col.gamma = is_jj ? R.gamma : col.gamma;
  col.pre = is_jj ? R.pre : col.pre;
  col.trow[JJ] = is_jj ? R.tau : col.trow[JJ];  // T[JJ][JJ] = tau_JJ
  col.prev_tau = R.tau;
}

}  // namespace qr
