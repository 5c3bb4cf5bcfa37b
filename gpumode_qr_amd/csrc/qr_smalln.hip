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
// workgroup barrier is used, so waves of a workgroup are independent.
#include "qr_device.hpp"

namespace qr {

constexpr int kSnWaves = 4;     // matrices (one per wave) per workgroup
constexpr int kSnVStride = 20;  // row stride of the V transpose buffer (floats)
// Wait states before each fused-DPP asm block of the column steps: 1 (two
// wait states) is what a DPP source written by the previous VALU instruction
// needs. No VALU instruction of this kernel writes EXEC, and a panel's MFMA
// results are first read by the panel's save stores, before any step.
constexpr int kSnNop = 1;

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

// Rare path (zero, tiny or huge column, sigma outside [2^-100, 2^100]): the
// exact power-of-two scaled norm ||x|| = 2^ex sqrt(sum (x 2^-ex)^2), with 2^ex >
// max |x| from frexp (no term can overflow or lose its significant bits), then
// slarfg's branches. x0..x15 are this lane's broadcast copies of the pivot
// column's rows (zeros where the panel has fewer row tiles), so the row-group
// reductions give the same value in every lane. Out of line: the code exists
// once instead of once per unrolled column step. Called with all lanes active.
__device__ __noinline__ Reflector smalln_slow_reflector(
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

template <int S, int JQ>
__device__ __forceinline__ void smalln_t_load(SmalnTz<JQ>& tz, const SmallnShared<S>& sh) {
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

template <int S, int JQ>
__device__ __forceinline__ void smalln_t_column(SmallnCol& col, const SmallnShared<S>& sh) {
  SmalnTz<JQ> tz;
  smalln_t_load<S, JQ>(tz, sh);
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
template <int S, int P, int JJ, bool kSafe, bool kFullN = false>
__device__ __forceinline__ void smalln_step(float (&c)[S][4 * S], SmallnShared<S>& sh,
                                            float* zrow, int n, uint64_t kin_mask, int& bad,
                                            SmallnCol& col) {
  constexpr int NT = S - P;  // row tiles at or below the panel's diagonal tile
  constexpr int gj = JJ >> 2, vj = JJ & 3;
  const int j = 16 * P + JJ;
  const bool upd = lane_in(lanes_k_gt(JJ) & kin_mask);
  const bool upd_row_j = lane_in(lanes_k_gt(JJ) & lanes_g_eq(gj) & kin_mask);
  const bool is_jj = lane_in(lanes_k_eq(JJ));
  constexpr int JT = JJ > 0 ? JJ - 1 : 0;  // column of T finished in this step
  SmalnTz<JT> tz;
  if constexpr (JJ > 0) smalln_t_load<S, JT>(tz, sh);

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
      dot4_bcast16_first<JJ, kSnNop>(dv[0], dv[1], dv[2], dv[3], c[P][4 * (P + 1)],
                             c[P][4 * (P + 1) + 1], c[P][4 * (P + 1) + 2],
                             c[P][4 * (P + 1) + 3]);
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) dv[v] = 0.0f;
    }
#pragma unroll
    for (int t = 2; t < NT; ++t)
      dot4_bcast16<JJ, kSnNop>(dv[0], dv[1], dv[2], dv[3], c[P][4 * (P + t)],
                               c[P][4 * (P + t) + 1], c[P][4 * (P + t) + 2],
                               c[P][4 * (P + t) + 3]);
    dot4_bcast16_below<JJ, kSnNop>(dv[0], dv[1], dv[2], dv[3], c[P][4 * P], c[P][4 * P + 1],
                                   c[P][4 * P + 2], c[P][4 * P + 3]);
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v) dv[v] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if constexpr (!kSafe) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float own = c[P][4 * (P + t) + v];
      if (t == 0) own = lane_in(lanes_g_ge((JJ - v + 4) / 4)) ? own : 0.0f;  // 4 g + v > JJ
      xb[t < NX ? t : 0][v] = row_bcast16<JJ>(own);
      dv[v] = fmaf(xb[t < NX ? t : 0][v], c[P][4 * (P + t) + v], dv[v]);
    }
  }
  // sigma and alpha, on the per-column critical path, come straight from the
  // four partial dots of lane JJ's row groups and from the lane that holds row
  // j; the per-lane sums over the row groups (needed by every column's update)
  // run beside them.
  const float dsum = (dv[0] + dv[1]) + (dv[2] + dv[3]);
  const float alpha = readlane_f(c[P][4 * P + vj], JJ + 16 * gj);
  // ds = x^T c_k summed over the row groups, e = row j of this column.
  float ds, e, dpart;
  rows16_sum_bcast<gj>(dsum, c[P][4 * P + vj], ds, e, dpart);
  const float sigma = readlane_f(dpart, JJ);  // lane JJ's dot is x^T x
  // No rows below the diagonal (the last column): tau = 0. With n = 16 S
  // known (kFullN) that is a compile-time fact, which saves the selects of
  // a runtime test in every step (cfg 2: 44.8 -> 43.0 us).
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
    axpy4_bcast16_below<JJ, kSnNop>(c[P][4 * P], c[P][4 * P + 1], c[P][4 * P + 2],
                                    c[P][4 * P + 3], ncx);
#pragma unroll
    for (int t = 1; t < NT; ++t)
      axpy4_bcast16<JJ, kSnNop>(c[P][4 * (P + t)], c[P][4 * (P + t) + 1],
                                c[P][4 * (P + t) + 2], c[P][4 * (P + t) + 3], ncx);
    c[P][4 * P + vj] = upd_row_j ? c[P][4 * P + vj] - cc : c[P][4 * P + vj];
  } else {
    bool fast = true;
    if (identity) {
      R = reflector_identity(alpha);
    } else if (reflector_fast_ok(alpha, sigma)) {
      R = reflector_fast(alpha, sigma);
    } else {
      float xa[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) xa[i] = (i < 4 * NT) ? xb[i / 4][i % 4] : 0.0f;
      R = smalln_slow_reflector(alpha, xa[0], xa[1], xa[2], xa[3], xa[4], xa[5], xa[6], xa[7],
                                xa[8], xa[9], xa[10], xa[11], xa[12], xa[13], xa[14], xa[15]);
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
          c[P][4 * (P + t) + v] = fmaf(-cx, xb[t][v], c[P][4 * (P + t) + v]);
    } else {
      const float cx = upd ? cc : 0.0f;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          c[P][4 * (P + t) + v] = fmaf(-cx, (xb[t][v] * R.pre) * R.gamma, c[P][4 * (P + t) + v]);
    }
    c[P][4 * P + vj] = upd_row_j ? c[P][4 * P + vj] - cc : c[P][4 * P + vj];
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

template <int S, bool kVec>
// At least two waves per SIMD (<= 256 VGPRs): 2048 matrices fill every SIMD
// twice, and the second wave hides the first one's per-column latency.
__global__ __launch_bounds__(64 * kSnWaves, 2)
__attribute__((amdgpu_waves_per_eu(2, 2))) void k_geqrf_smalln(
    const float* __restrict__ A, int64_t sAb, int64_t sAr, int64_t sAc, float* __restrict__ H,
    float* __restrict__ tau, int batch, int n) {
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
  // address and are replaced by zero, so the 16 S^2 loads issue back to back.
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
        float val = base[roff + coff];
        asm volatile("" : "+v"(val));  // keep the load unconditional
        c[s][4 * t + v] = (row < n && col < n) ? val : 0.0f;
      }
  });
  }

  // Strip s of H, stored as soon as its panel is packed (no later step
  // touches it), so the stores of strips 0 .. S-2 overlap the later panels.
  float* Hb = H + (int64_t)b * n * n + (int64_t)(4 * g) * n + k;
  auto store_strip = [&](auto SI) {
    constexpr int s = decltype(SI)::value;
    if (n == 16 * S) {
#pragma unroll
      for (int t = 0; t < S; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) Hb[(int64_t)(16 * t + v) * n + 16 * s] = c[s][4 * t + v];
    } else {
      int kk = k0, gg = g0;
      asm volatile("" : "+v"(kk), "+v"(gg));
#pragma unroll
      for (int t = 0; t < S; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (16 * t + 4 * gg + v < n && 16 * s + kk < n)
            Hb[(int64_t)(16 * t + v) * n + 16 * s] = c[s][4 * t + v];
    }
  };

  static_for<0, S>([&](auto PI) {
    constexpr int p = decltype(PI)::value;
    constexpr int NT = S - p;  // row tiles at or below the panel's diagonal tile
    const int kw = kVec ? 16 : min(16, n - 16 * p);  // >= 1: S = ceil(n / 16)
    // Lanes whose column exists (wave-uniform mask).
    const uint64_t kin_mask = kVec ? ~uint64_t(0) : __builtin_amdgcn_ballot_w64(k0 < kw);

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
      if (jj < kw) smalln_step<S, p, jj, false, kVec>(c, sh, zrow, n, kin_mask, bad, col);
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
        if (jj < kw) smalln_step<S, p, jj, true>(c, sh, zrow, n, kin_mask, unused, col);
      });
    }
    // The last column of T (the steps compute each column one step late).
    static_for<0, 16>([&](auto JI) {
      constexpr int jq = decltype(JI)::value;
      if (jq == kw - 1) smalln_t_column<S, jq>(col, sh);
    });
    const float2 rf = *reinterpret_cast<const float2*>(&sh.refl[k][0]);
    const bool kin = k < kw;
    const float my_beta = kin ? -rf.x : 0.0f, my_tau = kin ? rf.y : 0.0f;
    const float my_gamma = col.gamma, my_pre = col.pre;

    if (g == 0 && kin) tau[(int64_t)b * n + 16 * p + k] = my_tau;

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

// Host-side dispatch over the number of 16-column strips. H is (batch, n, n)
// contiguous and tau (batch, n) contiguous.
hipError_t launch_geqrf_smalln(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                               float* tau, int batch, int n, hipStream_t stream) {
  if (n < 1 || n > 64 || batch < 1) return hipErrorInvalidValue;
  const dim3 grid((batch + kSnWaves - 1) / kSnWaves), block(64 * kSnWaves);
  const bool vec = n == 64 && sAc == 1 && (sAr % 4) == 0 && (sAb % 4) == 0 &&
                   (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  if (vec) {
    hipLaunchKernelGGL((k_geqrf_smalln<4, true>), grid, block, 0, stream, A, sAb, sAr, sAc, H,
                       tau, batch, n);
    return hipGetLastError();
  }
#define QR_SMALLN_CASE(SV)                                                                  \
  case SV:                                                                                  \
    hipLaunchKernelGGL((k_geqrf_smalln<SV, false>), grid, block, 0, stream, A, sAb, sAr, sAc, \
                       H, tau, batch, n);                                                   \
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
  return hipGetLastError();
}

}  // namespace qr
