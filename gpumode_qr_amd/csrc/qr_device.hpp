// qr_device.hpp -- device helpers shared by the gfx950 QR kernels.
//
// Reflector convention (reference: src/qrbench/triton_kernels.py:686-700, made
// LAPACK-slarfg exact): for the column [alpha; x],
//   beta  = -sign(alpha) * hypot(alpha, ||x||),
//   tau   = (beta - alpha) / beta,
//   v     = [1; (x * pre) * gamma],  gamma = 1 / (alpha_s - beta_s),
// and ||x|| == 0 gives tau = 0, beta = alpha with x left untouched. `pre` is the
// power-of-two rescale of slarfg's |beta| < safmin loop (1 on the fast path).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace qr {

// LAPACK slamch('S') / slamch('E') = 2^-126 / 2^-24.
constexpr float kSafmin = 0x1p-102f;
constexpr float kRsafmn = 0x1p102f;
// Fast path is taken when sigma = sum(x^2) was computed without over/underflow
// damage and alpha^2 cannot overflow; then ||x|| = sqrt(sigma) and
// |beta| >= 2^-50 > safmin, so slarfg's rescale loop cannot trigger.
constexpr float kSigmaLo = 0x1p-100f;
constexpr float kSigmaHi = 0x1p100f;
constexpr float kAlphaHi = 0x1p50f;

struct Reflector {
  float beta;   // new diagonal entry R[j][j]
  float tau;    // reflector coefficient
  float gamma;  // v = (x * pre) * gamma below the diagonal
  float pre;    // power-of-two prescale (1 unless slarfg rescaled)
};

__device__ __forceinline__ bool reflector_fast_ok(float alpha, float sigma) {
  return sigma >= kSigmaLo && sigma <= kSigmaHi && fabsf(alpha) <= kAlphaHi;
}

// reflector_fast_ok on the bit patterns (sigma >= +0 as a sum of squares):
// for non-negative floats the bits order like the values, and NaN, Inf and
// -0 fall outside both ranges. On wave-uniform operands these are scalar
// integer instructions, so the per-column check costs no vector issue slots.
__device__ __forceinline__ bool reflector_fast_ok_bits(float alpha, float sigma) {
  constexpr uint32_t lo = 0x0d800000u;  // bits of kSigmaLo = 2^-100
  constexpr uint32_t hi = 0x71800000u;  // bits of kSigmaHi = 2^100
  constexpr uint32_t ahi = 0x58800000u; // bits of kAlphaHi = 2^50
  static_assert(__builtin_bit_cast(uint32_t, kSigmaLo) == lo, "2^-100");
  static_assert(__builtin_bit_cast(uint32_t, kSigmaHi) == hi, "2^100");
  static_assert(__builtin_bit_cast(uint32_t, kAlphaHi) == ahi, "2^50");
  const uint32_t sb = __float_as_uint(sigma);
  const uint32_t ab = __float_as_uint(alpha) & 0x7fffffffu;
  return (sb - lo) <= (hi - lo) && ab <= ahi;
}

// 1/x from v_rcp_f32 plus one Newton step (about 0.5 ulp) for normal x.
__device__ __forceinline__ float rcp_nr(float x) {
  const float r = __builtin_amdgcn_rcpf(x);
  return fmaf(r, fmaf(-x, r, 1.0f), r);
}

// Fast path: sigma = sum(x^2) in [2^-100, 2^100], |alpha| <= 2^50, so every
// operand below is a normal number; v_sqrt_f32 (1 ulp) and rcp_nr replace the
// IEEE divide/sqrt expansions, which sit on the per-column latency chain.
__device__ __forceinline__ Reflector reflector_fast(float alpha, float sigma) {
  Reflector r;
  const float norm = __builtin_amdgcn_sqrtf(fmaf(alpha, alpha, sigma));
  const float beta = -copysignf(norm, alpha);
  r.beta = beta;
  r.tau = (beta - alpha) * rcp_nr(beta);
  r.gamma = rcp_nr(alpha - beta);
  r.pre = 1.0f;
  return r;
}

// Same reflector with plain v_rcp_f32 (1 ulp) for the two reciprocals: two
// dependent instructions fewer on the per-column latency chain.
__device__ __forceinline__ Reflector reflector_fast_rcp(float alpha, float sigma) {
  Reflector r;
  const float norm = __builtin_amdgcn_sqrtf(fmaf(alpha, alpha, sigma));
  const float beta = -copysignf(norm, alpha);
  r.beta = beta;
  r.tau = (beta - alpha) * __builtin_amdgcn_rcpf(beta);
  r.gamma = __builtin_amdgcn_rcpf(alpha - beta);
  r.pre = 1.0f;
  return r;
}

// LAPACK slapy2: sqrt(x^2 + y^2) without destructive over/underflow.
__device__ __forceinline__ float lapy2(float x, float y) {
  const float xa = fabsf(x), ya = fabsf(y);
  const float w = fmaxf(xa, ya), z = fminf(xa, ya);
  if (z == 0.0f || w > 3.402823466e38f) return w;
  const float q = z / w;
  return w * sqrtf(1.0f + q * q);
}

// General path from the scaled norm ||x|| = xmax * sqrt(ssq), where
// ssq = sum((x_i / xmax)^2). Implements slarfg's branches exactly: zero norm,
// the |beta| < safmin rescale loop (at most one pass is ever needed in fp32,
// since |beta| >= 2^-149 and 2^-149 * 2^102 > safmin) and the final unscale.
__device__ __forceinline__ Reflector reflector_scaled(float alpha, float xmax, float ssq) {
  Reflector r;
  const float rt = sqrtf(ssq);
  const float xnorm = xmax * rt;
  if (xnorm == 0.0f) {
    r.beta = alpha;
    r.tau = 0.0f;
    r.gamma = 1.0f;
    r.pre = 1.0f;
    return r;
  }
  float beta = -copysignf(lapy2(alpha, xnorm), alpha);
  float a = alpha;
  float pre = 1.0f;
  int knt = 0;
  while (fabsf(beta) < kSafmin && knt < 20) {
    ++knt;
    pre *= kRsafmn;
    beta *= kRsafmn;
    a *= kRsafmn;
  }
  if (knt > 0) {
    const float xn = (xmax * pre) * rt;
    beta = -copysignf(lapy2(a, xn), a);
  }
  r.tau = (beta - a) / beta;
  r.gamma = 1.0f / (a - beta);
  for (int i = 0; i < knt; ++i) beta *= kSafmin;
  r.beta = beta;
  r.pre = pre;
  return r;
}

// Reflector that leaves everything unchanged (no rows below the diagonal).
__device__ __forceinline__ Reflector reflector_identity(float alpha) {
  Reflector r;
  r.beta = alpha;
  r.tau = 0.0f;
  r.gamma = 1.0f;
  r.pre = 1.0f;
  return r;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Broadcast lane J of each 16-lane DPP row to the whole row (gfx90a+ row_newbcast).
template <int J>
__device__ __forceinline__ float row_bcast16(float v) {
  static_assert(J >= 0 && J < 16, "row_newbcast lane");
  // Every lane reads a lane of its own row, so no "old" value is ever used:
  // mov_dpp with bound_ctrl needs no initialising v_mov.
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + J, 0xF, 0xF, true));
}

// Same broadcast as a volatile asm: the compiler may not merge two uses into
// one live register, so hot loops can re-broadcast instead of holding a copy.
template <int J>
__device__ __forceinline__ float row_bcast16_nocse(float v) {
  static_assert(J >= 0 && J < 16, "row_newbcast lane");
  float out;
  asm volatile("v_mov_b32_dpp %0, %1 row_newbcast:%2 row_mask:0xf bank_mask:0xf"
               : "=v"(out)
               : "v"(v), "i"(J));
  return out;
}

// a_v += x_v[J] * x_v for v < 4, where x_v[J] is x_v in lane J of the lane's
// 16-lane row (DPP row_newbcast folded into v_fmac_f32, which the compiler does
// not form by itself). The compiler's hazard tracking does not look inside
// inline asm, so each block starts with s_nop kNop (kNop + 1 wait states):
// the default 4 covers a VALU write of EXEC (5 wait states before a DPP
// instruction); 1 covers a VALU write of a source register (2), for callers
// with no VALU write of EXEC and no MFMA result read first by these blocks.
template <int J, int kNop = 4>
__device__ __forceinline__ void dot4_bcast16(float& a0, float& a1, float& a2, float& a3, float x0,
                                             float x1, float x2, float x3) {
  static_assert(J >= 0 && J < 16, "row_newbcast lane");
  asm("s_nop %c[nop]\n\t"
      "v_fmac_f32_dpp %0, %4, %4 row_newbcast:%8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %1, %5, %5 row_newbcast:%8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %2, %6, %6 row_newbcast:%8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %3, %7, %7 row_newbcast:%8 row_mask:0xf bank_mask:0xf bound_ctrl:1"
      : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3)
      : "v"(x0), "v"(x1), "v"(x2), "v"(x3), "i"(J), [nop] "i"(kNop));
}

// a_v = x_v[J] * x_v for v < 4: dot4_bcast16's first term, written instead of
// accumulated (no zeroed accumulators needed).
template <int J, int kNop = 4>
__device__ __forceinline__ void dot4_bcast16_first(float& a0, float& a1, float& a2, float& a3,
                                                   float x0, float x1, float x2, float x3) {
  static_assert(J >= 0 && J < 16, "row_newbcast lane");
  asm("s_nop %c[nop]\n\t"
      "v_mul_f32_dpp %0, %4, %4 row_newbcast:%8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_mul_f32_dpp %1, %5, %5 row_newbcast:%8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_mul_f32_dpp %2, %6, %6 row_newbcast:%8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_mul_f32_dpp %3, %7, %7 row_newbcast:%8 row_mask:0xf bank_mask:0xf bound_ctrl:1"
      : "=&v"(a0), "=&v"(a1), "=&v"(a2), "=&v"(a3)
      : "v"(x0), "v"(x1), "v"(x2), "v"(x3), "i"(J), [nop] "i"(kNop));
}

// x_v += x_v[J] * s for v < 4 (same broadcast and wait states as dot4_bcast16).
// Each instruction reads its DPP source before writing it, and no instruction
// reads a register written by the one before it.
template <int J, int kNop = 4>
__device__ __forceinline__ void axpy4_bcast16(float& x0, float& x1, float& x2, float& x3, float s) {
  static_assert(J >= 0 && J < 16, "row_newbcast lane");
  asm("s_nop %c[nop]\n\t"
      "v_fmac_f32_dpp %0, %0, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %1, %1, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %2, %2, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %3, %3, %4 row_newbcast:%5 row_mask:0xf bank_mask:0xf bound_ctrl:1"
      : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3)
      : "v"(s), "i"(J), [nop] "i"(kNop));
}

// Row mask of the 16-lane rows g whose row 4 g + v of a 16-row tile lies below
// row J (4 g + v > J): bit g enables lanes 16 g .. 16 g + 15.
template <int J, int V>
constexpr int rows_below_mask() {
  return (0xF << ((J - V + 4) / 4)) & 0xF;
}

// dot4_bcast16 for the tile that holds row J: a_v += x_v[J] x_v only in the
// rows below row J (rows_below_mask); the other rows keep a_v. DPP's row mask
// gates the destination write, not the source read.
template <int J, int kNop = 4>
__device__ __forceinline__ void dot4_bcast16_below(float& a0, float& a1, float& a2, float& a3,
                                                   float x0, float x1, float x2, float x3) {
  static_assert(J >= 0 && J < 16, "row_newbcast lane");
  asm("s_nop %c[nop]\n\t"
      "v_fmac_f32_dpp %0, %4, %4 row_newbcast:%8 row_mask:%9 bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %1, %5, %5 row_newbcast:%8 row_mask:%10 bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %2, %6, %6 row_newbcast:%8 row_mask:%11 bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %3, %7, %7 row_newbcast:%8 row_mask:%12 bank_mask:0xf bound_ctrl:1"
      : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3)
      : "v"(x0), "v"(x1), "v"(x2), "v"(x3), "i"(J), "i"(rows_below_mask<J, 0>()),
        "i"(rows_below_mask<J, 1>()), "i"(rows_below_mask<J, 2>()),
        "i"(rows_below_mask<J, 3>()), [nop] "i"(kNop));
}

// axpy4_bcast16 for the tile that holds row J: x_v += x_v[J] s only in the rows
// below row J.
template <int J, int kNop = 4>
__device__ __forceinline__ void axpy4_bcast16_below(float& x0, float& x1, float& x2, float& x3,
                                                    float s) {
  static_assert(J >= 0 && J < 16, "row_newbcast lane");
  asm("s_nop %c[nop]\n\t"
      "v_fmac_f32_dpp %0, %0, %4 row_newbcast:%5 row_mask:%6 bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %1, %1, %4 row_newbcast:%5 row_mask:%7 bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %2, %2, %4 row_newbcast:%5 row_mask:%8 bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %3, %3, %4 row_newbcast:%5 row_mask:%9 bank_mask:0xf bound_ctrl:1"
      : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3)
      : "v"(s), "i"(J), "i"(rows_below_mask<J, 0>()), "i"(rows_below_mask<J, 1>()),
        "i"(rows_below_mask<J, 2>()), "i"(rows_below_mask<J, 3>()), [nop] "i"(kNop));
}

// Sum over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float sum_over_rows16(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ float max_over_rows16(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// Sum over the four 16-lane rows with the gfx950 permlane swaps (VALU only,
// no LDS): after permlane32_swap(x, x) the two results hold x[l] and x[l ^ 32]
// in every lane, after permlane16_swap(y, y) y[l] and y[l ^ 16]. Every lane
// ends with the same ((x0 + x2) + (x1 + x3)) for its column.
__device__ __forceinline__ float rows16_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Row group GJ's value (lane k + 16 GJ) in every row group's lane k, by the
// same two swaps without adds: permlane16_swap(x, x) gives [x0, x0, x2, x2]
// and [x1, x1, x3, x3] (16-lane rows), permlane32_swap(y, y) of y = [p, p, q, q]
// gives [p, p, p, p] and [q, q, q, q].
template <int GJ>
__device__ __forceinline__ float rows16_bcast(float x) {
  static_assert(GJ >= 0 && GJ < 4, "row group");
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const unsigned y = (GJ & 1) ? a[1] : a[0];
  const auto b = __builtin_amdgcn_permlane32_swap(y, y, false, false);
  return __uint_as_float((GJ & 2) ? b[1] : b[0]);
}

__device__ __forceinline__ float rows16_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Lane masks of the 16 x 4 strip layout (lane l: column k = l & 15, row group
// g = l >> 4) as compile-time constants. lane_in(mask) is the lane's bit of a
// wave-uniform mask: a select on it reads the mask from an SGPR pair (set by
// scalar moves) instead of a per-lane compare.
constexpr uint64_t lanes_k_gt(int j) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if ((l & 15) > j) m |= uint64_t(1) << l;
  return m;
}
constexpr uint64_t lanes_k_eq(int j) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if ((l & 15) == j) m |= uint64_t(1) << l;
  return m;
}
constexpr uint64_t lanes_k_lt(int j) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if ((l & 15) < j) m |= uint64_t(1) << l;
  return m;
}
constexpr uint64_t lanes_g_eq(int g) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if ((l >> 4) == g) m |= uint64_t(1) << l;
  return m;
}
constexpr uint64_t lanes_g_ge(int g) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if ((l >> 4) >= g) m |= uint64_t(1) << l;
  return m;
}
__device__ __forceinline__ bool lane_in(uint64_t mask) {
  return __builtin_amdgcn_inverse_ballot_w64(mask);
}

// rows16_sum(s) and rows16_bcast<GJ>(x) sharing their swaps: x is masked to
// row group GJ and rides in the other half of the first permlane16_swap, so
// the pairs (s, x) are summed side by side. Every lane ends with
// sum = (s0 + s1) + (s2 + s3) and bcast = x of row group GJ (the other groups
// add zeros). part holds sum in row groups 0 and 2 one swap earlier.
template <int GJ>
__device__ __forceinline__ void rows16_sum_bcast(float s, float x, float& sum, float& bcast,
                                                 float& part) {
  static_assert(GJ >= 0 && GJ < 4, "row group");
  const float xm = lane_in(lanes_g_eq(GJ)) ? x : 0.0f;
  // [s0, x0, s2, x2] and [s1, x1, s3, x3]
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(xm), false,
                                                  false);
  const float c = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  // [c0, c1, c0, c1] and [c2, c3, c2, c3]
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(c), false,
                                                  false);
  const float d = __uint_as_float(b[0]) + __uint_as_float(b[1]);  // [S, X, S, X]
  part = d;
  const auto e = __builtin_amdgcn_permlane16_swap(__float_as_uint(d), __float_as_uint(d), false,
                                                  false);
  sum = __uint_as_float(e[0]);    // [S, S, S, S]
  bcast = __uint_as_float(e[1]);  // [X, X, X, X]
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

}  // namespace qr
