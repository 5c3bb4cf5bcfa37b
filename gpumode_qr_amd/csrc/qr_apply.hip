// qr_apply.hip -- Q from (H, tau): the block reflectors of a factorization
// applied to 16-column strips of C (C := Q^T C or Q C, and Q = Q I for orgqr),
// on the compact-WY machinery of the trailing update (qr_wy.hpp).
//
// Reference: the gates build Q with torch.linalg.householder_product and apply
// it by matmul (src/qrbench/checker.py:129-158). In its own source file so that
// its kernel instances do not change the code layout of the factorization's.
#include "qr_wy.hpp"

namespace qr {

// Apply nblk 16-wide reflector blocks (V_q at V + 16 q (ldv + 1) of each matrix,
// T_q at Tws + 256 q) to the 16-column strips of C (r rows, row stride ldc): C :=
// Q^T C with blocks in order 0..nblk-1 (kTrans), or C := Q C with blocks in order
// nblk-1..0, Q = (I - V_0 T_0 V_0^T) ... (I - V_{nblk-1} T_{nblk-1} V^T). 1-D grid
// of nstrips * batch workgroups, XCD-aware like k_trail.
template <int NW, int RL, int KS, bool kTrans>
__global__ __launch_bounds__(64 * NW) void k_apply(const float* __restrict__ V, int64_t sVb,
                                                   int64_t ldv, float* __restrict__ C,
                                                   int64_t sCb, int64_t ldc, int nblk, int r,
                                                   int ncols, const float* __restrict__ Tws,
                                                   int64_t sTwb, int kv_last) {
  __shared__ WyPipeShared<NW, RL, KS> wy;
  const int ngroups = (ncols + 16 * KS - 1) / (16 * KS);
  const int id = xcd_logical_id(blockIdx.x, gridDim.x);
  const int b = id / ngroups;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const float* Vb = V + (int64_t)b * sVb;
  const int s0 = 16 * KS * (id - b * ngroups);
  float* P = C + (int64_t)b * sCb + s0;
  const float* Tb = Tws + (int64_t)b * sTwb;
  auto ncol = [&](int st) {
    const int left = ncols - s0 - 16 * st;
    return left < 16 ? left : 16;
  };
  // i-th block applied: q = i (Q^T C) or nblk - 1 - i (Q C).
  auto block = [&](int i) {
    const int q = kTrans ? i : nblk - 1 - i;
    return VBlock{Vb + (int64_t)(16 * q) * ldv + 16 * q, 16 * q, q == nblk - 1 ? kv_last : 16};
  };

  float c[KS][RL];
  VChunk<NW, RL> ck;
#pragma unroll
  for (int st = 0; st < KS; ++st) load_strip<NW, RL>(c[st], P + 16 * st, ldc, r, ncol(st), w, lane);
  asm volatile("" ::: "memory");  // as in k_trail
  load_v_chunk<NW, RL>(ck, block(0), ldv, r, 0, w, lane);
  for (int i = 0; i < nblk; ++i) {
    const int q = kTrans ? i : nblk - 1 - i;
    apply_wy16p<NW, RL, KS, kTrans>(c, ck, block(i), Tb + 256 * q,
                                    block(i + 1 < nblk ? i + 1 : i), i + 1 < nblk, ldv, r, wy, w,
                                    lane);
  }
#pragma unroll
  for (int st = 0; st < KS; ++st)
    store_strip<NW, RL>(c[st], P + 16 * st, ldc, r, ncol(st), w, lane);
}

hipError_t launch_apply(const float* V, int64_t sVb, int64_t ldv, float* C, int64_t sCb,
                        int64_t ldc, int nblk, int r, int ncols, const float* Tws, int64_t sTwb,
                        bool trans, int kv_last, int batch, hipStream_t stream) {
  if (ncols <= 0) return hipSuccess;
  if (nblk < 1 || nblk > kMaxBlocks || r > kMaxStripRows || kv_last < 1 || kv_last > 16 ||
      r < 16 * (nblk - 1) + kv_last)
    return hipErrorInvalidValue;
  if ((int64_t)((ncols + 15) / 16) * batch > INT32_MAX) return hipErrorInvalidValue;
#define QR_APPLY_CASE(NWV, RLV)                                                                 \
  do {                                                                                          \
    constexpr int KS = TrailKS<NWV, RLV>::value;                                                \
    const dim3 grid((unsigned)((ncols + 16 * KS - 1) / (16 * KS) * (int64_t)batch));           \
    if (trans)                                                                                  \
      hipLaunchKernelGGL((k_apply<NWV, RLV, KS, true>), grid, dim3(64 * NWV), 0, stream, V,    \
                         sVb, ldv, C, sCb, ldc, nblk, r, ncols, Tws, sTwb, kv_last);            \
    else                                                                                        \
      hipLaunchKernelGGL((k_apply<NWV, RLV, KS, false>), grid, dim3(64 * NWV), 0, stream, V,   \
                         sVb, ldv, C, sCb, ldc, nblk, r, ncols, Tws, sTwb, kv_last);            \
  } while (0)
#if QR_TRAIL_WIDE
  // The trailing update's shapes (see launch_trail).
  if (r > kTrailWideMinRows && r <= 512) {
    QR_APPLY_CASE(16, 8);
  } else if (r > 512 && r <= 1024) {
    QR_APPLY_CASE(16, 16);
  } else if (r > 1024 && r <= 2048) {
    QR_APPLY_CASE(16, 32);
  } else {
    QR_STRIP_DISPATCH(r, QR_APPLY_CASE)
  }
#else
  QR_STRIP_DISPATCH(r, QR_APPLY_CASE)
#endif
#undef QR_APPLY_CASE
  return hipGetLastError();
}

}  // namespace qr
