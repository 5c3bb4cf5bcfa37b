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
// Strip layout (shared by both kernels): NW waves, lane l owns column l & 15;
// VGPR m = 4t + v holds row 16 (t NW + w) + 4 (l >> 4) + v. For a 16-row tile
// this is exactly the accumulator layout of v_mfma_f32_16x16x4_f32
// (D[4 (l/16) + v][l % 16]), and with the K order {v, v+4, v+8, v+12} it is also
// the B-operand layout, so W = V^T C and C -= V W2 run on MFMA straight from the
// registers that hold C.
#include "qr_device.hpp"

namespace qr {

template <int NW, int RL>
struct Strip {
  static_assert(RL % 4 == 0, "RL must be a multiple of 4");
  static constexpr int kTiles = RL / 4;
  static constexpr int kRows = 4 * NW * RL;
  __device__ static __forceinline__ int row(int t, int v, int w, int g) {
    return 16 * (t * NW + w) + 4 * g + v;
  }
  __device__ static __forceinline__ int tile_row0(int t, int w) { return 16 * (t * NW + w); }
};

// Row stride (floats) of the V tiles staged in LDS: 20 keeps both the b32 reads
// of the W phase and the b128 reads of the update phase free of bank conflicts.
constexpr int kVStride = 20;

// 16-row tiles of V staged per wave at a time (LDS budget: NW * tiles * 1.25 KB).
#ifndef QR_STAGE_TILES_MAX
#define QR_STAGE_TILES_MAX 8
#endif
template <int NW, int RL>
struct StageTiles {
  static constexpr int kMax = NW >= 16 ? 4 : QR_STAGE_TILES_MAX;
  static constexpr int value = (RL / 4) < kMax ? (RL / 4) : kMax;
};


// Element (i, col) of the unit lower-trapezoidal block V stored in place at P
// with rows 0..rv-1; i may be negative (rows above the block are zero).
__device__ __forceinline__ float v_elem(const float* __restrict__ P, int64_t ldh, int i, int col,
                                        int rv) {
  if (i < col || i >= rv) return 0.0f;
  if (i == col) return 1.0f;
  return P[(int64_t)i * ldh + col];
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// Compact-WY application of a sequence of 16-wide reflector blocks to a strip.
//
// * Each wave stages its own rows of V_q through LDS in chunks of kStageTiles
//   16-row tiles (row stride kVStride): the W phase reads them as b32 in the
//   A-operand layout, the update phase as b128 rows. Each chunk is loaded
//   from HBM into registers (VChunk) one stage ahead: the loads of the next
//   chunk, and at the end of a block those of the next block's first chunk, are
//   in flight while the MFMAs of the current chunk run.
// * The cross-wave reduction of W = V^T c takes two workgroup barriers: every
//   wave writes its 16 x 16 partial as one b128 per lane (the MFMA accumulator
//   layout, which is also the B-operand layout with K order {v, v+4, v+8,
//   v+12}), 256 threads sum them, and every wave forms W2 = T^T W (or T W)
//   from the sum with four MFMAs whose accumulator is exactly the operand of
//   the update. No barrier is needed after the update: a wave writes the next
//   partial only after the second barrier, when the sums have been read, and
//   the next sum only after the next first barrier, when every wave has read W.
// ---------------------------------------------------------------------------

// This wave's part of one V chunk, in registers: lane l holds row l/4, columns
// 4(l%4)..+3 of each of the chunk's tiles.
template <int NW, int RL>
struct VChunk {
  f32x4 t[StageTiles<NW, RL>::value];
};

// A reflector block: V_q at Vq (its row 0 is strip row q16), kv columns.
struct VBlock {
  const float* V;
  int q16;
  int kv;
};

// LDS of apply_wy16p for KS strips: per-wave V chunks, the NW partial W's of
// each strip and their sums.
template <int NW, int RL, int KS = 1>
struct WyPipeShared {
  float vbuf[NW][StageTiles<NW, RL>::value * 16 * kVStride];
  alignas(16) float red[KS][NW][64 * 4];
  alignas(16) float wsum[KS][64 * 4];
};

// Global loads of this wave's tiles [t0, t0 + kStageTiles) of block B: rows
// above V's diagonal and rows >= r are zero, the diagonal is 1, columns >= kv
// (a block narrower than 16 at the matrix edge) are zero and not read.
template <int NW, int RL>
__device__ __forceinline__ void load_v_chunk(VChunk<NW, RL>& ck, const VBlock& B, int64_t ldh,
                                             int r, int t0, int w, int lane) {
  constexpr int kStageTiles = StageTiles<NW, RL>::value;
  const int lr = lane >> 2, lc = 4 * (lane & 3);
  const bool vec4 = ((ldh & 3) == 0) && ((reinterpret_cast<uintptr_t>(B.V) & 15) == 0);
#pragma unroll
  for (int tt = 0; tt < kStageTiles; ++tt) {
    const int t = t0 + tt;
    f32x4 val = {0.0f, 0.0f, 0.0f, 0.0f};
    if (t < RL / 4) {
      const int r0 = 16 * (t * NW + w);
      const int i = r0 + lr - B.q16;  // row within V_q
      if (i >= 0 && r0 + lr < r) {
        const float* src = B.V + (int64_t)i * ldh + lc;
        if (vec4 && lc + 4 <= B.kv) {
          val = *reinterpret_cast<const f32x4*>(src);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) val[e] = (lc + e < B.kv) ? src[e] : 0.0f;
        }
        if (i < 16) {  // diagonal tile: unit lower-triangular mask
#pragma unroll
          for (int e = 0; e < 4; ++e)
            val[e] = (lc + e > i) ? 0.0f : ((lc + e == i) ? 1.0f : val[e]);
        }
      }
    }
    ck.t[tt] = val;
  }
}

template <int NW, int RL>
__device__ __forceinline__ void put_v_chunk(float* __restrict__ vb, const VChunk<NW, RL>& ck,
                                            int lane) {
  constexpr int kStageTiles = StageTiles<NW, RL>::value;
  const int lr = lane >> 2, lc = 4 * (lane & 3);
#pragma unroll
  for (int tt = 0; tt < kStageTiles; ++tt)
    *reinterpret_cast<f32x4*>(&vb[(tt * 16 + lr) * kVStride + lc]) = ck.t[tt];
}

// c[s] := (I - V T V^T)^T c[s] (kTransT) or (I - V T V^T) c[s], s < KS, for
// block B with factor Tq: KS 16-column strips share every V read and every
// barrier. On entry ck holds B's first chunk (from load_v_chunk); on return it
// holds the first chunk of Bn if has_next.
// Two workgroup barriers; every thread of the workgroup must call it.
template <int NW, int RL, int KS, bool kTransT = true>
__device__ __forceinline__ void apply_wy16p(float (&c)[KS][RL], VChunk<NW, RL>& ck,
                                            const VBlock& B, const float* __restrict__ Tq,
                                            const VBlock& Bn, bool has_next, int64_t ldh, int r,
                                            WyPipeShared<NW, RL, KS>& sh, int w, int lane) {
  using S = Strip<NW, RL>;
  constexpr int kStageTiles = StageTiles<NW, RL>::value;
  constexpr int kChunks = (S::kTiles + kStageTiles - 1) / kStageTiles;
  const int ii = lane & 15, kk = lane >> 4;
  float* vb = sh.vbuf[w];

  // T in the A-operand layout of the W2 product: lane (ii, kk), K step v holds
  // T[4 kk + v][ii] (W2 = T^T W) or T[ii][4 kk + v] (W2 = T W).
  float ta[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int q = 4 * kk + v;  // only the upper triangle of T is read
    ta[v] = kTransT ? ((q <= ii) ? Tq[q * 16 + ii] : 0.0f) : ((ii <= q) ? Tq[ii * 16 + q] : 0.0f);
  }

  // W (16 x 16 per strip) = V^T c, partial over this wave's rows.
  f32x4 accw[KS];
#pragma unroll
  for (int st = 0; st < KS; ++st) accw[st] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ch = 0; ch < kChunks; ++ch) {
    if (ch > 0) wave_sync();  // the previous chunk's LDS reads are done
    put_v_chunk<NW, RL>(vb, ck, lane);
    wave_sync();
    // Next chunk to stage: the W phase runs chunks 0..kChunks-1, the update
    // phase kChunks-1 (still in LDS) down to 0, then the next block's chunk 0.
    if (ch + 1 < kChunks)
      load_v_chunk<NW, RL>(ck, B, ldh, r, (ch + 1) * kStageTiles, w, lane);
    else if (kChunks >= 2)
      load_v_chunk<NW, RL>(ck, B, ldh, r, (kChunks - 2) * kStageTiles, w, lane);
    else if (has_next)
      load_v_chunk<NW, RL>(ck, Bn, ldh, r, 0, w, lane);
#pragma unroll
    for (int tt = 0; tt < kStageTiles; ++tt) {
      const int t = ch * kStageTiles + tt;
      if (t >= S::kTiles) break;  // compile-time
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float av = vb[(tt * 16 + 4 * kk + v) * kVStride + ii];
#pragma unroll
        for (int st = 0; st < KS; ++st)
          accw[st] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, c[st][4 * t + v], accw[st], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int st = 0; st < KS; ++st) *reinterpret_cast<f32x4*>(&sh.red[st][w][4 * lane]) = accw[st];
  __syncthreads();
  // Each of the first 256 KS threads sums the NW partials of one element
  // (consecutive addresses: no bank conflicts); then every wave reads W back in
  // the B-operand layout (lane (j, g), K step v: W[4 g + v][j]).
  static_assert(KS * 256 <= 64 * NW, "one summing thread per element of W");
  if (threadIdx.x < KS * 256) {
    const int st = KS == 1 ? 0 : threadIdx.x >> 8, el = threadIdx.x & 255;
    float sum = sh.red[st][0][el];
#pragma unroll
    for (int u = 1; u < NW; ++u) sum += sh.red[st][u][el];
    sh.wsum[st][el] = sum;
  }
  __syncthreads();
  // W2 in the accumulator layout: lane (ii, kk) holds W2[4 kk + s][ii] in w2[.][s].
  f32x4 w2[KS];
#pragma unroll
  for (int st = 0; st < KS; ++st) {
    const f32x4 ws = *reinterpret_cast<const f32x4*>(&sh.wsum[st][4 * lane]);
    w2[st] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int v = 0; v < 4; ++v)
      w2[st] = __builtin_amdgcn_mfma_f32_16x16x4f32(ta[v], ws[v], w2[st], 0, 0, 0);
  }

  // c -= V W2, K order permuted so that lane (ii, kk) reads V[row ii][4kk..4kk+3]
  // as one b128 and uses W2[4kk + s][ii] = w2[.][s].
#pragma unroll
  for (int ch = kChunks - 1; ch >= 0; --ch) {
    if (ch != kChunks - 1) {
      wave_sync();
      put_v_chunk<NW, RL>(vb, ck, lane);
      wave_sync();
      if (ch >= 1)
        load_v_chunk<NW, RL>(ck, B, ldh, r, (ch - 1) * kStageTiles, w, lane);
      else if (has_next)
        load_v_chunk<NW, RL>(ck, Bn, ldh, r, 0, w, lane);
    }
#pragma unroll
    for (int tt = 0; tt < kStageTiles; ++tt) {
      const int t = ch * kStageTiles + tt;
      if (t >= S::kTiles) break;  // compile-time
      const f32x4 a4 = *reinterpret_cast<const f32x4*>(&vb[(tt * 16 + ii) * kVStride + 4 * kk]);
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        f32x4 acc = {c[st][4 * t], c[st][4 * t + 1], c[st][4 * t + 2], c[st][4 * t + 3]};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(-a4[q], w2[st][q], acc, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; ++v) c[st][4 * t + v] = acc[v];
      }
    }
  }
  wave_sync();  // this wave's LDS chunk is rewritten by the next call
}

template <int NW, int RL>
__device__ __forceinline__ void load_strip(float (&c)[RL], const float* __restrict__ P,
                                           int64_t ldh, int r, int ncol, int w, int lane) {
  using S = Strip<NW, RL>;
  const int k = lane & 15, g = lane >> 4;
  const bool colok = k < ncol;
  const float* src = P + (int64_t)(16 * w + 4 * g) * ldh + k;
  const int64_t tstep = (int64_t)16 * NW * ldh;
#pragma unroll
  for (int t = 0; t < S::kTiles; ++t) {
    const int r0 = S::tile_row0(t, w);
    if (r0 + 16 <= r) {  // whole tile inside (uniform)
#pragma unroll
      for (int v = 0; v < 4; ++v) c[4 * t + v] = colok ? src[v * ldh] : 0.0f;
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        c[4 * t + v] = (colok && r0 + 4 * g + v < r) ? src[v * ldh] : 0.0f;
    }
    src += tstep;
  }
}

template <int NW, int RL>
__device__ __forceinline__ void store_strip(const float (&c)[RL], float* __restrict__ P,
                                            int64_t ldh, int r, int ncol, int w, int lane) {
  using S = Strip<NW, RL>;
  const int k = lane & 15, g = lane >> 4;
  const bool colok = k < ncol;
  float* dst = P + (int64_t)(16 * w + 4 * g) * ldh + k;
  const int64_t tstep = (int64_t)16 * NW * ldh;
#pragma unroll
  for (int t = 0; t < S::kTiles; ++t) {
    const int r0 = S::tile_row0(t, w);
    if (r0 >= r) break;
    if (r0 + 16 <= r) {  // whole tile inside (uniform)
      if (colok) {
#pragma unroll
        for (int v = 0; v < 4; ++v) dst[v * ldh] = c[4 * t + v];
      }
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (colok && r0 + 4 * g + v < r) dst[v * ldh] = c[4 * t + v];
    }
    dst += tstep;
  }
}

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

// Fast pass over the kw column steps of the panel whose diagonal rows
// 16p..16p+15 are tile 0 of wave p. The steps are unrolled, and x (column J
// below the diagonal) is read straight from the registers of lane J of each
// 16-lane row by DPP row_newbcast, folded into the v_fmac of the dot and of
// the update: no LDS traffic for x and one workgroup barrier per step.
// Returns false, with c and st meaningless, if some column was outside the
// fast reflector's range (zero, tiny or huge norm); the result is then to be
// recomputed by panel_general_pass.
template <int NW, int RL>
__device__ __forceinline__ bool panel_fast_pass(float (&c)[RL], PanelShared<NW, RL>& sh, int p,
                                                int r, int kw, int w, int lane, PanelCol& st) {
  using S = Strip<NW, RL>;
  const int k = lane & 15, g = lane >> 4;
  const int d0 = 16 * p;
  bool ok = true;
  static_for<0, 16>([&](auto jc) __attribute__((always_inline)) {
    constexpr int J = decltype(jc)::value;
    if (J >= kw) return;
    const int dj = d0 + J;
    if (w == p && g == (J >> 2)) sh.erow[J & 1][k] = c[J & 3];
    // Rows <= dj (where x is zero) all lie in tile 0.
    float dv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float xb = row_bcast16<J>(c[v]);
      dv[v] = ((S::row(0, v, w, g) > dj) ? xb : 0.0f) * c[v];
    }
#pragma unroll
    for (int t = 1; t < S::kTiles; ++t)
      dot4_bcast16<J>(dv[0], dv[1], dv[2], dv[3], c[4 * t], c[4 * t + 1], c[4 * t + 2],
                      c[4 * t + 3]);
    sh.red[J & 1][k][4 * w + g] = (dv[0] + dv[1]) + (dv[2] + dv[3]);
    __syncthreads();
    const float ds = panel_dot_sum<NW>(sh.red[J & 1][k]);
    const float e = sh.erow[J & 1][k];
    const float sigma = readlane_f(ds, J);
    const float alpha = readlane_f(e, J);
    const bool ident = dj >= r - 1;  // no rows below the diagonal
    ok = ok && (ident || reflector_fast_ok(alpha, sigma));
    Reflector R = reflector_fast_rcp(alpha, sigma);
    if (ident) R = reflector_identity(alpha);
    const float wk = fmaf(R.gamma, ds, e);  // v_J^T c_k
    const float cc = R.tau * wk;
    const bool upd = (k > J) && (k < kw);
    const float ncx = upd ? -(cc * R.gamma) : 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float xb = row_bcast16<J>(c[v]);
      c[v] = fmaf(ncx, (S::row(0, v, w, g) > dj) ? xb : 0.0f, c[v]);
    }
#pragma unroll
    for (int t = 1; t < S::kTiles; ++t)
      axpy4_bcast16<J>(c[4 * t], c[4 * t + 1], c[4 * t + 2], c[4 * t + 3], ncx);
    if (upd && w == p && g == (J >> 2)) c[J & 3] -= cc;  // v_J[dj] = 1
    // Column J of T needs z_k = V_k^T v_J = (c_k[dj] + gamma x^T c_k) gamma_k, k < J.
    if (w == 0 && g == 0 && k < J) sh.zbuf[J][k] = wk * st.gamma;
    if (k == J) {
      st.beta = R.beta;
      st.gamma = R.gamma;
      st.pre = 1.0f;
      st.tau = R.tau;
    }
  });
  return ok;
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

// c := panel p (kw columns at Blk + 16 p, r rows, strip layout) after the
// left-looking update with panels 0..p-1 of the outer block at Blk.
template <int NW, int RL>
__device__ __forceinline__ void panel_load_apply(float (&c)[1][RL], const float* __restrict__ Blk,
                                                 int64_t ldh, int p, int r, int kw,
                                                 const float* __restrict__ Tb,
                                                 WyPipeShared<NW, RL>& wy, int w, int lane) {
  auto block = [&](int q) { return VBlock{Blk + (int64_t)(16 * q) * ldh + 16 * q, 16 * q, 16}; };
  VChunk<NW, RL> ck;
  if (p > 0) load_v_chunk<NW, RL>(ck, block(0), ldh, r, 0, w, lane);
  load_strip<NW, RL>(c[0], Blk + 16 * p, ldh, r, kw, w, lane);
  for (int q = 0; q < p; ++q)
    apply_wy16p<NW, RL, 1>(c, ck, block(q), Tb + 256 * q, block(q + 1 < p ? q + 1 : q), q + 1 < p,
                           ldh, r, wy, w, lane);
}

// The fast pass can be switched off (every panel then takes the general pass).
#ifndef QR_PANEL_FAST
#define QR_PANEL_FAST 1
#endif
constexpr bool kPanelFastPass = QR_PANEL_FAST != 0;

// Factor panel p (columns 16p..16p+kw-1 of the outer block whose top-left is
// Blk, r rows) after applying panels 0..p-1 of the block (their T's at Tb).
// Writes V_p / R in place, tau_p, and T_p at Tb + 256 p.
template <int NW, int RL>
__global__ __launch_bounds__(64 * NW) void k_panel(float* __restrict__ H, int64_t sHb,
                                                   int64_t ldh, int J0, int p, int r, int kw,
                                                   float* __restrict__ tau, int64_t sTaub,
                                                   float* __restrict__ Tws, int64_t sTwb) {
  using S = Strip<NW, RL>;
  __shared__ PanelShared<NW, RL> sh;

  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int k = lane & 15, g = lane >> 4;
  float* Blk = H + (int64_t)b * sHb + (int64_t)J0 * ldh + J0;
  float* P = Blk + 16 * p;
  float* Tb = Tws + (int64_t)b * sTwb;

  // The panel after the left-looking update with panels 0..p-1; the panel in
  // HBM is not written before the end, so the general pass can start over.
  float cs[1][RL];
  float (&c)[RL] = cs[0];
  panel_load_apply<NW, RL>(cs, Blk, ldh, p, r, kw, Tb, sh.wy, w, lane);

  PanelCol st;
  bool ok = false;
  if constexpr (kPanelFastPass) ok = panel_fast_pass<NW, RL>(c, sh, p, r, kw, w, lane, st);
  if (!ok) [[unlikely]] {
    if constexpr (kPanelFastPass) {
      __syncthreads();  // every wave is past its last read of erow / red
      panel_load_apply<NW, RL>(cs, Blk, ldh, p, r, kw, Tb, sh.wy, w, lane);
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
  if (w != 0) return;
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

// The dispatcher hands workgroup i to XCD i mod kXcds, and each XCD has its
// own L2. Renumber so that each XCD receives a contiguous range of logical
// ids, in dispatch order: the strips of one matrix then run on one XCD, close
// in time, and share its V block and the 128-byte lines of neighbouring
// strips through that L2 instead of fetching them once per XCD.
constexpr int kXcds = 8;

__device__ __forceinline__ int xcd_logical_id(int id, int total) {
  const int xcd = id % kXcds, slot = id / kXcds;
  const int q = total / kXcds, rem = total % kXcds;
  return xcd * q + (xcd < rem ? xcd : rem) + slot;
}

// Columns c0.. c0+ncols-1 (relative to the outer block at J0, r rows) :=
// Q^T C with the nblk 16-wide reflector blocks of the outer block, applied
// in order 0..nblk-1. Each workgroup updates KS adjacent 16-column strips;
// 1-D grid of ngroups * batch workgroups, ngroups = ceil(ncols / (16 KS)),
// group-major within a matrix after the XCD renumbering.
template <int NW, int RL, int KS>
__global__ __launch_bounds__(64 * NW) void k_trail(float* __restrict__ H, int64_t sHb,
                                                   int64_t ldh, int J0, int nblk, int r, int c0,
                                                   int ncols, const float* __restrict__ Tws,
                                                   int64_t sTwb) {
  __shared__ WyPipeShared<NW, RL, KS> wy;
  const int ngroups = (ncols + 16 * KS - 1) / (16 * KS);
  const int id = xcd_logical_id(blockIdx.x, gridDim.x);
  const int b = id / ngroups;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  float* Blk = H + (int64_t)b * sHb + (int64_t)J0 * ldh + J0;
  const int s0 = 16 * KS * (id - b * ngroups);
  float* P = Blk + c0 + s0;
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
  for (int st = 0; st < KS; ++st) load_strip<NW, RL>(c[st], P + 16 * st, ldh, r, ncol(st), w, lane);
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

// Strips per workgroup of the trailing update / Q application: two for the
// 16-wave workgroups of up to 1024 rows (a wave's share of two strips fits
// the 128-VGPR budget of 4 waves per SIMD), else one. Eight-wave workgroups
// (r <= 512) keep one strip: there the lower register count buys a third
// resident workgroup per CU, which measured faster.
#ifndef QR_TRAIL_KS_MAX
#define QR_TRAIL_KS_MAX 2
#endif
template <int NW, int RL>
struct TrailKS {
  static constexpr int value = (NW >= 16 && RL <= 16 && QR_TRAIL_KS_MAX >= 2) ? 2 : 1;
};

// (NW, RL) for r rows: 4 NW RL >= r and NW > p for every panel index used.
#define QR_STRIP_DISPATCH(r, CASE)   \
  if ((r) <= 128) {                  \
    CASE(8, 4);                      \
  } else if ((r) <= 256) {           \
    CASE(8, 8);                      \
  } else if ((r) <= 512) {           \
    CASE(8, 16);                     \
  } else if ((r) <= 1024) {          \
    CASE(8, 32);                     \
  } else if ((r) <= 2048) {          \
    CASE(8, 64);                     \
  } else {                           \
    CASE(16, 64);                    \
  }

constexpr int kMaxStripRows = 4096;
#ifndef QR_TRAIL_WIDE
#define QR_TRAIL_WIDE 1
#endif
#ifndef QR_TRAIL_WIDE_MIN_ROWS
#define QR_TRAIL_WIDE_MIN_ROWS 256
#endif
constexpr int kTrailWideMinRows = QR_TRAIL_WIDE_MIN_ROWS;
constexpr int kMaxBlocks = 8;

hipError_t launch_panel(float* H, int64_t sHb, int64_t ldh, int J0, int p, int r, int kw,
                        float* tau, int64_t sTaub, float* Tws, int64_t sTwb, int batch,
                        hipStream_t stream) {
  if (kw < 1 || kw > 16 || p < 0 || p >= kMaxBlocks || r > kMaxStripRows || r < 16 * p + kw)
    return hipErrorInvalidValue;
#define QR_PANEL_CASE(NWV, RLV)                                                             \
  hipLaunchKernelGGL((k_panel<NWV, RLV>), dim3(batch), dim3(64 * NWV), 0, stream, H, sHb, ldh, \
                     J0, p, r, kw, tau, sTaub, Tws, sTwb)
  QR_STRIP_DISPATCH(r, QR_PANEL_CASE)
#undef QR_PANEL_CASE
  return hipGetLastError();
}

hipError_t launch_trail(float* H, int64_t sHb, int64_t ldh, int J0, int nblk, int r, int c0,
                        int ncols, const float* Tws, int64_t sTwb, int batch,
                        hipStream_t stream) {
  if (ncols <= 0) return hipSuccess;
  if (nblk < 1 || nblk > kMaxBlocks || r > kMaxStripRows || r < 16 * (nblk - 1) + 1)
    return hipErrorInvalidValue;
  if ((int64_t)((ncols + 15) / 16) * batch > INT32_MAX) return hipErrorInvalidValue;
#define QR_TRAIL_CASE(NWV, RLV)                                                                 \
  do {                                                                                          \
    constexpr int KS = TrailKS<NWV, RLV>::value;                                                \
    const dim3 grid((unsigned)((ncols + 16 * KS - 1) / (16 * KS) * (int64_t)batch));           \
    hipLaunchKernelGGL((k_trail<NWV, RLV, KS>), grid, dim3(64 * NWV), 0, stream, H, sHb, ldh,  \
                       J0, nblk, r, c0, ncols, Tws, sTwb);                                      \
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
  QR_STRIP_DISPATCH(r, QR_APPLY_CASE)
#undef QR_APPLY_CASE
  return hipGetLastError();
}

}  // namespace qr
