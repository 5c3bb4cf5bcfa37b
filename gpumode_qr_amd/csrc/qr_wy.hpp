// qr_wy.hpp -- the strip layout and the compact-WY block-reflector application
// shared by the panel kernel (its left-looking update), the trailing update and
// the Q application (orgqr / ormqr).
//
// Strip layout: NW waves, lane l owns column l & 15; VGPR m = 4t + v holds row
// 16 (t NW + w) + 4 (l >> 4) + v. For a 16-row tile this is exactly the
// accumulator layout of v_mfma_f32_16x16x4_f32 (D[4 (l/16) + v][l % 16]), and
// with the K order {v, v+4, v+8, v+12} it is also the B-operand layout, so
// W = V^T C and C -= V W2 run on MFMA straight from the registers that hold C.
//
// Reference: the trailing GEMMs C -= V (T^T (V^T C)) of the blocked loop,
// src/qrbench/variants.py:800-804.
#pragma once

#include <atomic>

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
// Two at 8 waves: the 512-row panel kernel then needs 38 KB of LDS, so three of
// its workgroups share a CU. The 16-wave kernels stage four, except for strips
// of 2049-4096 rows (RL = 64), which stage two: measured b2 n4096 7.30 -> 7.15
// ms (58 KB of LDS instead of 99 KB, 16 bytes of spills per lane instead of
// 36); at 2048 rows and below two cost more (b64 n1024 2.29 -> 2.37 ms).
#ifndef QR_STAGE_TILES_MAX
#define QR_STAGE_TILES_MAX 2
#endif
template <int NW, int RL>
struct StageTiles {
  static constexpr int kMax = NW >= 16 ? (RL >= 64 ? 2 : 4) : QR_STAGE_TILES_MAX;
  static constexpr int value = (RL / 4) < kMax ? (RL / 4) : kMax;
};


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

// Compute units of the current device (cached per device; 256 if the query
// fails).
inline int device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        v <= 0)
      v = 256;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
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

}  // namespace qr
