// qr_api.hip -- the C ABI of libqr_gfx950.so (include/qr_gfx950.h), the
// blocked factorisation driver, and per-launch event tracing.
//
// Driver (reference: _hh_panel_blocked_qr, src/qrbench/variants.py:761-805, and
// the n <= 128 fused route of make_hh_fused_smalln, :739-758):
//   n <= 64 : one launch of the fused small-n kernel (A -> H directly).
//   n >  64 : copy A -> H, then for each outer block of P 16-wide panels at
//             column J0: P panel launches (panel p first applies panels 0..p-1
//             of the block to its columns, then factors them; V and tau in
//             place, T_p to the workspace), then one trailing launch that
//             applies the P block reflectors to every column right of the block.
// Everything is enqueued on the caller's stream; nothing synchronises except
// qr_trace_read, which waits for the events it reads.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <mutex>
#include <vector>

#include "../../include/qr_gfx950.h"

namespace qr {
hipError_t launch_geqrf_smalln(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                               int64_t sHb, int64_t ldh, float* tau, int64_t sTaub, int batch,
                               int n, hipStream_t stream);
hipError_t launch_geqrf_midn(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                             int64_t sHb, int64_t ldh, float* tau, int64_t sTaub, int batch,
                             int n, hipStream_t stream);
int midn_max_n();
hipError_t launch_panel(float* H, int64_t sHb, int64_t ldh, int J0, int p, int r, int kw,
                        float* tau, int64_t sTaub, float* Tws, int64_t sTwb, const float* A,
                        int64_t sAb, int64_t lda, int batch, hipStream_t stream,
                        const int* only);
hipError_t launch_panel_seq(float* H, int64_t sHb, int64_t ldh, int J0, int nblk, int r,
                            float* tau, int64_t sTaub, float* Tws, int64_t sTwb, const float* A,
                            int64_t sAb, int64_t lda, int batch, hipStream_t stream,
                            const int* only);
size_t cq_workspace_floats(int batch);
hipError_t launch_cq_block(const float* Src, int64_t sSb, int64_t lds, float* Hb, int64_t sHb,
                           int64_t ldh, int r, float* tau, int64_t sTaub, float* Tws,
                           int64_t sTwb, float* ws, int batch, bool fused, int one_pass,
                           hipStream_t stream);
const int* cq_flags(float* ws, int batch);
size_t cq_flags_offset_floats(int batch);
hipError_t launch_cq_reset(float* ws, int batch, hipStream_t stream);
hipError_t launch_trail(float* H, int64_t sHb, int64_t ldh, int J0, int nblk, int r, int c0,
                        int ncols, const float* Tws, int64_t sTwb, const float* A, int64_t sAb,
                        int64_t lda, int batch, hipStream_t stream);
hipError_t trail_grid(int r, int ncols, int batch, int64_t* wgs, int64_t* resident);
hipError_t launch_copy_in(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                          int64_t sHb, int batch, int n, hipStream_t stream);
hipError_t launch_larft(const float* V, int64_t sVb, int64_t ldv, int m, int k, const float* tau,
                        int64_t sTaub, float* T, int64_t sTb, int64_t ldt, int batch,
                        hipStream_t stream);
hipError_t launch_larft_panels(const float* H, int64_t sHb, int64_t ldh, int n, const float* tau,
                               int64_t sTaub, float* T, int64_t sTb, int batch,
                               hipStream_t stream);
hipError_t launch_apply(const float* V, int64_t sVb, int64_t ldv, float* C, int64_t sCb,
                        int64_t ldc, int nblk, int r, int ncols, const float* Tws, int64_t sTwb,
                        bool trans, int kv_last, int batch, hipStream_t stream);
hipError_t launch_eye(float* Q, int64_t sQb, int64_t ldq, int batch, int n, hipStream_t stream);
hipError_t launch_orgqr_smalln(const float* H, int64_t sHb, int64_t ldh, const float* tau,
                               int64_t sTaub, float* Q, int64_t sQb, int64_t ldq, int batch,
                               int n, hipStream_t stream);
}  // namespace qr

namespace {

constexpr int kAbiVersion = 5;
constexpr int kMaxN = 4096;
constexpr int kSmallN = 64;
constexpr int kPanel = 16;
constexpr int kMaxBlocks = 8;  // 16-wide panels per outer block
constexpr int kTStride = kMaxBlocks * kPanel * kPanel;  // T floats per matrix
constexpr size_t kAlign = 256;

size_t align_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

// Workspace of the blocked route: per matrix, the 16 x 16 T of each panel of
// the current outer block.
size_t ws_t_bytes(int batch) { return align_up((size_t)batch * kTStride * sizeof(float)); }

// Workspace of the CholeskyQR2 block route (Gram partials, 64 x 64 factors,
// per-matrix fallback flags); reused by every block of a call.
size_t ws_cq_bytes(int batch) { return align_up(qr::cq_workspace_floats(batch) * sizeof(float)); }

// Outer blocks of 64 columns with at least this many rows take the CholeskyQR2
// route: 128 rows in calls of at most 64 matrices, 576 above (with many
// matrices the Householder panels of short blocks are throughput-bound and
// cheaper). opts->cholqr = 0 switches the route off; opts->cholqr_min_rows
// sets the bound (the route needs r > 64).
int cq_min_rows(int batch, const qr_options& o) {
  if (!o.cholqr) return 1 << 30;
  if (o.cholqr_min_rows) return o.cholqr_min_rows;
  return batch <= 64 ? 128 : 576;
}

// Panels per outer block (opts->outer_panels, 0 = 4).
int outer_blocks(const qr_options& o) { return o.outer_panels ? o.outer_panels : 4; }

bool options_valid(const qr_options& o) {
  return (o.cholqr == 0 || o.cholqr == 1) &&
         (o.cholqr_min_rows == 0 || (o.cholqr_min_rows >= 65 && o.cholqr_min_rows <= kMaxN)) &&
         (o.cholqr_one_pass >= 0 && o.cholqr_one_pass <= 2) &&
         (o.cholqr_fused == 0 || o.cholqr_fused == 1) && (o.lookahead == 0 || o.lookahead == 1) &&
         o.outer_panels >= 0 && o.outer_panels <= kMaxBlocks && o.midn >= 0 && o.midn <= 2;
}

constexpr qr_options kDefaultOptions = {1, 0, 1, 0, 1, 0, 1};

// 64 < n <= 192 in one launch of the fused mid-n kernel (one workgroup per
// matrix) up to batch * ceil(n / 16) = 8192 waves of work: measured against
// the blocked route, 0.5-0.65x its time up to 128 matrices at n = 80..192 and
// 0.86-0.93x at 512; at 2048 matrices 0.88x for n = 80, 0.97x for n = 128 and
// 1.3x for n = 176-192 (a workgroup per matrix holds a CU longer than the
// blocked route's throughput-bound panels).
// The blocked route's last r <= 192 columns go to the same kernel, in place,
// under a tighter bound of 2048: measured against the blocked tail (ms),
// b40 n352 0.365 -> 0.327, b40 n200 0.193 -> 0.144, b60 n1024 2.229 -> 2.210,
// b2 n4096 7.266 -> 7.243, but b300 n300 0.557 -> 0.569 and b640 n512
// 2.493 -> 2.596 (there the blocked tail's panels overlap the previous
// block's update on the second stream).
constexpr int64_t kMidnMaxWaves = 8192;
constexpr int64_t kMidnTailMaxWaves = 2048;
bool midn_route(int batch, int n, const qr_options& o, bool tail = false) {
  if (o.midn == 0 || n <= kSmallN || n > qr::midn_max_n()) return false;
  return o.midn == 2 ||
         (int64_t)batch * ((n + 15) / 16) <= (tail ? kMidnTailMaxWaves : kMidnMaxWaves);
}

int to_status(hipError_t e) { return e == hipSuccess ? QR_OK : QR_ELAUNCH; }

// ---------------------------------------------------------------- tracing --
// When a kernel's bit is set in the trace mask, each of its launches is
// bracketed by two HIP events on the launch stream, and the launch's
// algorithmic flops and bytes are recorded next to them.
struct TraceRec {
  hipEvent_t start;
  hipEvent_t stop;
  int kernel;
  double flops;
  double bytes;
};

std::mutex g_trace_mu;
unsigned g_trace_mask = 0;
// Set while this thread runs qr_geqrf_f32_noalloc: its launches are never
// traced, so it creates no events.
thread_local bool t_untraced = false;
std::vector<TraceRec> g_trace;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t pool_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Runs `launch` on `s`, traced if `kernel` is enabled.
template <typename F>
hipError_t traced(int kernel, double flops, double bytes, hipStream_t s, F&& launch) {
  unsigned mask;
  {
    std::lock_guard<std::mutex> lk(g_trace_mu);
    mask = g_trace_mask;
  }
  if (t_untraced || !(mask & (1u << kernel))) return launch();
  hipEvent_t a, b;
  {
    std::lock_guard<std::mutex> lk(g_trace_mu);
    a = pool_event();
    b = pool_event();
  }
  if (!a || !b) return launch();
  hipEventRecord(a, s);
  const hipError_t e = launch();
  hipEventRecord(b, s);
  std::lock_guard<std::mutex> lk(g_trace_mu);
  g_trace.push_back({a, b, kernel, flops, bytes});
  return e;
}

// Algorithmic work per launch (whole batch), used for roofline figures.
double panel_flops(int r, int kw) {  // sgeqr2 on r x kw + the T recurrence
  return 2.0 * r * kw * kw - 2.0 / 3.0 * kw * kw * kw + 1.0 / 3.0 * kw * kw * kw;
}

// Highest element offset (+1) touched by a (batch, n, n) view with these strides.
bool extent(int batch, int n, int64_t sb, int64_t sr, int64_t sc, int64_t* out) {
  if (sb < 0 || sr < 0 || sc < 0) return false;
  *out = (int64_t)(batch - 1) * sb + (int64_t)(n - 1) * sr + (int64_t)(n - 1) * sc + 1;
  return true;
}

bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
  const char* pa = static_cast<const char*>(a);
  const char* pb = static_cast<const char*>(b);
  return pa < pb + bbytes && pb < pa + abytes;
}

int check_geqrf_args(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, const float* H,
                     const float* tau, int batch, int n) {
  if (batch < 0 || n < 0) return QR_EINVAL;
  if (n > kMaxN) return QR_EUNSUPPORTED;
  if (batch == 0 || n == 0) return QR_OK;
  if (!A || !H || !tau) return QR_EINVAL;
  int64_t ext = 0;
  if (!extent(batch, n, sAb, sAr, sAc, &ext)) return QR_EINVAL;
  const size_t hbytes = (size_t)batch * n * n * sizeof(float);
  const size_t tbytes = (size_t)batch * n * sizeof(float);
  if (overlaps(A, (size_t)ext * sizeof(float), H, hbytes)) return QR_EINVAL;
  if (overlaps(A, (size_t)ext * sizeof(float), tau, tbytes)) return QR_EINVAL;
  if (overlaps(H, hbytes, tau, tbytes)) return QR_EINVAL;
  return QR_OK;
}

// H and tau at strides (sHb, ldh, 1) and (sTaub, 1); A may be H itself.
hipError_t run_smalln(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                      int64_t sHb, int64_t ldh, float* tau, int64_t sTaub, int batch, int n,
                      hipStream_t s) {
  const double flops = 4.0 / 3.0 * n * n * (double)n * batch;
  const double bytes = (2.0 * n * n + n) * 4.0 * batch;
  return traced(QR_KERNEL_SMALLN, flops, bytes, s, [&] {
    return qr::launch_geqrf_smalln(A, sAb, sAr, sAc, H, sHb, ldh, tau, sTaub, batch, n, s);
  });
}

// The fused mid-n kernel (64 < n <= 192, one workgroup per matrix), traced with
// the small-n kernel as the fused whole-matrix family.
// H and tau of (batch, n, n) and (batch, n) matrices at strides (sHb, ldh, 1)
// and (sTaub, 1); A may be H itself (in-place factorisation of the blocked
// route's last columns).
hipError_t run_midn(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H, int64_t sHb,
                    int64_t ldh, float* tau, int64_t sTaub, int batch, int n, hipStream_t s) {
  const double flops = 4.0 / 3.0 * n * n * (double)n * batch;
  const double bytes = (2.0 * n * n + n) * 4.0 * batch;
  return traced(QR_KERNEL_SMALLN, flops, bytes, s, [&] {
    return qr::launch_geqrf_midn(A, sAb, sAr, sAc, H, sHb, ldh, tau, sTaub, batch, n, s);
  });
}

// A (when not null): where the outer block's columns are read from instead of H
// (row stride lda, unit column stride); the results still go to H.
hipError_t run_panel(float* H, int64_t sHb, int64_t ldh, int J0, int p, int r, int kw, float* tau,
                     int64_t sTaub, float* T, int64_t sTb, int batch, hipStream_t s,
                     const float* A = nullptr, int64_t sAb = 0, int64_t lda = 0,
                     const int* only = nullptr) {
  // left-looking MFMA work (panels 0..p-1) + the panel's own factorisation
  const double flops = (4.0 * r * kPanel * kPanel * p + panel_flops(r - 16 * p, kw)) * batch;
  const double bytes = (2.0 * r * kw + (double)r * kPanel * p + kw + kPanel * kPanel * (p + 1)) *
                       4.0 * batch;
  return traced(QR_KERNEL_PANEL, flops, bytes, s, [&] {
    return qr::launch_panel(H, sHb, ldh, J0, p, r, kw, tau, sTaub, T, sTb, A, sAb, lda, batch, s,
                            only);
  });
}

// One 64-column block by CholeskyQR2 + Householder reconstruction. Work per
// matrix: four r x 64 x 64 MFMA passes at 5/8 density (two Grams, A M1, the
// rows below times M); bytes: the block read three times, V written once.
hipError_t run_cq_block(const float* Src, int64_t sSb, int64_t lds, float* Hb, int64_t sHb,
                        int64_t ldh, int r, float* tau, int64_t sTaub, float* T, int64_t sTb,
                        float* ws, int batch, const qr_options& o, hipStream_t s) {
  const double flops = 4.0 * 2.0 * r * 64.0 * 64.0 * 0.625 * batch;
  const double bytes = 4.0 * r * 64.0 * 4.0 * batch;
  return traced(QR_KERNEL_CHOLQR, flops, bytes, s, [&] {
    return qr::launch_cq_block(Src, sSb, lds, Hb, sHb, ldh, r, tau, sTaub, T, sTb, ws, batch,
                               o.cholqr_fused != 0, o.cholqr_one_pass, s);
  });
}

// Columns c0 .. c0+ncols-1 (relative to the outer block at J0) := Q^T C.
hipError_t run_trail(float* H, int64_t sHb, int64_t ldh, int J0, int nblk, int r, int c0,
                     int ncols, const float* T, int64_t sTb, int batch, hipStream_t s,
                     const float* A = nullptr, int64_t sAb = 0, int64_t lda = 0) {
  double rows = 0.0;  // sum over the blocks of their row counts
  for (int q = 0; q < nblk; ++q) rows += r - kPanel * q;
  const double flops = 4.0 * kPanel * (double)ncols * rows * batch;
  const double bytes = (2.0 * r * ncols + rows * kPanel) * 4.0 * batch;
  return traced(QR_KERNEL_TRAIL, flops, bytes, s, [&] {
    return qr::launch_trail(H, sHb, ldh, J0, nblk, r, c0, ncols, T, sTb, A, sAb, lda, batch, s);
  });
}

// Second stream (default priority) and three events per device for the
// look-ahead schedule of qr_geqrf_f32; created on first use, kept for the
// life of the process.
//
// panels_done and rest_done only order kernels of two streams of one device,
// and every kernel dispatch already acquires and releases at device scope, so
// they are created without the system-scope fence (that fence writes caches
// back for the host at every record: about 1 % of cfgs 3-5). all_done hands
// the last side-stream update back to the caller's stream and keeps the
// system-scope fence, so what the caller's stream completes is visible as
// after any other kernel.
struct Lookahead {
  hipStream_t s2 = nullptr;
  hipEvent_t panels_done = nullptr;
  hipEvent_t rest_done = nullptr;
  hipEvent_t all_done = nullptr;
};

std::mutex g_la_mu;
// Held for the whole enqueue of a call that uses the second stream: the
// stream and its events are shared by every call on the device, so two host
// threads must not interleave their records and waits (a call's side-stream
// wait could otherwise capture another call's "panels done").
std::mutex g_la_call_mu;
std::vector<Lookahead> g_la;

bool lookahead_for_current_device(Lookahead* out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return false;
  std::lock_guard<std::mutex> lk(g_la_mu);
  if ((int)g_la.size() <= dev) g_la.resize(dev + 1);
  Lookahead& la = g_la[dev];
  if (!la.s2) {
    hipStream_t st = nullptr;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) return false;
    hipEvent_t a = nullptr, b = nullptr, c = nullptr;
    const unsigned local = hipEventDisableTiming | hipEventDisableSystemFence;
    if (hipEventCreateWithFlags(&a, local) != hipSuccess ||
        hipEventCreateWithFlags(&b, local) != hipSuccess ||
        hipEventCreateWithFlags(&c, hipEventDisableTiming) != hipSuccess) {
      if (a) hipEventDestroy(a);
      if (b) hipEventDestroy(b);
      hipStreamDestroy(st);
      return false;
    }
    la.s2 = st;
    la.panels_done = a;
    la.rest_done = b;
    la.all_done = c;
  }
  *out = la;
  return true;
}

}  // namespace

extern "C" {

const char* qr_status_string(int status) {
  switch (status) {
    case QR_OK: return "ok";
    case QR_EINVAL: return "invalid argument";
    case QR_EUNSUPPORTED: return "unsupported matrix size";
    case QR_EWORKSPACE: return "workspace too small";
    case QR_ELAUNCH: return "HIP kernel launch failed";
    default: return "unknown status";
  }
}

int qr_abi_version(void) { return kAbiVersion; }

int qr_max_n(void) { return kMaxN; }

size_t qr_geqrf_f32_workspace(int batch, int n) {
  if (batch <= 0 || n <= kSmallN || n > kMaxN) return 0;
  return 2 * ws_t_bytes(batch) + ws_cq_bytes(batch);
}

int qr_fused_smalln_f32(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                        float* tau, int batch, int n, void* stream) {
  int st = check_geqrf_args(A, sAb, sAr, sAc, H, tau, batch, n);
  if (st != QR_OK || batch == 0 || n == 0) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n <= kSmallN)
    return to_status(run_smalln(A, sAb, sAr, sAc, H, (int64_t)n * n, n, tau, n, batch, n, s));
  if (n <= qr::midn_max_n())
    return to_status(run_midn(A, sAb, sAr, sAc, H, (int64_t)n * n, n, tau, n, batch, n, s));
  return QR_EUNSUPPORTED;
}

void qr_default_options(qr_options* opts) {
  if (opts) *opts = kDefaultOptions;
}

size_t qr_geqrf_f32_route_codes_offset(int batch, int n) {
  if (batch <= 0 || n <= kSmallN || n > kMaxN) return 0;
  return 2 * ws_t_bytes(batch) + qr::cq_flags_offset_floats(batch) * sizeof(float);
}

int qr_geqrf_f32(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H, float* tau,
                 int batch, int n, void* workspace, size_t workspace_bytes, void* stream) {
  return qr_geqrf_f32_ex(A, sAb, sAr, sAc, H, tau, batch, n, workspace, workspace_bytes, nullptr,
                         stream);
}

int qr_geqrf_f32_ex(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H, float* tau,
                    int batch, int n, void* workspace, size_t workspace_bytes,
                    const qr_options* opts, void* stream) {
  const qr_options o = opts ? *opts : kDefaultOptions;
  if (!options_valid(o)) return QR_EINVAL;
  int st = check_geqrf_args(A, sAb, sAr, sAc, H, tau, batch, n);
  if (st != QR_OK || batch == 0 || n == 0) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t nn = (int64_t)n * n;
  if (n <= kSmallN)
    return to_status(run_smalln(A, sAb, sAr, sAc, H, (int64_t)n * n, n, tau, n, batch, n, s));

  const size_t need = qr_geqrf_f32_workspace(batch, n);
  if (workspace_bytes < need || !workspace) return QR_EWORKSPACE;
  if (midn_route(batch, n, o))
    return to_status(run_midn(A, sAb, sAr, sAc, H, nn, n, tau, n, batch, n, s));
  // Two T slots per matrix: outer block k uses slot k & 1, so the panels of
  // block k+1 never overwrite T factors that block k's trailing update reads.
  float* Tslot[2] = {static_cast<float*>(workspace),
                     static_cast<float*>(workspace) + (size_t)batch * kTStride};
  float* cq_ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + 2 * ws_t_bytes(batch));
  const int cq_rows = cq_min_rows(batch, o);
  bool cq_ready = false;

  // With a unit column stride the first outer block reads A itself: its panels
  // and trailing updates write every element of H, so no copy is needed.
  // Other layouts (e.g. a transposed view) are copied into H first.
  const bool direct = sAc == 1;
  hipError_t e = hipSuccess;
  if (!direct) {
    e = traced(QR_KERNEL_COPY, 0.0, 2.0 * nn * 4.0 * batch, s, [&] {
      return qr::launch_copy_in(A, sAb, sAr, sAc, H, nn, batch, n, s);
    });
    if (e != hipSuccess) return QR_ELAUNCH;
  }
  const int P = outer_blocks(o);
  const int NB = kPanel * P;

  // Look-ahead schedule. On the caller's stream s: the panels of block k, then
  // the update of block k+1's columns only, then the panels of block k+1. On s2:
  // the update of every column right of block k+1, which runs concurrently
  // with the panels of block k+1. Events order the two streams:
  //   s2 waits for "panels of block k done" before updating with them;
  //   s waits for "rest of block k done" before touching columns >= J0 + 2 NB;
  //   at the end s waits for everything s2 did ("all done").
  Lookahead la;
  const bool use_la = o.lookahead && n > 2 * NB && lookahead_for_current_device(&la);
  std::unique_lock<std::mutex> la_lock(g_la_call_mu, std::defer_lock);
  if (use_la) la_lock.lock();
  bool rest_pending = false;  // s2 holds work that s must wait for
  bool s2_used = false;

  int blk = 0;
  for (int J0 = 0; J0 < n; J0 += NB, ++blk) {
    float* Tws = Tslot[blk & 1];
    const float* Ab = (direct && J0 == 0) ? A : nullptr;  // source of this block's columns
    const int r = n - J0;
    // The last r <= 192 columns in one launch of the fused mid-n kernel, in
    // place on H's trailing r x r block.
    // The last <= 64 columns: one small-n launch, in place (not with midn = 0).
    if (J0 > 0 && r <= kSmallN && o.midn != 0) {
      if (rest_pending) {
        if (hipStreamWaitEvent(s, la.rest_done, 0) != hipSuccess) return QR_ELAUNCH;
        rest_pending = false;
      }
      float* Hs = H + (int64_t)J0 * n + J0;
      e = run_smalln(Hs, nn, n, 1, Hs, nn, n, tau + J0, n, batch, r, s);
      if (e != hipSuccess) return QR_ELAUNCH;
      break;
    }
    if (J0 > 0 && midn_route(batch, r, o, true)) {
      if (rest_pending) {
        if (hipStreamWaitEvent(s, la.rest_done, 0) != hipSuccess) return QR_ELAUNCH;
        rest_pending = false;
      }
      float* Hs = H + (int64_t)J0 * n + J0;
      e = run_midn(Hs, nn, n, 1, Hs, nn, n, tau + J0, n, batch, r, s);
      if (e != hipSuccess) return QR_ELAUNCH;
      break;
    }
    const int nblk = (r + kPanel - 1) / kPanel < P ? (r + kPanel - 1) / kPanel : P;
    // A full 64-column block with enough rows: CholeskyQR2 + reconstruction,
    // then the panels for the matrices it flagged (the rest return at once).
    const int* only = nullptr;
    if (P * kPanel == 64 && J0 + 64 <= n && r >= cq_rows) {
      if (!cq_ready) {  // arrival counters of the fused Gram kernels start at zero
        if (qr::launch_cq_reset(cq_ws, batch, s) != hipSuccess) return QR_ELAUNCH;
        cq_ready = true;
      }
      const float* Src = Ab ? Ab : H + (int64_t)J0 * n + J0;
      const int64_t sSb = Ab ? sAb : nn, lds = Ab ? sAr : n;
      e = run_cq_block(Src, sSb, lds, H + (int64_t)J0 * n + J0, nn, n, r, tau + J0, n, Tws,
                       kTStride, cq_ws, batch, o, s);
      if (e != hipSuccess) return QR_ELAUNCH;
      only = qr::cq_flags(cq_ws, batch);
    }
    if (only) {  // one launch for the flagged matrices' panels
      e = traced(QR_KERNEL_PANEL, 0.0, 0.0, s, [&] {
        return qr::launch_panel_seq(H, nn, n, J0, nblk, r, tau, n, Tws, kTStride, Ab, sAb, sAr,
                                    batch, s, only);
      });
      if (e != hipSuccess) return QR_ELAUNCH;
    }
    for (int p = 0; p < nblk && !only; ++p) {
      const int kw = (r - kPanel * p) < kPanel ? (r - kPanel * p) : kPanel;
      e = run_panel(H, nn, n, J0, p, r, kw, tau, n, Tws, kTStride, batch, s, Ab, sAb, sAr);
      if (e != hipSuccess) return QR_ELAUNCH;
    }
    const int ncols = r - kPanel * nblk;
    if (ncols <= 0) continue;
    if (!use_la) {
      e = run_trail(H, nn, n, J0, nblk, r, kPanel * nblk, ncols, Tws, kTStride, batch, s, Ab, sAb,
                    sAr);
      if (e != hipSuccess) return QR_ELAUNCH;
      continue;
    }
    // When the whole update fits on the device in one round of workgroups, a
    // split buys no overlap, only the cross-stream packets between the panels
    // and the next update (about 10 us per block): one launch on s instead.
    // Every strip's arithmetic is the same either way.
    {
      int64_t wgs = 0, resident = 1;
      if (qr::trail_grid(r, ncols, batch, &wgs, &resident) != hipSuccess) return QR_ELAUNCH;
      if (wgs <= resident) {
        if (rest_pending) {
          if (hipStreamWaitEvent(s, la.rest_done, 0) != hipSuccess) return QR_ELAUNCH;
          rest_pending = false;
        }
        e = run_trail(H, nn, n, J0, nblk, r, kPanel * nblk, ncols, Tws, kTStride, batch, s, Ab,
                      sAb, sAr);
        if (e != hipSuccess) return QR_ELAUNCH;
        continue;
      }
    }
    const int next = ncols < NB ? ncols : NB;
    const int rest = ncols - next;
    // Columns of block k+1 were last updated by the rest-update of block k-1.
    if (rest_pending) {
      if (hipStreamWaitEvent(s, la.rest_done, 0) != hipSuccess) return QR_ELAUNCH;
      rest_pending = false;
    }
    if (rest > 0) {
      if (hipEventRecord(la.panels_done, s) != hipSuccess) return QR_ELAUNCH;
      if (hipStreamWaitEvent(la.s2, la.panels_done, 0) != hipSuccess) return QR_ELAUNCH;
      e = run_trail(H, nn, n, J0, nblk, r, kPanel * nblk + next, rest, Tws, kTStride, batch,
                    la.s2, Ab, sAb, sAr);
      if (e != hipSuccess) return QR_ELAUNCH;
      if (hipEventRecord(la.rest_done, la.s2) != hipSuccess) return QR_ELAUNCH;
      rest_pending = true;
      s2_used = true;
    }
    e = run_trail(H, nn, n, J0, nblk, r, kPanel * nblk, next, Tws, kTStride, batch, s, Ab, sAb,
                  sAr);
    if (e != hipSuccess) return QR_ELAUNCH;
  }
  if (s2_used) {
    if (hipEventRecord(la.all_done, la.s2) != hipSuccess ||
        hipStreamWaitEvent(s, la.all_done, 0) != hipSuccess)
      return QR_ELAUNCH;
  }
  return QR_OK;
}

}  // extern "C"

namespace {

// Workspace of qr_geqrf_f32_noalloc: a static device array, one copy on each
// GPU the library runs on, held until the process ends. Host code must use
// the per-device address from hipGetSymbolAddress, never `scratch` itself
// (in host code that name is a host-side stand-in, not a device address).
__device__ __align__(256) unsigned char scratch[QR_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device (with that device current); nullptr if the lookup fails.
void* scratch_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int qr_geqrf_f32_noalloc(const float* A, int64_t sAb, int64_t sAr, int64_t sAc, float* H,
                         float* tau, int batch, int n, void* stream) {
  int st = check_geqrf_args(A, sAb, sAr, sAc, H, tau, batch, n);
  if (st != QR_OK || batch == 0 || n == 0) return st;
  const size_t need = qr_geqrf_f32_workspace(batch, n);
  if (need > QR_NOALLOC_SCRATCH_BYTES) return QR_EWORKSPACE;
  void* ws = nullptr;
  if (need > 0) {
    ws = scratch_for_current_device();
    if (!ws) return QR_ELAUNCH;
  }
  // Everything on the caller's stream: no second stream, no events, no
  // occupancy query; the same kernels and results as with look-ahead.
  qr_options o = kDefaultOptions;
  o.lookahead = 0;
  t_untraced = true;
  st = qr_geqrf_f32_ex(A, sAb, sAr, sAc, H, tau, batch, n, ws, need, &o, stream);
  t_untraced = false;
  return st;
}

int qr_panel_f32(float* H, int64_t sHb, int64_t ldh, int j0, int p, int r, int kw, float* tau,
                 int64_t sTaub, float* T, int64_t sTb, int batch, void* stream) {
  if (batch < 0 || j0 < 0 || p < 0 || r < 0 || kw < 0 || sHb < 0 || sTaub < 0 || sTb < 0)
    return QR_EINVAL;
  if (batch == 0 || r == 0 || kw == 0) return QR_OK;
  if (!H || !tau || !T) return QR_EINVAL;
  if (kw > kPanel || p >= kMaxBlocks || r < kPanel * p + kw || ldh < j0 + kPanel * p + kw)
    return QR_EINVAL;
  if (r > kMaxN) return QR_EUNSUPPORTED;
  if (sTb < (int64_t)kPanel * kPanel * (p + 1)) return QR_EINVAL;
  return to_status(
      run_panel(H, sHb, ldh, j0, p, r, kw, tau, sTaub, T, sTb, batch, static_cast<hipStream_t>(stream)));
}

int qr_larft_f32(const float* V, int64_t sVb, int64_t ldv, int m, int k, const float* tau,
                 int64_t sTaub, float* T, int64_t sTb, int64_t ldt, int batch, void* stream) {
  if (batch < 0 || m < 0 || k < 0 || sVb < 0 || sTaub < 0 || sTb < 0) return QR_EINVAL;
  if (batch == 0 || k == 0) return QR_OK;
  if (!V || !tau || !T) return QR_EINVAL;
  if (k > 64) return QR_EUNSUPPORTED;
  if (m < k || ldv < k || ldt < k || sTb < (int64_t)(k - 1) * ldt + k) return QR_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const double flops = ((double)m * k * k + k * k * (double)k / 3.0) * batch;
  return to_status(traced(QR_KERNEL_LARFT, flops, ((double)m * k + k + k * k) * 4.0 * batch, s,
                          [&] {
                            return qr::launch_larft(V, sVb, ldv, m, k, tau, sTaub, T, sTb, ldt,
                                                    batch, s);
                          }));
}

int qr_wy_update_f32(float* H, int64_t sHb, int64_t ldh, int j0, int nblk, int r, int c,
                     const float* T, int64_t sTb, int batch, void* stream) {
  if (batch < 0 || j0 < 0 || nblk < 0 || r < 0 || c < 0 || sHb < 0 || sTb < 0) return QR_EINVAL;
  if (batch == 0 || r == 0 || c == 0 || nblk == 0) return QR_OK;
  if (!H || !T) return QR_EINVAL;
  if (nblk > kMaxBlocks || r < kPanel * (nblk - 1) + 1 || ldh < j0 + kPanel * nblk + c ||
      sTb < (int64_t)kPanel * kPanel * nblk)
    return QR_EINVAL;
  if (r > kMaxN) return QR_EUNSUPPORTED;
  return to_status(run_trail(H, sHb, ldh, j0, nblk, r, kPanel * nblk, c, T, sTb, batch,
                             static_cast<hipStream_t>(stream)));
}

size_t qr_ormqr_f32_workspace(int batch, int n) {
  if (batch <= 0 || n <= 0 || n > kMaxN) return 0;
  return align_up((size_t)batch * ((n + kPanel - 1) / kPanel) * kPanel * kPanel * sizeof(float));
}

}  // extern "C"

namespace {

// T of every panel (larft from H, tau), then the 16-wide block reflectors in
// groups of kMaxBlocks panels: Q^T C applies them first to last, Q C last to
// first. With from_diag, the group starting at row J0 only touches columns
// J0.. of C (orgqr on the identity: columns left of J0 are unit vectors that
// are zero in rows J0.., so those blocks leave them unchanged).
int apply_q(const float* H, int64_t sHb, int64_t ldh, const float* tau, int64_t sTaub, float* C,
            int64_t sCb, int64_t ldc, int n, int m, bool trans, bool from_diag, int batch,
            float* Tw, hipStream_t s) {
  const int np = (n + kPanel - 1) / kPanel;
  const int64_t sTw = (int64_t)np * kPanel * kPanel;
  const double lf = (16.0 * 16.0 * n + 16.0 * 16.0 * 16.0 / 3.0) * np * batch;
  hipError_t e = traced(QR_KERNEL_LARFT, lf, ((double)n * n + n + 256.0 * np) * 4.0 * batch, s,
                        [&] { return qr::launch_larft_panels(H, sHb, ldh, n, tau, sTaub, Tw, sTw,
                                                             batch, s); });
  if (e != hipSuccess) return to_status(e);
  const int ngroups = (np + kMaxBlocks - 1) / kMaxBlocks;
  for (int gi = 0; gi < ngroups; ++gi) {
    const int g = trans ? gi : ngroups - 1 - gi;
    const int q0 = g * kMaxBlocks;
    const int nblk = (np - q0) < kMaxBlocks ? (np - q0) : kMaxBlocks;
    const int J0 = kPanel * q0;
    const int r = n - J0;
    const int c0 = from_diag ? J0 : 0;
    const int ncols = m - c0;
    const int kv_last = n - kPanel * (q0 + nblk - 1);
    double rows = 0.0;
    for (int q = 0; q < nblk; ++q) rows += (double)(r - kPanel * q);
    const double flops = 4.0 * kPanel * (double)ncols * rows * batch;
    const double bytes = (2.0 * r * ncols + rows * kPanel) * 4.0 * batch;
    e = traced(QR_KERNEL_APPLY, flops, bytes, s, [&] {
      return qr::launch_apply(H + (int64_t)J0 * ldh + J0, sHb, ldh, C + (int64_t)J0 * ldc + c0,
                              sCb, ldc, nblk, r, ncols, Tw + (int64_t)q0 * kPanel * kPanel, sTw,
                              trans, kv_last > kPanel ? kPanel : kv_last, batch, s);
    });
    if (e != hipSuccess) return to_status(e);
  }
  return QR_OK;
}

}  // namespace

extern "C" {

int qr_ormqr_f32(const float* H, int64_t sHb, int64_t ldh, const float* tau, int64_t sTaub,
                 float* C, int64_t sCb, int64_t ldc, int n, int m, int trans, int batch,
                 void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 0 || n < 0 || m < 0 || sHb < 0 || sTaub < 0 || sCb < 0) return QR_EINVAL;
  if (trans != 0 && trans != 1) return QR_EINVAL;
  if (batch == 0 || n == 0 || m == 0) return QR_OK;
  if (!H || !tau || !C) return QR_EINVAL;
  if (n > kMaxN) return QR_EUNSUPPORTED;
  if (ldh < n || ldc < m || sTaub < n) return QR_EINVAL;
  if (batch > 1 && (sHb < (int64_t)(n - 1) * ldh + n || sCb < (int64_t)(n - 1) * ldc + m))
    return QR_EINVAL;
  if (!workspace || workspace_bytes < qr_ormqr_f32_workspace(batch, n)) return QR_EWORKSPACE;
  return apply_q(H, sHb, ldh, tau, sTaub, C, sCb, ldc, n, m, trans != 0, false, batch,
                 static_cast<float*>(workspace), static_cast<hipStream_t>(stream));
}

int qr_orgqr_f32(const float* H, int64_t sHb, int64_t ldh, const float* tau, int64_t sTaub,
                 float* Q, int64_t sQb, int64_t ldq, int n, int batch, void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (batch < 0 || n < 0 || sHb < 0 || sTaub < 0 || sQb < 0) return QR_EINVAL;
  if (batch == 0 || n == 0) return QR_OK;
  if (!H || !tau || !Q) return QR_EINVAL;
  if (n > kMaxN) return QR_EUNSUPPORTED;
  if (ldh < n || ldq < n || sTaub < n) return QR_EINVAL;
  if (batch > 1 && (sHb < (int64_t)(n - 1) * ldh + n || sQb < (int64_t)(n - 1) * ldq + n))
    return QR_EINVAL;
  if (overlaps(H, ((size_t)(batch - 1) * sHb + (size_t)(n - 1) * ldh + n) * sizeof(float), Q,
               ((size_t)(batch - 1) * sQb + (size_t)(n - 1) * ldq + n) * sizeof(float)))
    return QR_EINVAL;
  if (!workspace || workspace_bytes < qr_ormqr_f32_workspace(batch, n)) return QR_EWORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n <= kSmallN) {  // one wavefront per matrix forms Q in registers: one launch
    const double flops = 4.0 / 3.0 * n * n * (double)n * batch;
    return to_status(traced(QR_KERNEL_APPLY, flops, (2.0 * n * n + n) * 4.0 * batch, s, [&] {
      return qr::launch_orgqr_smalln(H, sHb, ldh, tau, sTaub, Q, sQb, ldq, batch, n, s);
    }));
  }
  const hipError_t e = traced(QR_KERNEL_COPY, 0.0, (double)n * n * 4.0 * batch, s,
                              [&] { return qr::launch_eye(Q, sQb, ldq, batch, n, s); });
  if (e != hipSuccess) return to_status(e);
  return apply_q(H, sHb, ldh, tau, sTaub, Q, sQb, ldq, n, n, false, true, batch,
                 static_cast<float*>(workspace), s);
}

int qr_trace_enable(unsigned kernel_mask) {
  std::lock_guard<std::mutex> lk(g_trace_mu);
  g_trace_mask = kernel_mask;
  return QR_OK;
}

int qr_trace_reset(void) {
  std::lock_guard<std::mutex> lk(g_trace_mu);
  for (auto& t : g_trace) {
    g_event_pool.push_back(t.start);
    g_event_pool.push_back(t.stop);
  }
  g_trace.clear();
  return QR_OK;
}

int qr_trace_read(int kernel, int* launches, double* total_ms, double* flops, double* bytes) {
  if (!launches || !total_ms || !flops || !bytes) return QR_EINVAL;
  std::lock_guard<std::mutex> lk(g_trace_mu);
  int cnt = 0;
  double ms = 0.0, fl = 0.0, by = 0.0;
  for (auto& t : g_trace) {
    if (t.kernel != kernel) continue;
    if (hipEventSynchronize(t.stop) != hipSuccess) return QR_ELAUNCH;
    float dt = 0.0f;
    if (hipEventElapsedTime(&dt, t.start, t.stop) != hipSuccess) return QR_ELAUNCH;
    ++cnt;
    ms += dt;
    fl += t.flops;
    by += t.bytes;
  }
  *launches = cnt;
  *total_ms = ms;
  *flops = fl;
  *bytes = by;
  return QR_OK;
}

}  // extern "C"
