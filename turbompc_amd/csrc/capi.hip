// C ABI of libtmpc_hip (declared in include/tmpc.h): argument validation,
// workspace carving and the asynchronous launch schedules.  Nothing here
// allocates device memory or synchronises the host with the stream.
#include "../../include/tmpc.h"

#include <algorithm>
#include <mutex>
#include <vector>

#include "admm_direct.hpp"
#include "admm_stream.hpp"
#include "common.hpp"
#include "factor.hpp"
#include "pcg.hpp"
#include "factor_rows.hpp"
#include "kkt_factor.hpp"
#include "pcg_lds.hpp"
#include "obstacle.hpp"
#include "linear.hpp"
#include "quadrotor.hpp"
#include "adjoint.hpp"
#include "sqp.hpp"
#include "merit.hpp"

// Workspace of tmpc_admm_direct_noalloc: one copy per GPU, at its own device
// address, held until the process ends.  Host code never uses this name as an
// address: it asks each device for the array's address once
// (noalloc_scratch() below) and passes that pointer.
static __device__ __align__(256) unsigned char scratch[TMPC_NOALLOC_SCRATCH_BYTES];

namespace tmpc {
namespace {

constexpr size_t kAlign = 256;

// events of tmpc_set_timing_events (process-wide)
hipEvent_t g_iter_events[2] = {nullptr, nullptr};
inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

constexpr int kMaxDevices = 64;

// A second stream for work that overlaps the factorization (default
// priority, one per host thread and device, created on first use), with the
// events that fork it from and join it back to the caller's stream.  The
// factorization runs at one wavefront per SIMD and waits on its pivot chain
// for much of the time, so a short memory-bound kernel beside it costs
// little.  nullptr where it cannot be had (the work then runs in order on
// the caller's stream).
struct SideStream {
  hipStream_t q = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
thread_local SideStream t_side[kMaxDevices];

SideStream* side_stream(hipStream_t s) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  if (s != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess || (int)sdev != dev) return nullptr;
  }
  SideStream& x = t_side[dev];
  if (x.q == nullptr) {
    SideStream y;
    if (hipStreamCreateWithFlags(&y.q, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&y.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&y.join, hipEventDisableTiming) != hipSuccess) {
      if (y.fork) (void)hipEventDestroy(y.fork);
      (void)hipStreamDestroy(y.q);
      return nullptr;
    }
    x = y;
  }
  return &x;
}

struct Carver {
  char* base;
  size_t off = 0;
  template <typename U>
  U* take(size_t count) {
    U* p = reinterpret_cast<U*>(base + off);
    off += align_up(count * sizeof(U));
    return p;
  }
};

bool dims_ok(const tmpc_dims* d) {
  return d && d->B >= 1 && d->T >= 2 && d->n >= 1 && d->n <= 64 && d->m >= 0 && d->m <= 64 &&
         d->nx >= 1 && d->nx <= d->n && d->n0 >= 1 && d->n0 <= d->n;
}

Dims to_dims(const tmpc_dims* d) {
  return Dims{d->B, d->T, d->T - 1, d->n, d->nx, d->n0, d->m, d->n};
}

// The stage-record shapes the streaming kernels are built for: n in {6, 9,
// 16, 17}, nx <= n - 1, and either m <= kMaxStreamM with nx + m <= n (the
// stacked constraint rows of a stage fit the problem's n lanes) or a wide
// form: n = 9 with nx + m <= kWideRows and m <= kWideMaxM, n = 16 with
// nx + m <= kWide16Rows and m <= kWide16MaxM; stage-run offsets are 32-bit
// element offsets.
inline bool stream_wide(const Dims& d) { return d.nx + d.m > d.n; }
// row lanes per problem of the wide form
inline int stream_wide_rows(const Dims& d) { return d.n == 16 ? kWide16Rows : kWideRows; }

inline bool stream_shape_ok(const Dims& d) {
  if (!(d.n == 6 || d.n == 9 || d.n == 16 || d.n == 17)) return false;
  if (d.nx > d.n - 1) return false;
  if (stream_wide(d)) {
    const bool w9 = d.n == 9 && d.nx + d.m <= kWideRows && d.m <= kWideMaxM;
    const bool w16 = d.n == 16 && d.nx + d.m <= kWide16Rows && d.m <= kWide16MaxM;
    if (!w9 && !w16) return false;
  } else if (d.m > kMaxStreamM) {
    return false;
  }
  const RecGeom g = rec_geom(d);
  const int widest = std::max(std::max(g.amp, g.rvp), th_pitch(d.n));
  return (long long)d.T * d.B * widest < (1LL << 31);
}

// Record dims of the streaming path: the block width n rounded up to the
// smallest width above that fits the shape, the extra variables being
// decoupled dummies (stage_pack_kernel); the QP and state keep rows of nq = n.
// d itself when no width fits (the generic kernels then run).
inline Dims stream_record_dims(const Dims& d) {
  for (int w : {6, 9, 16, 17}) {
    if (w < d.n) continue;
    Dims r = d;
    r.n = w;
    if (stream_shape_ok(r)) return r;
  }
  return d;
}

// Stage records of the streaming path (admm_stream.hpp), on the record dims,
// and the padded A0 [B][n0][n] when the records are wider than the QP.
template <typename R>
size_t stream_ws_bytes(const Dims& d) {
  const Dims r = stream_record_dims(d);
  const RecGeom g = rec_geom(r);
  const size_t B = d.B, T = d.T;
  return align_up(T * B * g.amp * sizeof(R)) + align_up(T * B * g.rvp * sizeof(R)) +
         align_up(T * B * th_pitch(r.n) * sizeof(R)) + align_up(B * d.n0 * r.n * sizeof(R));
}

template <typename R>
size_t direct_ws_bytes(const Dims& d) {
  const size_t B = d.B, T = d.T, n = d.n;
  const int nth = stream_record_dims(d).n;  // >= n
  return align_up(T * B * th_pitch(nth) * sizeof(R)) + 2 * align_up(T * B * n * sizeof(R)) +
         align_up(B * 4 * sizeof(int32_t)) + align_up(B * 8 * sizeof(R)) + stream_ws_bytes<R>(d);
}

// Shapes of the AINV form (stage-invariant A_minus entries resident in LDS,
// admm_stream.hpp): the n = 17 records with G rows, nx n <= kAinvMaxEntries.
// (Built for n = 9 too, it streamed no A_minus entry of config 5's
// time-invariant dynamics and took 25.04 against 24.84 ms per 200-iteration
// launch: that kernel waits on its per-stage dependence chain, not on HBM.)
// Bytes of the compressed runs: [N][waves][rows of 64 16-byte chunks], at
// most 256 entries per problem with one or two problems per wavefront
// (admm_stream.hpp), addressed with 32-bit byte offsets.
inline size_t ainv_runs_bytes(const Dims& d, size_t elem_bytes) {
  return (size_t)d.N * (d.B + 1) * 256 * elem_bytes;
}
inline bool ainv_shape_ok(const Dims& dr, size_t elem_bytes) {
  return dr.n == 17 && dr.m > 0 && !stream_wide(dr) && dr.nx * dr.n <= kAinvMaxEntries && stream_shape_ok(dr) &&
         ainv_runs_bytes(dr, elem_bytes) < (1ULL << 31);
}

// The AINV form's part of the workspace, after the rest: the compressed runs
// (which hold the partial masks first) and the mask words last.
template <typename R>
size_t ainv_ws_bytes(const Dims& d) {
  const Dims r = stream_record_dims(d);
  if (!ainv_shape_ok(r, sizeof(R))) return 0;
  return align_up(ainv_runs_bytes(r, sizeof(R))) + align_up(kAinvWords * sizeof(uint32_t));
}

// What tmpc_admm_direct_workspace_bytes reports: room for every form.  A
// workspace of at least direct_ws_bytes runs every problem; the AINV form
// needs the whole size.
template <typename R>
size_t direct_ws_bytes_full(const Dims& d) {
  return direct_ws_bytes<R>(d) + ainv_ws_bytes<R>(d);
}

template <typename R>
struct DirectWs {
  R *thinv, *w, *gam, *res;
  int32_t* ctl;
  R *am, *rv, *dm;  // stage records of the streaming path
  R* a0p;           // A0 with rows of the records' width
  R* ac;            // AINV: compressed A_minus runs (null without room)
  uint32_t* amask;  // AINV: mask words
};

template <typename R>
DirectWs<R> carve_direct(void* ws, size_t wsb, const Dims& d) {
  Carver c{static_cast<char*>(ws)};
  DirectWs<R> w;
  const Dims r = stream_record_dims(d);
  const size_t B = d.B, T = d.T, n = d.n;
  const RecGeom g = rec_geom(r);
  w.thinv = c.take<R>(T * B * th_pitch(r.n));
  w.w = c.take<R>(T * B * n);
  w.gam = c.take<R>(T * B * n);
  w.ctl = c.take<int32_t>(B * 4);
  w.res = c.take<R>(B * 8);
  w.am = c.take<R>(T * B * g.amp);
  w.rv = c.take<R>(T * B * g.rvp);
  w.dm = c.take<R>(T * B * th_pitch(r.n));
  w.a0p = c.take<R>(B * d.n0 * r.n);
  w.ac = nullptr;
  w.amask = nullptr;
  if (ainv_shape_ok(r, sizeof(R)) && wsb >= direct_ws_bytes_full<R>(d)) {
    w.ac = reinterpret_cast<R*>(c.take<char>(ainv_runs_bytes(r, sizeof(R))));
    w.amask = c.take<uint32_t>(kAinvWords);
  }
  return w;
}

template <typename R>
QPDev<R> to_qp(const tmpc_qp* q) {
  return QPDev<R>{static_cast<const R*>(q->D),  static_cast<const R*>(q->E),
                  static_cast<const R*>(q->q),  static_cast<const R*>(q->A0),
                  static_cast<const R*>(q->A_minus), static_cast<const R*>(q->A_plus),
                  static_cast<const R*>(q->G),  static_cast<const R*>(q->l),
                  static_cast<const R*>(q->u),  static_cast<const R*>(q->c0),
                  static_cast<const R*>(q->c),  static_cast<const R*>(q->slack_weight)};
}

template <typename R>
StateDev<R> to_state(const tmpc_state* s) {
  return StateDev<R>{static_cast<R*>(s->x),  static_cast<R*>(s->z_g), static_cast<R*>(s->y_g),
                     static_cast<R*>(s->y_f0), static_cast<R*>(s->y_f), static_cast<R*>(s->xi_g),
                     static_cast<R*>(s->rho)};
}

bool qp_ok(const tmpc_qp* q, int m) {
  if (!q || !q->D || !q->E || !q->q || !q->A0 || !q->A_minus || !q->A_plus || !q->c0 || !q->c)
    return false;
  if (m > 0 && (!q->G || !q->l || !q->u)) return false;
  return true;
}

bool state_ok(const tmpc_state* s, int m) {
  if (!s || !s->x || !s->y_f0 || !s->y_f || !s->rho) return false;
  if (m > 0 && (!s->z_g || !s->y_g || !s->xi_g)) return false;
  return true;
}

int launch_status() {
  return hipGetLastError() == hipSuccess ? TMPC_OK : TMPC_ELAUNCH;
}

// Dynamic LDS above the 64 KiB default needs an explicit opt-in per kernel.
template <typename K>
void lds_optin(K kernel, size_t bytes) {
  if (bytes > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)bytes);
}

// copies the warm start into the working/output state (skipped when aliased)
template <typename R>
int copy_state(hipStream_t s, const Dims& d, const tmpc_state* in, const tmpc_state* out) {
  const size_t B = d.B, T = d.T, N = d.N;
  const void* src[7] = {in->x, in->z_g, in->y_g, in->y_f0, in->y_f, in->xi_g, in->rho};
  void* dst[7] = {out->x, out->z_g, out->y_g, out->y_f0, out->y_f, out->xi_g, out->rho};
  const size_t cnt[7] = {B * T * d.n, B * T * d.m, B * T * d.m, B * d.n0, B * N * d.nx, B * T * d.m, B};
  for (int k = 0; k < 7; ++k) {
    if (cnt[k] == 0 || src[k] == dst[k]) continue;
    if (!src[k] || !dst[k]) return TMPC_EBADARG;
    if (hipMemcpyAsync(dst[k], src[k], cnt[k] * sizeof(R), hipMemcpyDeviceToDevice, s) != hipSuccess)
      return TMPC_ELAUNCH;
  }
  return TMPC_OK;
}

template <typename R>
int launch_nonfinite_flags(hipStream_t s, const Dims& d, const StateDev<R>& st, uint32_t* iters) {
  hipLaunchKernelGGL((nonfinite_flag_kernel<R>), dim3(d.B), dim3(kWave), 0, s, d, st, iters);
  return launch_status();
}

template <typename R>
int launch_factor_qp(hipStream_t s, const Dims& d, const QPDev<R>& q, const R* rho, R sigma,
                     R rho_f_factor, int32_t* ctl, R* thinv) {
  const size_t smem = factor_smem_bytes(d);
  lds_optin(factor_kernel<R, SRC_QP>, smem);
  hipLaunchKernelGGL((factor_kernel<R, SRC_QP>), dim3(d.B), dim3(kWave), smem, s, d, q,
                     (const R*)nullptr, rho, sigma, rho_f_factor, ctl, thinv);
  return launch_status();
}

template <typename R, int NC, bool STD>
void launch_chunk_nc(hipStream_t s, const AdmmArgs<R>& a) {
  const int grid = (a.d.B + a.P - 1) / a.P;
  hipLaunchKernelGGL((admm_chunk_kernel<R, NC, STD>), dim3(grid), dim3(kWave), 0, s, a);
}

template <typename R, bool STD>
void launch_chunk(hipStream_t s, const AdmmArgs<R>& a) {
  switch (a.d.n) {
    case 6: launch_chunk_nc<R, 6, STD>(s, a); break;
    case 9: launch_chunk_nc<R, 9, STD>(s, a); break;
    case 16: launch_chunk_nc<R, 16, STD>(s, a); break;
    case 17: launch_chunk_nc<R, 17, STD>(s, a); break;
    default: launch_chunk_nc<R, 0, STD>(s, a); break;
  }
}

// Streaming kernel (explicit-integrator structure, record shapes as in
// stream_shape_ok, on the record dims of stream_record_dims).  P problems per
// wavefront: two from B = 2048.  One wavefront per SIMD carrying two problems
// beats two wavefronts of one (config 5, fp64 B = 2048: 28.7 vs 30.3 ms per
// solve), and two per wavefront beat three at every larger batch measured
// (config 3: 1.94 vs 2.10 ms at B = 4096, 5.74 vs 6.46 at 12288, 7.77 vs 8.47
// at 16384; config 5 at 4096 and 8192), since three groups straddle DPP rows
// and move their vectors through LDS slots.  The wide n = 9 form is the
// exception from B = 12288 (config 4: 7.95 vs 8.51 ms at 12288, even at
// 16384, 6.30 vs 5.69 at 8192).
constexpr size_t kMaxLds = 160 * 1024;

// Stages per sweep batch (DPF).  The n <= 9 records are short enough that a
// two-stage batch keeps more loads in flight per wavefront without leaving
// LDS for a second wavefront (config 5, fp64 B = 2048: 28.0 -> 24.8 ms per
// 200-iteration launch); at n = 16/17 the larger slots cost occupancy (config
// 3: 1.94 -> 2.02 ms per launch), so they sweep one stage at a time.
constexpr int stream_depth(int nc) { return nc <= 9 ? 2 : 1; }

inline int stream_problems_per_wave(int B, uint32_t flags, bool wide9) {
  const int forced = (int)((flags >> 8) & 3u);
  if (forced) return forced;
  if (wide9 && B >= 12288) return 3;
  return B >= 2048 ? 2 : 1;
}

// The factorization is bound by instruction issue rather than latency, so it
// packs more problems per wavefront (fewer instructions per problem) as soon
// as that still leaves about one wavefront per SIMD.
inline int factor_problems_per_wave(int B, uint32_t flags) {
  const int forced = (int)((flags >> 8) & 3u);
  return forced ? forced : std::max(1, std::min(3, B / 1024));
}

// d: the record dims (stream_record_dims)
template <typename R>
bool stream_ok(const Dims& d, int P, bool diag) {
  if (!stream_shape_ok(d)) return false;
  if (stream_wide(d) && P > kWave / stream_wide_rows(d)) return false;
  const StreamLayout L = stream_layout(d, P, stream_depth(d.n), diag);
  return (size_t)L.total * sizeof(R) <= kMaxLds;
}

template <typename R, int NC, int P, int NL = NC, int MM = kMaxStreamM, bool GRES = false, bool AINV = false>
void launch_stream_p(hipStream_t s, const StreamArgs<R>& a) {
  constexpr int DPF = stream_depth(NC);
  const StreamLayout L = stream_layout(a.d, P, DPF, a.diag != 0);
  const size_t smem = (size_t)L.total * sizeof(R);
  lds_optin(admm_stream_kernel<R, NC, P, DPF, NL, MM, GRES, AINV>, smem);
  const int grid = (a.d.B + P - 1) / P;
  hipLaunchKernelGGL((admm_stream_kernel<R, NC, P, DPF, NL, MM, GRES, AINV>), dim3(grid), dim3(kWave), smem, s,
                     a);
}

// gres: G_t is the same for every stage and problem (TMPC_FLAG_CONST_G).  Its
// form (the G rows resident in LDS, A_minus rows streamed) is built for the
// n = 17 records with one or two problems per wavefront, where it pays: config
// 3, 1.995 -> 1.924 ms per launch (G is 68 of the 292 words of a record); at
// n = 9 in fp64 (config 5, 27 of 84 words) the scattered A-row stores cost
// more than the bytes they save (25.05 -> 25.51 ms).  ainv (with gres, the
// same shapes, ainv_shape_ok): the AINV form, the stage-invariant A_minus
// entries resident as well (a.amask, a.ac set)
template <typename R, int NC, int NL = NC, int MM = kMaxStreamM>
void launch_stream_nc(hipStream_t s, const StreamArgs<R>& a, int P, bool gres, bool ainv) {
  constexpr bool kGres = NL == NC && NC == 17;
  constexpr bool kAinv = kGres;
  switch (P) {
    case 1:
      if (kAinv && gres && ainv)
        launch_stream_p<R, NC, 1, NL, MM, kAinv, kAinv>(s, a);
      else if (kGres && gres)
        launch_stream_p<R, NC, 1, NL, MM, kGres>(s, a);
      else
        launch_stream_p<R, NC, 1, NL, MM>(s, a);
      break;
    case 2:
      if (kAinv && gres && ainv)
        launch_stream_p<R, NC, 2, NL, MM, kAinv, kAinv>(s, a);
      else if (kGres && gres)
        launch_stream_p<R, NC, 2, NL, MM, kGres>(s, a);
      else
        launch_stream_p<R, NC, 2, NL, MM>(s, a);
      break;
    default:
      if constexpr (3 * NL <= kWave) launch_stream_p<R, NC, 3, NL, MM>(s, a);  // stream_ok rules out the rest
      break;
  }
}

template <typename R>
void launch_stream(hipStream_t s, const StreamArgs<R>& a, int P, bool gres, bool ainv) {
  switch (a.d.n) {
    case 6: launch_stream_nc<R, 6>(s, a, P, gres, false); break;
    case 9:
      if (stream_wide(a.d))
        launch_stream_nc<R, 9, kWideRows, kWideMaxM>(s, a, P, gres, false);
      else
        launch_stream_nc<R, 9>(s, a, P, gres, false);
      break;
    case 16:
      if (stream_wide(a.d))
        launch_stream_nc<R, 16, kWide16Rows, kWide16MaxM>(s, a, P, gres, false);
      else
        launch_stream_nc<R, 16>(s, a, P, gres, false);
      break;
    default: launch_stream_nc<R, 17>(s, a, P, gres, ainv); break;
  }
}

template <typename R, int NC, int P, int NL = NC, int MM = kMaxStreamM>
void launch_factor_std_p(hipStream_t s, const Dims& d, const DirectWs<R>& w, const QPDev<R>& q, const R* rho,
                         R sigma, R rho_f_factor, int32_t* ctl, bool diag) {
  const size_t smem = factor_layout<R>(d, P, diag).bytes;
  lds_optin(factor_std_kernel<R, NC, P, NL, MM>, smem);
  const int grid = (d.B + P - 1) / P;
  hipLaunchKernelGGL((factor_std_kernel<R, NC, P, NL, MM>), dim3(grid), dim3(kWave), smem, s, d, (const R*)w.am,
                     (const R*)w.dm, q.A0, rho, sigma, rho_f_factor, ctl, w.thinv, diag ? 1 : 0);
}

template <typename R, int NC, int NL = NC, int MM = kMaxStreamM>
void launch_factor_std_nc(hipStream_t s, const Dims& d, const DirectWs<R>& w, const QPDev<R>& q, const R* rho,
                          R sigma, R rho_f_factor, int32_t* ctl, int P, bool diag) {
  switch (P) {
    case 1: launch_factor_std_p<R, NC, 1, NL, MM>(s, d, w, q, rho, sigma, rho_f_factor, ctl, diag); break;
    case 2: launch_factor_std_p<R, NC, 2, NL, MM>(s, d, w, q, rho, sigma, rho_f_factor, ctl, diag); break;
    default: launch_factor_std_p<R, NC, 3, NL, MM>(s, d, w, q, rho, sigma, rho_f_factor, ctl, diag); break;
  }
}

template <typename R, int NC, int NR, bool DIAG, bool FULL>
void launch_factor_row_k(hipStream_t s, const Dims& d, const DirectWs<R>& w, const QPDev<R>& q, const R* rho,
                         R sigma, R rho_f_factor, int32_t* ctl) {
  constexpr int per_wave = kWave / kFacRow;
  const int grid = (d.B + per_wave - 1) / per_wave;
  hipLaunchKernelGGL((factor_row_kernel<R, NC, NR, DIAG, FULL>), dim3(grid), dim3(kWave), 0, s, d, (const R*)w.am,
                     (const R*)w.dm, q.A0, rho, sigma, rho_f_factor, ctl, w.thinv);
}

// DIAG and FULL (nx + m == NR) select the specialised forms; the wide forms
// (NR > NC) always test their rows
template <typename R, int NC, int NR>
void launch_factor_row_nc(hipStream_t s, const Dims& d, const DirectWs<R>& w, const QPDev<R>& q, const R* rho,
                          R sigma, R rho_f_factor, int32_t* ctl, bool diag) {
  const bool full = NR == NC && d.nx + d.m == NR;
  if (diag) {
    if (full)
      launch_factor_row_k<R, NC, NR, true, NR == NC>(s, d, w, q, rho, sigma, rho_f_factor, ctl);
    else
      launch_factor_row_k<R, NC, NR, true, false>(s, d, w, q, rho, sigma, rho_f_factor, ctl);
  } else {
    if (full)
      launch_factor_row_k<R, NC, NR, false, NR == NC>(s, d, w, q, rho, sigma, rho_f_factor, ctl);
    else
      launch_factor_row_k<R, NC, NR, false, false>(s, d, w, q, rho, sigma, rho_f_factor, ctl);
  }
}

// fp64 factorization from the stage records (explicit-integrator structure):
// one problem per 16-lane row (factor_rows.hpp), or with `groups` the
// lane-group kernel with P problems per wavefront
template <typename R>
int launch_factor_std(hipStream_t s, const Dims& d, const DirectWs<R>& w, const QPDev<R>& q, const R* rho,
                      R sigma, R rho_f_factor, int32_t* ctl, int P, bool diag, bool groups = false) {
  if (!groups) {
    switch (d.n) {
      case 6: launch_factor_row_nc<R, 6, 6>(s, d, w, q, rho, sigma, rho_f_factor, ctl, diag); break;
      case 9:
        if (stream_wide(d))
          launch_factor_row_nc<R, 9, kWideRows>(s, d, w, q, rho, sigma, rho_f_factor, ctl, diag);
        else
          launch_factor_row_nc<R, 9, 9>(s, d, w, q, rho, sigma, rho_f_factor, ctl, diag);
        break;
      case 16:
        if (stream_wide(d))
          launch_factor_row_nc<R, 16, kWide16Rows>(s, d, w, q, rho, sigma, rho_f_factor, ctl, diag);
        else
          launch_factor_row_nc<R, 16, 16>(s, d, w, q, rho, sigma, rho_f_factor, ctl, diag);
        break;
      default: launch_factor_row_nc<R, 17, 17>(s, d, w, q, rho, sigma, rho_f_factor, ctl, diag); break;
    }
    return launch_status();
  }
  switch (d.n) {
    case 6: launch_factor_std_nc<R, 6>(s, d, w, q, rho, sigma, rho_f_factor, ctl, P, diag); break;
    case 9:
      if (stream_wide(d))
        launch_factor_std_nc<R, 9, kWideRows, kWideMaxM>(s, d, w, q, rho, sigma, rho_f_factor, ctl, P, diag);
      else
        launch_factor_std_nc<R, 9>(s, d, w, q, rho, sigma, rho_f_factor, ctl, P, diag);
      break;
    case 16:
      if (stream_wide(d))
        launch_factor_std_nc<R, 16, kWide16Rows, kWide16MaxM>(s, d, w, q, rho, sigma, rho_f_factor, ctl, P, diag);
      else
        launch_factor_std_nc<R, 16>(s, d, w, q, rho, sigma, rho_f_factor, ctl, P, diag);
      break;
    default: launch_factor_std_nc<R, 17>(s, d, w, q, rho, sigma, rho_f_factor, ctl, P, diag); break;
  }
  return launch_status();
}

// dr: the record dims, A0r: A0 with rows of the records' width
template <typename R>
StreamArgs<R> stream_args(const AdmmArgs<R>& a, const DirectWs<R>& w, const Dims& dr, const R* A0r, bool diag,
                          const tmpc_sqp_step* sq) {
  StreamArgs<R> s;
  s.chk_conv = sq ? static_cast<R*>(sq->conv) : nullptr;
  s.chk_eq = sq ? static_cast<R*>(sq->eq_err) : nullptr;
  s.chk_iq = sq ? static_cast<R*>(sq->ineq_err) : nullptr;
  s.chk_g = sq ? static_cast<R*>(sq->g_out) : nullptr;
  s.act_in = sq ? sq->active_in : nullptr;
  s.act_out = sq ? sq->active_out : nullptr;
  s.chk_tol = sq ? (R)sq->tol : R(0);
  s.d = dr;
  s.diag = diag ? 1 : 0;
  s.th = w.thinv;
  s.dm = w.dm;
  s.am = w.am;
  s.rv = w.rv;
  s.A0 = A0r;
  s.c0 = a.qp.c0;
  s.slack_w = a.qp.slack_w;
  s.y_f0 = a.st.y_f0;
  s.rho = a.st.rho;
  s.ctl = a.ctl;
  s.res = a.res;
  s.iters_out = a.iters_out;
  s.sigma = a.sigma;
  s.alpha = a.alpha;
  s.rho_f_factor = a.rho_f_factor;
  s.eps_abs = a.eps_abs;
  s.eps_rel = a.eps_rel;
  s.rho_min = a.rho_min;
  s.rho_max = a.rho_max;
  s.rho_tol = a.rho_tol;
  s.max_iter = a.max_iter;
  s.check_every = a.check_every;
  s.adapt_every = a.adapt_every;
  s.use_slack = a.use_slack;
  s.it_lo = a.it_lo;
  s.it_hi = a.it_hi;
  s.first_chunk = a.first_chunk;
  s.amask = w.amask;
  s.ac = w.ac;
  return s;
}

// Iterations after which a rho change (and so a refactorization) can happen:
// it >= 2, it % adapt_every == 0 and it % check_every == 0 (admm.py:504-508).
std::vector<int> chunk_bounds(int max_iter, int check_every, int adapt_every) {
  const int last = std::max(max_iter, 1);  // cond_fun always runs iteration 0
  std::vector<int> b{0};
  if (adapt_every > 0)
    for (int it = 2; it < last; ++it) {
      const bool ck = check_every > 0 ? (it % check_every == 0) : (it == 0);
      if (it % adapt_every == 0 && ck) b.push_back(it + 1);
    }
  if (b.back() != last) b.push_back(last);
  return b;
}

template <typename R>
int sqp_check_impl(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const R* x, const R* y0, const R* yf,
                   const R* yg, const R* slack, double slack_w, uint32_t flags, R* conv, R* eq, R* iq, R* gout,
                   const R* slack_wp = nullptr);

template <typename R>
int quad_impl(hipStream_t s, int B, int N, const R* states, int64_t ls, const R* controls, int64_t lu, double dt,
              const double* params, R* Am, R* c, QuadRecOut<R> rec);

// The quadrotor model of an SQP step that linearizes its own dynamics rows.
struct QuadLin {
  double dt;
  const double* params;  // host, 7
};

template <typename R>
int obstacle_lin_impl(hipStream_t s, int B, int N, int nx, int nu, int dim, int K, const R* states, int ls,
                      const R* centers, const R* radii, int m, int row0, R* G, R* l, R* u, ObsRecOut<R> rec);

// The obstacle rows of an SQP step that linearizes them itself: K spheres in
// the first dim state coordinates, rows row0 .. row0 + K - 1 of each stage.
struct ObsLin {
  int dim, K, row0;
  const void* centers;  // (B, K, dim) of the QP's type
  const void* radii;    // (B, K)
};

// sq != nullptr: one SQP step -- the first-order check of the input iterate,
// the activity test, and the ADMM solve of the problems that pass it.  ql
// != nullptr (with sq): the QP's A_minus and c are outputs, the quadrotor's
// RK4 linearization at the input iterate (the state's x rows [x_t; u_t]),
// written before anything reads them and, where warm stage records take
// them, into the records as well (no repack).  ol != nullptr (with sq): the
// same for the obstacle rows of G, l and u (the other rows are inputs).
template <typename R>
int admm_direct_impl(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp,
                     const tmpc_state* in, tmpc_state* out, uint32_t* iters,
                     const tmpc_admm_cfg* cfg, void* ws, size_t wsb, const tmpc_sqp_step* sq = nullptr,
                     const QuadLin* ql = nullptr, const ObsLin* ol = nullptr, bool overlap = true) {
  if (!dims_ok(dims)) return TMPC_EBADSHAPE;
  if (!cfg || !iters || !qp_ok(qp, dims->m) || !state_ok(in, dims->m) || !state_ok(out, dims->m))
    return TMPC_EBADARG;
  // conv NULL: the activity is given (active_in), no check is evaluated
  if (sq && (!sq->active_out || (!sq->conv && (sq->eq_err || sq->ineq_err || sq->g_out)))) return TMPC_EBADARG;
  const bool given = sq && !sq->conv;
  if (cfg->use_slack && dims->m > 0 && !qp->slack_weight) return TMPC_EBADARG;
  const Dims d = to_dims(dims);
  if (!ws || wsb < direct_ws_bytes<R>(d)) return TMPC_EWORKSPACE;
  int st = copy_state<R>(s, d, in, out);
  if (st) return st;
  const DirectWs<R> w = carve_direct<R>(ws, wsb, d);
  AdmmArgs<R> a;
  a.d = d;
  a.qp = to_qp<R>(qp);
  a.st = to_state<R>(out);
  a.thinv = w.thinv;
  a.w = w.w;
  a.gam = w.gam;
  a.ctl = w.ctl;
  a.res = w.res;
  a.iters_out = iters;
  a.sigma = (R)cfg->sigma;
  a.alpha = (R)cfg->alpha;
  a.rho_f_factor = (R)cfg->rho_f_factor;
  a.eps_abs = (R)cfg->eps_abs;
  a.eps_rel = (R)cfg->eps_rel;
  a.rho_min = (R)cfg->rho_min;
  a.rho_max = (R)cfg->rho_max;
  a.rho_tol = (R)cfg->adaptive_rho_tolerance;
  a.max_iter = cfg->max_iter;
  a.check_every = cfg->check_every;
  a.adapt_every = cfg->adapt_rho_every;
  a.use_slack = cfg->use_slack ? 1 : 0;
  a.g = std::max(d.n, d.m);
  a.P = kWave / a.g;
  a.act = nullptr;
  const bool std_dyn = (cfg->flags & TMPC_FLAG_STD_DYNAMICS) != 0;
  const int fp = factor_problems_per_wave(d.B, cfg->flags);
  const bool fgroups = (cfg->flags & TMPC_FLAG_FACTOR_GROUPS) != 0;
  const bool diag = (cfg->flags & TMPC_FLAG_DIAG_COST) != 0;
  const bool const_g = (cfg->flags & TMPC_FLAG_CONST_G) != 0 && d.m > 0;
  // the streaming path works on records of width dr.n >= d.n (dummies past n)
  const Dims dr = stream_record_dims(d);
  int sp = stream_problems_per_wave(d.B, cfg->flags, stream_wide(dr) && dr.n == 9);
  if (stream_wide(dr) && (cfg->flags & TMPC_FLAG_STREAM_P(3)) == 0)
    sp = std::min(sp, kWave / stream_wide_rows(dr));  // the wide forms' groups are larger
  const bool stream = std_dyn && (cfg->flags & TMPC_FLAG_GENERIC_KERNEL) == 0 && stream_ok<R>(dr, sp, diag);
  // the AINV form: asked for, with the resident G rows, at most two problems
  // per wavefront, and the whole workspace
  const bool ainv = stream && const_g && (cfg->flags & TMPC_FLAG_INVARIANT_A) != 0 && ainv_shape_ok(dr, sizeof(R)) && sp <= 2 &&
                    w.ac != nullptr;
  const bool pad = dr.n != d.n;
  QPDev<R> qr = a.qp;  // the QP as the record kernels read it
  if (pad) qr.A0 = w.a0p;
  // warm stage records that a model's own linearization writes directly
  const bool rows_in_records = stream && (cfg->flags & TMPC_FLAG_WARM_RECORDS) != 0 && !pad;
  bool dyn_in_records = false, ineq_in_records = false;
  if (ql) {
    if (d.n != 17 || d.nx != 13) return TMPC_EBADSHAPE;
    QuadRecOut<R> rec{};
    dyn_in_records = rows_in_records;
    if (dyn_in_records) {
      const RecGeom g = rec_geom(dr, diag);
      rec.am = w.am;
      rec.rv = w.rv;
      rec.amp = g.amp;
      rec.rvp = g.rvp;
      rec.c_off = g.c;
    }
    st = quad_impl<R>(s, d.B, d.N, a.st.x, d.n, a.st.x + 13, d.n, ql->dt, ql->params, const_cast<R*>(a.qp.Am),
                      const_cast<R*>(a.qp.c), rec);
    if (st) return st;
  }
  if (ol && ol->K > 0) {
    ObsRecOut<R> rec{};
    ineq_in_records = rows_in_records;
    if (ineq_in_records) {
      const RecGeom g = rec_geom(dr, diag);
      rec.am = w.am;
      rec.rv = w.rv;
      rec.amp = g.amp;
      rec.rvp = g.rvp;
      rec.g_off = (d.nx + ol->row0) * dr.n;  // the G rows follow the A_minus rows
      rec.l_off = g.l + ol->row0;
      rec.u_off = g.u + ol->row0;
    }
    st = obstacle_lin_impl<R>(s, d.B, d.N, d.nx, d.n - d.nx, ol->dim, ol->K, a.st.x, d.n,
                              static_cast<const R*>(ol->centers), static_cast<const R*>(ol->radii), d.m, ol->row0,
                              const_cast<R*>(a.qp.G), const_cast<R*>(a.qp.l), const_cast<R*>(a.qp.u), rec);
    if (st) return st;
  }
  if (given) {
    // the activity as given: act_out = act_in, which the kernels read as the
    // per-problem start state (the streaming kernel reads act_in itself)
    hipLaunchKernelGGL((sqp_activity_kernel<R>), dim3((d.B + 255) / 256), dim3(256), 0, s, d.B, (const R*)nullptr,
                       R(0), sq->active_in, sq->active_out);
    st = launch_status();
    if (st) return st;
    if (!stream) a.act = sq->active_out;
  } else if (sq && !stream) {
    // generic path: the check kernel on the input iterate, then the activity
    // test, which the ADMM kernel reads as its per-problem start state
    const bool slack = cfg->use_slack && d.m > 0;
    st = sqp_check_impl<R>(s, dims, qp, a.st.x, a.st.y_f0, a.st.y_f, a.st.y_g, slack ? a.st.xi : nullptr, 0.0,
                           cfg->flags, static_cast<R*>(sq->conv), static_cast<R*>(sq->eq_err),
                           static_cast<R*>(sq->ineq_err), static_cast<R*>(sq->g_out),
                           slack ? static_cast<const R*>(qp->slack_weight) : nullptr);
    if (st) return st;
    hipLaunchKernelGGL((sqp_activity_kernel<R>), dim3((d.B + 255) / 256), dim3(256), 0, s, d.B,
                       (const R*)sq->conv, (R)sq->tol, sq->active_in, sq->active_out);
    st = launch_status();
    if (st) return st;
    a.act = sq->active_out;
  }
  if (stream && (cfg->flags & TMPC_FLAG_WARM_RECORDS)) {
    const unsigned gx = (unsigned)((d.B + kRepackProblems - 1) / kRepackProblems);
    // the A_minus and c rows are rewritten unless they did not change or the
    // quadrotor step already wrote them; G, l and u when they changed, unless
    // the obstacle step wrote them (its other rows are the previous call's)
    const bool dyn_rows = !dyn_in_records && (cfg->flags & TMPC_FLAG_WARM_SAME_DYNAMICS) == 0;
    const bool ineq_rows = d.m > 0 && !ineq_in_records && ((cfg->flags & TMPC_FLAG_WARM_INEQ) != 0 || ol);
    if (ineq_rows)
      hipLaunchKernelGGL((stage_repack_dynamics_kernel<R, true>), dim3(gx, (unsigned)d.T), dim3(256), 0, s, dr,
                         a.qp.Am, a.qp.c, a.qp.G, a.qp.l, a.qp.u, w.am, w.rv, diag ? 1 : 0, dyn_rows ? 1 : 0);
    else if (dyn_rows)
      hipLaunchKernelGGL((stage_repack_dynamics_kernel<R, false>), dim3(gx, (unsigned)d.N), dim3(256), 0, s, dr,
                         a.qp.Am, a.qp.c, a.qp.G, a.qp.l, a.qp.u, w.am, w.rv, diag ? 1 : 0, 1);
    st = launch_status();
    if (st) return st;
  } else if (stream) {
    hipLaunchKernelGGL((stage_pack_kernel<R>), dim3((unsigned)((d.B + kPackWaves - 1) / kPackWaves), (unsigned)d.T),
                       dim3(kWave * kPackWaves), 0, s, dr, a.qp, a.st, w.am, w.rv, w.dm, diag ? 1 : 0,
                       pad ? w.a0p : (R*)nullptr);
    st = launch_status();
    if (st) return st;
  }
  // the stage-invariant entries of this call's A_minus rows: partial masks
  // in the compressed-run region (written later by the streaming kernel),
  // then their OR (kernels only, no memset, so the call can be captured).
  // They read the stage records the factorization reads (and write nothing
  // it touches), so they run beside it on the side stream where there is
  // one: forked after the records are written, joined before the iterations.
  auto launch_ainv = [&](hipStream_t q) {
    if (d.N > 1) {
      const int nparts = (d.B + kAinvWaves - 1) / kAinvWaves;
      uint32_t* part = reinterpret_cast<uint32_t*>(w.ac);
      hipLaunchKernelGGL((ainv_partial_kernel<R>), dim3((unsigned)nparts), dim3(kWave * kAinvWaves), 0, q, dr,
                         (const R*)w.am, part);
      hipLaunchKernelGGL(ainv_reduce_kernel, dim3(1), dim3(256), 0, q, (const uint32_t*)part, nparts, w.amask);
    } else {
      hipLaunchKernelGGL((fill_kernel<uint32_t>), dim3(1), dim3(256), 0, q, w.amask, (size_t)kAinvWords, 0u);
    }
    return launch_status();
  };
  SideStream* side = ainv && overlap ? side_stream(s) : nullptr;
  if (side) {
    if (hipEventRecord(side->fork, s) != hipSuccess || hipStreamWaitEvent(side->q, side->fork, 0) != hipSuccess)
      return TMPC_ELAUNCH;
    st = launch_ainv(side->q);
    if (st) return st;
    if (hipEventRecord(side->join, side->q) != hipSuccess) return TMPC_ELAUNCH;
  }
  st = stream ? launch_factor_std<R>(s, dr, w, qr, a.st.rho, a.sigma, a.rho_f_factor, nullptr, fp, diag, fgroups)
              : launch_factor_qp<R>(s, d, a.qp, a.st.rho, a.sigma, a.rho_f_factor, nullptr, w.thinv);
  if (side && hipStreamWaitEvent(s, side->join, 0) != hipSuccess) return TMPC_ELAUNCH;
  if (st) return st;
  if (ainv && !side) {
    st = launch_ainv(s);
    if (st) return st;
  }
  const std::vector<int> bounds = chunk_bounds(cfg->max_iter, cfg->check_every, cfg->adapt_rho_every);
  if (g_iter_events[0] && hipEventRecord(g_iter_events[0], s) != hipSuccess) return TMPC_ELAUNCH;
  for (size_t c = 0; c + 1 < bounds.size(); ++c) {
    if (c > 0) {
      st = stream ? launch_factor_std<R>(s, dr, w, qr, a.st.rho, a.sigma, a.rho_f_factor, w.ctl, fp, diag, fgroups)
                  : launch_factor_qp<R>(s, d, a.qp, a.st.rho, a.sigma, a.rho_f_factor, w.ctl, w.thinv);
      if (st) return st;
    }
    a.it_lo = bounds[c];
    a.it_hi = bounds[c + 1];
    a.first_chunk = c == 0 ? 1 : 0;
    if (stream)
      launch_stream<R>(s, stream_args<R>(a, w, dr, qr.A0, diag, sq), sp, const_g, ainv);
    else if (std_dyn)
      launch_chunk<R, true>(s, a);
    else
      launch_chunk<R, false>(s, a);
    st = launch_status();
    if (st) return st;
  }
  if (g_iter_events[1] && hipEventRecord(g_iter_events[1], s) != hipSuccess) return TMPC_ELAUNCH;
  if (stream) {  // the unpack also sets the non-finite flags
    hipLaunchKernelGGL((stage_unpack_kernel<R>),
                       dim3((unsigned)((d.B + kUnpackProblems - 1) / kUnpackProblems), (unsigned)d.T), dim3(256), 0,
                       s, dr, (const R*)w.rv, a.st, iters);
    return launch_status();
  }
  return launch_nonfinite_flags<R>(s, d, a.st, iters);
}

// ------------------------------------------------------- allocation-free ----
// Device address of `scratch` on each device, looked up once per device with
// that device current (each GPU holds its own copy at its own address).
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int noalloc_scratch(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TMPC_ELAUNCH;
  if (s != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess) return TMPC_EBADARG;
    if ((int)sdev != dev) return TMPC_EBADARG;  // the stream belongs to another device
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return TMPC_ELAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TMPC_OK;
}

// The kernels of tmpc_admm_direct_* initialise every workspace word they read
// (per-problem control words and residuals in the first chunk, the factor and
// stage records before the iterations), so the scratch needs no clearing.
template <typename R>
int admm_direct_noalloc_impl(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                             tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg) {
  if (!dims_ok(dims)) return TMPC_EBADSHAPE;
  if (!cfg) return TMPC_EBADARG;
  if (cfg->flags & TMPC_FLAG_WARM_RECORDS) return TMPC_EBADARG;
  const size_t need = direct_ws_bytes_full<R>(to_dims(dims));
  if (need > TMPC_NOALLOC_SCRATCH_BYTES) return TMPC_ESCRATCH;
  void* ws = nullptr;
  const int st = noalloc_scratch(s, &ws);
  if (st) return st;
  // everything on the caller's stream: no side stream is created here
  return admm_direct_impl<R>(s, dims, qp, in, out, iters, cfg, ws, TMPC_NOALLOC_SCRATCH_BYTES, nullptr, nullptr,
                             nullptr, false);
}

// ---------------------------------------------------------------- blktri ----
template <typename R>
int blktri_factor_impl(hipStream_t s, int B, int T, int n, const R* S, void* ws, size_t wsb) {
  tmpc_dims td{B, T, n, 1, 1, 0};
  if (!dims_ok(&td)) return TMPC_EBADSHAPE;
  if (!S) return TMPC_EBADARG;
  const Dims d = to_dims(&td);
  if (!ws || wsb < align_up((size_t)T * B * th_pitch(n) * sizeof(R))) return TMPC_EWORKSPACE;
  QPDev<R> q{};
  const size_t smem = factor_smem_bytes(d);
  lds_optin(factor_kernel<R, SRC_S>, smem);
  hipLaunchKernelGGL((factor_kernel<R, SRC_S>), dim3(B), dim3(kWave), smem, s, d, q, S,
                     (const R*)nullptr, R(0), R(0), (int32_t*)nullptr, static_cast<R*>(ws));
  return launch_status();
}

template <typename R, int NC>
void launch_blktri_solve_nc(hipStream_t s, const Dims& d, int g, int P, const R* S, const R* th,
                            const R* rhs, R* x) {
  hipLaunchKernelGGL((blktri_solve_kernel<R, NC>), dim3((d.B + P - 1) / P), dim3(kWave), 0, s, d, g,
                     P, S, th, rhs, x);
}

template <typename R>
int blktri_solve_impl(hipStream_t s, int B, int T, int n, const R* S, const R* rhs, R* x,
                      const void* ws, size_t wsb) {
  tmpc_dims td{B, T, n, 1, 1, 0};
  if (!dims_ok(&td)) return TMPC_EBADSHAPE;
  if (!S || !rhs || !x) return TMPC_EBADARG;
  const Dims d = to_dims(&td);
  if (!ws || wsb < align_up((size_t)T * B * th_pitch(n) * sizeof(R))) return TMPC_EWORKSPACE;
  const R* th = static_cast<const R*>(ws);
  const int g = n, P = kWave / n;
  switch (n) {
    case 6: launch_blktri_solve_nc<R, 6>(s, d, g, P, S, th, rhs, x); break;
    case 9: launch_blktri_solve_nc<R, 9>(s, d, g, P, S, th, rhs, x); break;
    case 16: launch_blktri_solve_nc<R, 16>(s, d, g, P, S, th, rhs, x); break;
    case 17: launch_blktri_solve_nc<R, 17>(s, d, g, P, S, th, rhs, x); break;
    default: launch_blktri_solve_nc<R, 0>(s, d, g, P, S, th, rhs, x); break;
  }
  return launch_status();
}

// --------------------------------------------------------------- adjoint ----
KktDims kkt_dims(const Dims& d) {
  KktDims k;
  k.B = d.B;
  k.T = d.T;
  k.N = d.N;
  k.n = d.n;
  k.nx = d.nx;
  k.n0 = d.n0;
  k.m = d.m;
  k.p = std::max(d.n0, d.nx);
  k.nb = d.n + k.p + d.m;
  return k;
}

template <typename R>
size_t adjoint_ws_bytes(const Dims& d) {
  const KktDims k = kkt_dims(d);
  const size_t B = d.B, T = d.T, nb = k.nb;
  return align_up(B * T * nb * 3 * nb * sizeof(R)) + align_up(T * B * th_pitch(k.nb) * sizeof(R)) +
         5 * align_up(B * T * nb * sizeof(R)) + align_up(B * sizeof(R));
}

// The rows-in-lanes KKT factorization and solves (kkt_factor.hpp) for n <= 16
// and nb <= 32, reading the QP blocks directly: block capacities NC (Z) and
// NBC (rows per problem), P problems per wavefront.  Shapes they do not cover take the assembled-matrix path
// (kkt_assemble_kernel, factor_kernel, blktri_solve_kernel).
// 0: not covered; 1, 2, 3: the (NC, NBC) capacities (9, 18), (9, 32), (16, 32)
inline int kkt_rows_form(const KktDims& k) {
  if (k.n <= 9 && k.nb <= 18) return 1;
  if (k.n <= 9 && k.nb <= 32) return 2;
  if (k.n <= 16 && k.nb <= 32) return 3;
  return 0;
}
// Problems per wavefront: enough that the launch holds about one wavefront per
// SIMD (1024 on the chip; the factorization's registers allow one per SIMD,
// and packing beats a second resident wavefront for the sweeps as well: 374 vs
// 489 us per solve at B = 2048), up to the groups a wavefront holds.
inline int kkt_rows_p(const KktDims& k) {
  const int pmax = kkt_rows_form(k) == 1 ? 3 : 2;  // 64 / NBC groups
  return std::max(1, std::min(pmax, (k.B + 1023) / 1024));
}
inline unsigned kkt_rows_grid(const KktDims& k, int P) { return (unsigned)((k.B + P - 1) / P); }

// P in {1, 2, 3} (3 where three groups of NBC lanes fit a wavefront)
#define TMPC_KKT_ROWS_LAUNCH(KERNEL, ...)                                                                      \
  do {                                                                                                        \
    if constexpr (3 * NBC <= kWave) {                                                                         \
      if (P >= 3) {                                                                                           \
        hipLaunchKernelGGL((KERNEL<R, NC, NBC, 3>), dim3(kkt_rows_grid(k, 3)), dim3(kWave), 0, s, k, __VA_ARGS__); \
        break;                                                                                                \
      }                                                                                                       \
    }                                                                                                         \
    if (P >= 2)                                                                                               \
      hipLaunchKernelGGL((KERNEL<R, NC, NBC, 2>), dim3(kkt_rows_grid(k, 2)), dim3(kWave), 0, s, k, __VA_ARGS__);   \
    else                                                                                                      \
      hipLaunchKernelGGL((KERNEL<R, NC, NBC, 1>), dim3(k.B), dim3(kWave), 0, s, k, __VA_ARGS__);                   \
  } while (0)

template <typename R, int NC, int NBC>
void launch_kkt_rows_nc(hipStream_t s, const KktDims& k, int P, const QPDev<R>& q, const R* shift, R* th) {
  TMPC_KKT_ROWS_LAUNCH(factor_kkt_rows_kernel, q, shift, th);
}

template <typename R, int NC, int NBC>
void launch_kkt_solve_nc(hipStream_t s, const KktDims& k, int P, const QPDev<R>& q, const R* th, const R* rhs,
                         R* x) {
  TMPC_KKT_ROWS_LAUNCH(kkt_solve_rows_kernel, q, th, rhs, x);
}

// the residual's units are (problem, stage) pairs: as many per wavefront as fit
template <typename R, int NC, int NBC>
void launch_kkt_residual_nc(hipStream_t s, const KktDims& k, const QPDev<R>& q, const R* x, R* r) {
  constexpr int PU = kWave / NBC;
  const unsigned grid = (unsigned)(((size_t)k.B * k.T + PU - 1) / PU);
  hipLaunchKernelGGL((kkt_residual_rows_kernel<R, NC, NBC, PU>), dim3(grid), dim3(kWave), 0, s, k, q, x, r);
}
#undef TMPC_KKT_ROWS_LAUNCH

// which: 0 factor (writes th), 1 solve (in: right-hand side, null for the
// system's own; out: x), 2 residual (in: x; out: r)
template <typename R>
void launch_kkt_rows(hipStream_t s, const KktDims& k, int which, const QPDev<R>& q, const R* shift, R* th,
                     const R* in, R* out) {
  const int P = kkt_rows_p(k);
  switch (kkt_rows_form(k) * 4 + which) {
    case 4: launch_kkt_rows_nc<R, 9, 18>(s, k, P, q, shift, th); break;
    case 5: launch_kkt_solve_nc<R, 9, 18>(s, k, P, q, th, in, out); break;
    case 6: launch_kkt_residual_nc<R, 9, 18>(s, k, q, in, out); break;
    case 8: launch_kkt_rows_nc<R, 9, 32>(s, k, P, q, shift, th); break;
    case 9: launch_kkt_solve_nc<R, 9, 32>(s, k, P, q, th, in, out); break;
    case 10: launch_kkt_residual_nc<R, 9, 32>(s, k, q, in, out); break;
    case 12: launch_kkt_rows_nc<R, 16, 32>(s, k, P, q, shift, th); break;
    case 13: launch_kkt_solve_nc<R, 16, 32>(s, k, P, q, th, in, out); break;
    case 14: launch_kkt_residual_nc<R, 16, 32>(s, k, q, in, out); break;
    default: break;
  }
}

template <typename R>
int adjoint_impl(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, R* dz, R* mult, double reg,
                 int32_t refine, uint32_t flags, void* ws, size_t wsb) {
  if (!dims_ok(dims)) return TMPC_EBADSHAPE;
  if (!qp || !qp->D || !qp->E || !qp->q || !qp->A0 || !qp->A_minus || !qp->A_plus || !dz || !mult)
    return TMPC_EBADARG;
  if (dims->m > 0 && !qp->G) return TMPC_EBADARG;
  const Dims d = to_dims(dims);
  const KktDims k = kkt_dims(d);
  if (k.nb > kWave) return TMPC_EBADSHAPE;
  if ((size_t)d.B * d.T > (size_t)INT32_MAX) return TMPC_EBADSHAPE;  // residual units are counted in int
  if (!ws || wsb < adjoint_ws_bytes<R>(d)) return TMPC_EWORKSPACE;
  const bool f64 = sizeof(R) == 8;
  const R eps = reg > 0 ? (R)reg : R(1e-12);
  const int steps = refine >= 0 ? refine : (f64 ? 2 : 3);
  const size_t B = d.B, T = d.T, nb = k.nb, L = B * T * nb;
  Carver c{static_cast<char*>(ws)};
  R* K = c.take<R>(B * T * nb * 3 * nb);
  R* th = c.take<R>(T * B * th_pitch(k.nb));
  R* dreg = c.take<R>(L);
  R* rhs = c.take<R>(L);
  R* x = c.take<R>(L);
  R* r = c.take<R>(L);
  R* dx = c.take<R>(L);
  R* shift = c.take<R>(B);
  const QPDev<R> q = to_qp<R>(qp);
  hipLaunchKernelGGL((kkt_scale_kernel<R>), dim3(d.B), dim3(256), 0, s, k, q.D, eps, shift);
  // rows in lanes from the QP blocks (kkt_factor.hpp) where the shape allows
  // it; else the assembled stage-block matrix, factor_kernel (factor.hpp,
  // SRC_S) and blktri_solve_kernel.  TMPC_FLAG_GENERIC_KERNEL selects the
  // latter (cross-checks).
  const bool rows = (flags & TMPC_FLAG_GENERIC_KERNEL) == 0 && kkt_rows_form(k) != 0;
  Dims kd{d.B, d.T, d.N, k.nb, 1, 1, 0, k.nb};
  if (rows) {
    launch_kkt_rows<R>(s, k, 0, q, shift, th, nullptr, nullptr);
    launch_kkt_rows<R>(s, k, 1, q, nullptr, th, nullptr, x);
  } else {
    hipLaunchKernelGGL((kkt_assemble_kernel<R>), dim3(d.B * d.T), dim3(256), 0, s, k, q, shift, K, dreg, rhs);
    const size_t smem = factor_smem_bytes(kd);
    lds_optin(factor_kernel<R, SRC_S>, smem);
    hipLaunchKernelGGL((factor_kernel<R, SRC_S>), dim3(d.B), dim3(kWave), smem, s, kd, QPDev<R>{}, (const R*)K,
                       (const R*)nullptr, R(0), R(0), (int32_t*)nullptr, th);
    launch_blktri_solve_nc<R, 0>(s, kd, k.nb, kWave / k.nb, K, th, rhs, x);
  }
  int st = launch_status();
  if (st) return st;
  for (int it = 0; it < steps; ++it) {
    if (rows) {
      launch_kkt_rows<R>(s, k, 2, q, nullptr, th, x, r);
      launch_kkt_rows<R>(s, k, 1, q, nullptr, th, r, dx);
    } else {
      const int Pg = kWave / k.nb;
      hipLaunchKernelGGL((kkt_residual_kernel<R>), dim3((k.B + Pg - 1) / Pg), dim3(kWave), 0, s, k, Pg, K, dreg,
                         rhs, x, r);
      launch_blktri_solve_nc<R, 0>(s, kd, k.nb, kWave / k.nb, K, th, r, dx);
    }
    hipLaunchKernelGGL((axpy_kernel<R>), dim3((unsigned)((L + 255) / 256)), dim3(256), 0, s, L, (const R*)dx, x);
  }
  hipLaunchKernelGGL((kkt_unpack_kernel<R>), dim3(d.B), dim3(256), 0, s, k, (const R*)x, dz, mult);
  return launch_status();
}

// ----------------------------------------------------------- PCG family ----
template <typename R>
size_t pcg_vec_bytes(const Dims& d) { return 5 * align_up((size_t)d.B * d.T * d.n * sizeof(R)); }

template <typename R>
size_t admm_pcg_ws_bytes(const Dims& d) {
  const size_t B = d.B, T = d.T, n = d.n;
  return 2 * align_up(B * T * n * 3 * n * sizeof(R)) + 2 * align_up(T * B * n * sizeof(R)) +
         align_up(B * 4 * sizeof(int32_t)) + align_up(B * 8 * sizeof(R)) + pcg_vec_bytes<R>(d);
}

template <typename R>
PcgVecs<R> carve_vecs(Carver& c, const Dims& d, R* x) {
  const size_t L = (size_t)d.B * d.T * d.n;
  PcgVecs<R> v;
  v.x = c.take<R>(L);
  if (x) v.x = x;
  v.r = c.take<R>(L);
  v.p = c.take<R>(L);
  v.q = c.take<R>(L);
  v.rt = c.take<R>(L);
  return v;
}

template <typename R>
int launch_schur_build(hipStream_t s, const Dims& d, const QPDev<R>& q, const R* rho, R sigma, R rfac,
                       int32_t* ctl, R* S, R* Phi) {
  const size_t smem = factor_smem_bytes(d);
  lds_optin(schur_build_kernel<R>, smem);
  hipLaunchKernelGGL((schur_build_kernel<R>), dim3(d.B), dim3(kWave), smem, s, d, q, rho, sigma, rfac, ctl,
                     S, Phi);
  return launch_status();
}

template <typename R>
int schur_build_impl(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const R* rho, double sigma,
                     double rfac, R* S, R* Phi) {
  if (!dims_ok(dims)) return TMPC_EBADSHAPE;
  if (!qp_ok(qp, dims->m) || !rho || !S || !Phi) return TMPC_EBADARG;
  const Dims d = to_dims(dims);
  return launch_schur_build<R>(s, d, to_qp<R>(qp), rho, (R)sigma, (R)rfac, nullptr, S, Phi);
}

template <typename R, int NC>
void launch_pcg_nc(hipStream_t s, const Dims& d, int g, int P, const R* S, const R* Phi, const R* rhs,
                   const R* x0, const PcgVecs<R>& v, uint32_t* iters, R eps, int max_iter) {
  hipLaunchKernelGGL((pcg_kernel<R, NC>), dim3((d.B + P - 1) / P), dim3(kWave), 0, s, d, g, P, S, Phi, rhs,
                     x0, v, iters, eps, max_iter);
}

template <typename R>
int schur_pcg_impl(hipStream_t s, int B, int T, int n, const R* S, const R* Phi, const R* rhs, const R* x0,
                   R* x, uint32_t* iters, double eps, int max_iter, void* ws, size_t wsb) {
  tmpc_dims td{B, T, n, 1, 1, 0};
  if (!dims_ok(&td)) return TMPC_EBADSHAPE;
  if (!S || !Phi || !rhs || !x0 || !x || !iters) return TMPC_EBADARG;
  if (x == x0) return TMPC_EBADARG;
  const Dims d = to_dims(&td);
  if (!ws || wsb < pcg_vec_bytes<R>(d)) return TMPC_EWORKSPACE;
  Carver c{static_cast<char*>(ws)};
  const PcgVecs<R> v = carve_vecs<R>(c, d, x);
  const int g = n, P = kWave / n;
  switch (n) {
    case 6: launch_pcg_nc<R, 6>(s, d, g, P, S, Phi, rhs, x0, v, iters, (R)eps, max_iter); break;
    case 9: launch_pcg_nc<R, 9>(s, d, g, P, S, Phi, rhs, x0, v, iters, (R)eps, max_iter); break;
    case 16: launch_pcg_nc<R, 16>(s, d, g, P, S, Phi, rhs, x0, v, iters, (R)eps, max_iter); break;
    case 17: launch_pcg_nc<R, 17>(s, d, g, P, S, Phi, rhs, x0, v, iters, (R)eps, max_iter); break;
    default: launch_pcg_nc<R, 0>(s, d, g, P, S, Phi, rhs, x0, v, iters, (R)eps, max_iter); break;
  }
  return launch_status();
}

template <typename R, int NC>
void launch_admm_pcg_nc(hipStream_t s, const AdmmPcgArgs<R>& pa) {
  const int grid = (pa.a.d.B + pa.a.P - 1) / pa.a.P;
  hipLaunchKernelGGL((admm_pcg_chunk_kernel<R, NC>), dim3(grid), dim3(kWave), 0, s, pa);
}

// LDS-resident PCG ADMM (explicit-integrator QPs): one problem per workgroup,
// theta_t rows in LDS when they fit (mode 2), else in the workspace (mode 1).
template <typename R, int NC, bool THL>
int launch_pcg_lds_th(hipStream_t s, const AdmmPcgArgs<R>& pa) {
  const size_t smem = pcg_lds_layout<R>(pa.a.d, THL).bytes;
  if (smem > kMaxLds) return TMPC_EBADSHAPE;
  lds_optin(admm_pcg_lds_kernel<R, NC, THL>, smem);
  hipLaunchKernelGGL((admm_pcg_lds_kernel<R, NC, THL>), dim3(pa.a.d.B), dim3(kPcgThreads), smem, s, pa);
  return launch_status();
}

template <typename R, int NC>
int launch_pcg_lds_nc(hipStream_t s, const AdmmPcgArgs<R>& pa, int mode) {
  return mode == 2 ? launch_pcg_lds_th<R, NC, true>(s, pa) : launch_pcg_lds_th<R, NC, false>(s, pa);
}

template <typename R, int NC>
int launch_pcg_dpp_nc(hipStream_t s, const AdmmPcgArgs<R>& pa) {
  // A_minus in registers for fp32; in LDS for fp64 (the theta rows take the registers)
  constexpr bool amr = sizeof(R) == 4;
  const size_t smem = pcg_dpp_layout<R>(pa.a.d, amr).bytes;
  if (smem > kMaxLds) return TMPC_EBADSHAPE;
  lds_optin(admm_pcg_dpp_kernel<R, NC, amr>, smem);
  hipLaunchKernelGGL((admm_pcg_dpp_kernel<R, NC, amr>), dim3(pa.a.d.B), dim3(kPcgThreads), smem, s, pa);
  return launch_status();
}

template <typename R>
int launch_pcg_dpp(hipStream_t s, const AdmmPcgArgs<R>& pa) {
  switch (pa.a.d.n) {
    case 6: return launch_pcg_dpp_nc<R, 6>(s, pa);
    case 9: return launch_pcg_dpp_nc<R, 9>(s, pa);
    case 16: return launch_pcg_dpp_nc<R, 16>(s, pa);
    default: return TMPC_EBADSHAPE;
  }
}

template <typename R>
bool pcg_dpp_covers(const Dims& d) {
  return pcg_dpp_fits(d) && pcg_dpp_layout<R>(d, sizeof(R) == 4).bytes <= kMaxLds;
}

template <typename R>
int launch_pcg_lds(hipStream_t s, const AdmmPcgArgs<R>& pa, int mode) {
  switch (pa.a.d.n) {
    case 6: return launch_pcg_lds_nc<R, 6>(s, pa, mode);
    case 9: return launch_pcg_lds_nc<R, 9>(s, pa, mode);
    case 16: return launch_pcg_lds_nc<R, 16>(s, pa, mode);
    case 17: return launch_pcg_lds_nc<R, 17>(s, pa, mode);
    default: return TMPC_EBADSHAPE;
  }
}

template <typename R>
int admm_pcg_impl(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                  tmpc_state* out, uint32_t* iters, uint32_t* pcg_iters, const tmpc_admm_cfg* cfg, void* ws,
                  size_t wsb) {
  if (!dims_ok(dims)) return TMPC_EBADSHAPE;
  if (!cfg || !iters || !qp_ok(qp, dims->m) || !state_ok(in, dims->m) || !state_ok(out, dims->m))
    return TMPC_EBADARG;
  if (cfg->use_slack && dims->m > 0 && !qp->slack_weight) return TMPC_EBADARG;
  const Dims d = to_dims(dims);
  if (!ws || wsb < admm_pcg_ws_bytes<R>(d)) return TMPC_EWORKSPACE;
  int st = copy_state<R>(s, d, in, out);
  if (st) return st;
  if (pcg_iters && cfg->max_iter > 0) {
    const size_t cnt = (size_t)d.B * cfg->max_iter;
    if ((cnt + 255) / 256 > (size_t)INT32_MAX) return TMPC_EBADSHAPE;
    hipLaunchKernelGGL((fill_kernel<uint32_t>), dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, s, pcg_iters,
                       cnt, 0u);
    st = launch_status();
    if (st) return st;
  }
  const size_t B = d.B, T = d.T, n = d.n;
  Carver c{static_cast<char*>(ws)};
  R* S = c.take<R>(B * T * n * 3 * n);
  R* Phi = c.take<R>(B * T * n * 3 * n);
  AdmmPcgArgs<R> pa;
  AdmmArgs<R>& a = pa.a;
  a.w = c.take<R>(T * B * n);
  a.gam = c.take<R>(T * B * n);
  a.ctl = c.take<int32_t>(B * 4);
  a.res = c.take<R>(B * 8);
  pa.v = carve_vecs<R>(c, d, nullptr);
  a.d = d;
  a.qp = to_qp<R>(qp);
  a.st = to_state<R>(out);
  a.thinv = nullptr;
  a.iters_out = iters;
  a.sigma = (R)cfg->sigma;
  a.alpha = (R)cfg->alpha;
  a.rho_f_factor = (R)cfg->rho_f_factor;
  a.eps_abs = (R)cfg->eps_abs;
  a.eps_rel = (R)cfg->eps_rel;
  a.rho_min = (R)cfg->rho_min;
  a.rho_max = (R)cfg->rho_max;
  a.rho_tol = (R)cfg->adaptive_rho_tolerance;
  a.max_iter = cfg->max_iter;
  a.check_every = cfg->check_every;
  a.adapt_every = cfg->adapt_rho_every;
  a.use_slack = cfg->use_slack ? 1 : 0;
  a.g = std::max(d.n, d.m);
  a.P = kWave / a.g;
  pa.S = S;
  pa.Phi = Phi;
  pa.pcg_iters = pcg_iters;
  pa.pcg_eps = (R)cfg->pcg_eps;
  pa.pcg_max_iter = cfg->pcg_max_iter;
  const bool std_dyn = (cfg->flags & TMPC_FLAG_STD_DYNAMICS) != 0;
  const int lds_mode = pcg_lds_mode<R>(d);
  // kernel choice: 1 row-broadcast, 2 LDS-resident, 3 chunked (pcg_lds.hpp, pcg.hpp)
  int kern = (int)((cfg->flags >> 10) & 3u);
  if (kern == 0) {
    if (!std_dyn || (cfg->flags & TMPC_FLAG_GENERIC_KERNEL)) kern = 3;
    else kern = pcg_dpp_covers<R>(d) ? 1 : lds_mode ? 2 : 3;
  } else if ((kern == 1 && (!std_dyn || !pcg_dpp_covers<R>(d))) || (kern == 2 && (!std_dyn || !lds_mode))) {
    return TMPC_EBADSHAPE;
  }
  if (kern != 3) {
    // the whole solve in one launch, one problem per workgroup, rho changes
    // rebuilt in the kernel
    if (g_iter_events[0] && hipEventRecord(g_iter_events[0], s) != hipSuccess) return TMPC_ELAUNCH;
    st = kern == 1 ? launch_pcg_dpp<R>(s, pa) : launch_pcg_lds<R>(s, pa, lds_mode);
    if (st) return st;
    if (g_iter_events[1] && hipEventRecord(g_iter_events[1], s) != hipSuccess) return TMPC_ELAUNCH;
    return launch_nonfinite_flags<R>(s, d, a.st, iters);
  }
  st = launch_schur_build<R>(s, d, a.qp, a.st.rho, a.sigma, a.rho_f_factor, nullptr, S, Phi);
  if (st) return st;
  const std::vector<int> bounds = chunk_bounds(cfg->max_iter, cfg->check_every, cfg->adapt_rho_every);
  if (g_iter_events[0] && hipEventRecord(g_iter_events[0], s) != hipSuccess) return TMPC_ELAUNCH;
  for (size_t k = 0; k + 1 < bounds.size(); ++k) {
    if (k > 0) {
      st = launch_schur_build<R>(s, d, a.qp, a.st.rho, a.sigma, a.rho_f_factor, a.ctl, S, Phi);
      if (st) return st;
    }
    a.it_lo = bounds[k];
    a.it_hi = bounds[k + 1];
    a.first_chunk = k == 0 ? 1 : 0;
    switch (d.n) {
      case 6: launch_admm_pcg_nc<R, 6>(s, pa); break;
      case 9: launch_admm_pcg_nc<R, 9>(s, pa); break;
      case 16: launch_admm_pcg_nc<R, 16>(s, pa); break;
      case 17: launch_admm_pcg_nc<R, 17>(s, pa); break;
      default: launch_admm_pcg_nc<R, 0>(s, pa); break;
    }
    st = launch_status();
    if (st) return st;
  }
  if (g_iter_events[1] && hipEventRecord(g_iter_events[1], s) != hipSuccess) return TMPC_ELAUNCH;
  return launch_nonfinite_flags<R>(s, d, a.st, iters);
}

// ------------------------------------------------------------ quadrotor ----
template <typename R>
int quad_impl(hipStream_t s, int B, int N, const R* states, int64_t ls, const R* controls, int64_t lu, double dt,
              const double* params, R* Am, R* c, QuadRecOut<R> rec) {
  if (B < 1 || N < 1) return TMPC_EBADSHAPE;
  if (!states || !controls || !params || !Am || !c) return TMPC_EBADARG;
  if (ls < 13 || lu < 4 || ls > (1 << 20) || lu > (1 << 20)) return TMPC_EBADARG;
  QuadParams<R> P{(R)params[0], (R)params[1], (R)params[2], (R)params[3],
                  (R)params[4], (R)params[5], (R)params[6]};
  const long long total = (long long)B * N * 18;
  const int blk = 256;
  const long long grid = (total + blk - 1) / blk;
  hipLaunchKernelGGL((quad_linearize_kernel<R>), dim3((unsigned)grid), dim3(blk), 0, s, B, N, states, (int)ls,
                     controls, (int)lu, (R)dt, P, Am, c, rec);
  return launch_status();
}

template <typename R>
int quad_step_impl(hipStream_t s, int B, int N, const R* states, const R* controls, double dt, const double* params,
                   R* next) {
  if (B < 1 || N < 1) return TMPC_EBADSHAPE;
  if (!states || !controls || !params || !next) return TMPC_EBADARG;
  QuadParams<R> P{(R)params[0], (R)params[1], (R)params[2], (R)params[3],
                  (R)params[4], (R)params[5], (R)params[6]};
  const long long total = (long long)B * N;
  const long long grid = (total + 255) / 256;
  if (grid > INT32_MAX) return TMPC_EBADSHAPE;
  hipLaunchKernelGGL((quad_step_kernel<R>), dim3((unsigned)grid), dim3(256), 0, s, B, N, states, controls, (R)dt, P,
                     next);
  return launch_status();
}

template <typename R>
int quad_hess_impl(hipStream_t s, int B, int N, const R* states, const R* controls, double dt,
                   const double* params, const R* lambdas, R* H) {
  if (B < 1 || N < 1) return TMPC_EBADSHAPE;
  if (!states || !controls || !params || !lambdas || !H) return TMPC_EBADARG;
  QuadParams<R> P{(R)params[0], (R)params[1], (R)params[2], (R)params[3],
                  (R)params[4], (R)params[5], (R)params[6]};
  const long long total = (long long)B * (N + 1) * (17 * 18 / 2);
  const int blk = 256;
  const long long grid = (total + blk - 1) / blk;
  if (grid > INT32_MAX) return TMPC_EBADSHAPE;
  hipLaunchKernelGGL((quad_lag_hessian_kernel<R>), dim3((unsigned)grid), dim3(blk), 0, s, B, N, states, controls,
                     (R)dt, P, lambdas, H);
  return launch_status();
}


template <typename R>
int linear_step_impl(hipStream_t s, int B, int N, int nx, int nu, const R* states, const R* controls, const R* A,
                     const R* Bm, const R* b, R* next) {
  if (B < 1 || N < 1 || nx < 1 || nu < 0) return TMPC_EBADSHAPE;
  const long long total = (long long)B * N * nx;  // one thread per (problem, stage, row)
  if (total >= INT32_MAX) return TMPC_EBADSHAPE;
  if (!states || !controls || !A || (nu > 0 && !Bm) || !b || !next) return TMPC_EBADARG;
  hipLaunchKernelGGL((linear_step_kernel<R>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, B, N, nx, nu,
                     states, controls, A, Bm, b, next);
  return launch_status();
}

// ------------------------------------------------------------- obstacles ----
inline int obstacle_check(int B, int N, int nx, int nu, int dim, int K, int m, int row0) {
  if (B < 1 || N < 1 || nx < 1 || nu < 0 || nx + nu > 64 || dim < 1 || dim > nx || K < 0 || row0 < 0 ||
      row0 + K > m)
    return TMPC_EBADSHAPE;
  return TMPC_OK;
}

template <typename R>
int obstacle_lin_impl(hipStream_t s, int B, int N, int nx, int nu, int dim, int K, const R* states, int ls,
                      const R* centers, const R* radii, int m, int row0, R* G, R* l, R* u, ObsRecOut<R> rec) {
  int st = obstacle_check(B, N, nx, nu, dim, K, m, row0);
  if (st) return st;
  if (K == 0) return TMPC_OK;
  if (!states || !centers || !radii || !G || !l || !u) return TMPC_EBADARG;
  if (ls < nx) return TMPC_EBADSHAPE;
  const int T = N + 1, n = nx + nu;
  const long long rows = (long long)B * T * K;  // one thread per obstacle row
  if (rows >= INT32_MAX) return TMPC_EBADSHAPE;
  const int blk = kObstacleBlock;
  const long long grid = (rows + blk - 1) / blk;
  const size_t smem = (size_t)blk * (2 * sizeof(size_t) + n * sizeof(R));  // n <= 64: at most 66 KB
  lds_optin(obstacle_linearize_kernel<R>, smem);
  hipLaunchKernelGGL((obstacle_linearize_kernel<R>), dim3((unsigned)grid), dim3(blk), smem, s, B, T, ls, n, dim, K,
                     states, centers, radii, m, row0, G, l, u, rec);
  return launch_status();
}

template <typename R>
int obstacle_hess_impl(hipStream_t s, int B, int N, int nx, int nu, int dim, int K, const R* states,
                       const R* centers, const R* radii, int m, int row0, const R* mus, R* H) {
  int st = obstacle_check(B, N, nx, nu, dim, K, m, row0);
  if (st) return st;
  if (!states || !H || !mus || (K > 0 && (!centers || !radii))) return TMPC_EBADARG;
  const int T = N + 1, n = nx + nu;
  const long long stages = (long long)B * T;  // one thread per stage
  if (stages >= INT32_MAX) return TMPC_EBADSHAPE;
  const int blk = 256;
  const long long grid = (stages + blk - 1) / blk;
  hipLaunchKernelGGL((obstacle_hessian_kernel<R>), dim3((unsigned)grid), dim3(blk), 0, s, B, T, nx, n, dim, K,
                     states, centers, radii, m, row0, mus, H);
  return launch_status();
}

// ------------------------------------------------------------- SQP check ----
template <typename R, int NC>
void launch_sqp_nc(hipStream_t s, const Dims& d, bool std_dyn, int diag, const QPDev<R>& q, const R* x,
                   const R* y0, const R* yf, const R* yg, const R* sl, R sw, R* conv, R* eq, R* iq, R* gout,
                   const R* swp) {
  const int spw = check_stages_per_wave(d.B, d.T);
  const dim3 grid(d.B * ((d.T + spw - 1) / spw));
  const size_t smem = check_smem_bytes<R>(d.n, d.nx, d.m);
  lds_optin(sqp_check_stage_kernel<R, NC, true>, smem);
  lds_optin(sqp_check_stage_kernel<R, NC, false>, smem);
  if (std_dyn)
    hipLaunchKernelGGL((sqp_check_stage_kernel<R, NC, true>), grid, dim3(kWave), smem, s, d, q, x, y0, yf, yg, sl, sw,
                       swp, conv, eq, iq, gout, diag, spw);
  else
    hipLaunchKernelGGL((sqp_check_stage_kernel<R, NC, false>), grid, dim3(kWave), smem, s, d, q, x, y0, yf, yg, sl, sw,
                       swp, conv, eq, iq, gout, diag, spw);
}

template <typename R>
int sqp_check_impl(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const R* x, const R* y0, const R* yf,
                   const R* yg, const R* slack, double slack_w, uint32_t flags, R* conv, R* eq, R* iq, R* gout,
                   const R* slack_wp) {
  if (!dims_ok(dims)) return TMPC_EBADSHAPE;
  if (!qp_ok(qp, dims->m) || !x || !y0 || !yf || !conv || (dims->m > 0 && !yg)) return TMPC_EBADARG;
  const Dims d = to_dims(dims);
  if ((long long)d.B * d.T > INT32_MAX) return TMPC_EBADSHAPE;
  const QPDev<R> q = to_qp<R>(qp);
  hipLaunchKernelGGL((sqp_check_init_kernel<R>), dim3((d.B + 255) / 256), dim3(256), 0, s, d.B, conv, eq, iq);
  const bool std_dyn = flags & TMPC_FLAG_STD_DYNAMICS;
  const int diag = (flags & TMPC_FLAG_DIAG_COST) ? 1 : 0;
  switch (d.n) {
    case 6: launch_sqp_nc<R, 6>(s, d, std_dyn, diag, q, x, y0, yf, yg, slack, (R)slack_w, conv, eq, iq, gout, slack_wp); break;
    case 9: launch_sqp_nc<R, 9>(s, d, std_dyn, diag, q, x, y0, yf, yg, slack, (R)slack_w, conv, eq, iq, gout, slack_wp); break;
    case 16: launch_sqp_nc<R, 16>(s, d, std_dyn, diag, q, x, y0, yf, yg, slack, (R)slack_w, conv, eq, iq, gout, slack_wp); break;
    case 17: launch_sqp_nc<R, 17>(s, d, std_dyn, diag, q, x, y0, yf, yg, slack, (R)slack_w, conv, eq, iq, gout, slack_wp); break;
    default: launch_sqp_nc<R, 0>(s, d, std_dyn, diag, q, x, y0, yf, yg, slack, (R)slack_w, conv, eq, iq, gout, slack_wp); break;
  }
  return launch_status();
}

}  // namespace
}  // namespace tmpc

using namespace tmpc;

// ------------------------------------------------------ merit terms ----
template <typename R>
int merit_impl(hipStream_t s, const tmpc_merit_terms* m) {
  if (!m) return TMPC_EBADARG;
  if (m->P < 0 || m->B0 < 1 || m->P % m->B0 != 0 || m->T < 2 || m->nx < 1 || m->nx > kMeritMaxVars ||
      m->nu < 0 || m->nu > kMeritMaxVars || m->mbox < 0 || m->mbox > kMeritMaxRows)
    return TMPC_EBADSHAPE;
  if (m->P == 0) return TMPC_OK;
  if (m->lin_A && (!m->lin_b || (m->nu > 0 && !m->lin_B))) return TMPC_EBADARG;
  if (!m->states || (m->nu > 0 && !m->controls) || (!m->next && !m->lin_A) || !m->x0 || !m->w || !m->zref ||
      !m->cost || !m->eq ||
      !m->iq || (m->dstates && m->nu > 0 && !m->dcontrols) || (m->dslacks && !m->slacks))
    return TMPC_EBADARG;
  if (m->mbox > 0 && (!m->box_idx || !m->box_lo || !m->box_hi)) return TMPC_EBADARG;
  if (m->nobs < 0 || m->nobs > kMeritMaxObstacles || (m->nobs > 0 && (m->dim < 1 || m->dim > m->nx)))
    return TMPC_EBADSHAPE;
  if (m->nobs > 0 && (!m->centers || !m->radii)) return TMPC_EBADARG;
  if (m->scaled && (!m->state_scale || (m->nu > 0 && !m->control_scale) || (m->mbox > 0 && !m->box_scale)))
    return TMPC_EBADARG;
  MeritArgs<R> a{};
  a.P = m->P; a.B0 = m->B0; a.T = m->T; a.nx = m->nx; a.nu = m->nu; a.mbox = m->mbox;
  a.states = static_cast<const R*>(m->states);
  a.controls = static_cast<const R*>(m->controls);
  a.next = static_cast<const R*>(m->next);
  a.lin_A = static_cast<const R*>(m->lin_A);
  a.lin_B = static_cast<const R*>(m->lin_B);
  a.lin_b = static_cast<const R*>(m->lin_b);
  a.x0 = static_cast<const R*>(m->x0);
  a.u0 = static_cast<const R*>(m->u0);
  a.w = static_cast<const R*>(m->w);
  a.zref = static_cast<const R*>(m->zref);
  a.scaled = m->scaled ? 1 : 0;
  for (int j = 0; j < m->mbox; ++j) {
    if (m->box_idx[j] < 0 || m->box_idx[j] >= m->nx + m->nu) return TMPC_EBADARG;
    a.box_idx[j] = m->box_idx[j];
    a.box_lo[j] = (R)m->box_lo[j];
    a.box_hi[j] = (R)m->box_hi[j];
    a.box_scale[j] = m->scaled ? (R)m->box_scale[j] : R(1);
  }
  if (m->scaled) {
    for (int k = 0; k < m->nx; ++k) a.sscale[k] = (R)m->state_scale[k];
    for (int k = 0; k < m->nu; ++k) a.cscale[k] = (R)m->control_scale[k];
  }
  a.nobs = m->nobs;
  a.dim = m->nobs > 0 ? m->dim : 0;
  a.centers = static_cast<const R*>(m->centers);
  a.radii = static_cast<const R*>(m->radii);
  a.obs_scale = m->scaled && m->nobs > 0 ? (R)m->obs_scale : R(1);
  a.slacks = static_cast<const R*>(m->slacks);
  a.gamma = (R)m->gamma;
  a.dstates = static_cast<const R*>(m->dstates);
  a.dcontrols = static_cast<const R*>(m->dcontrols);
  a.dslacks = static_cast<const R*>(m->dslacks);
  a.cost = static_cast<R*>(m->cost);
  a.dcost = static_cast<R*>(m->dcost);
  a.eq = static_cast<R*>(m->eq);
  a.iq = static_cast<R*>(m->iq);
  constexpr int per_block = 256 / kWave;
  const long long grid = ((long long)m->P + per_block - 1) / per_block;
  if (grid > 0x7fffffffLL) return TMPC_EBADSHAPE;
  hipLaunchKernelGGL((ocp_merit_terms_kernel<R>), dim3((unsigned)grid), dim3(256), 0, s, a);
  return launch_status();
}

template <typename R>
int choose_impl(hipStream_t s, int32_t B, int32_t A, const R* cost, const R* dcost, const R* eq, const R* iq,
                const R* cost_a, const R* eq_a, const R* iq_a, const double* alphas, double eta, double mu_min,
                double mu_max, double floor_, R* alpha_out, R* mu_out) {
  if (B < 0 || A < 1 || A > kMaxAlphas) return TMPC_EBADSHAPE;
  if (B == 0) return TMPC_OK;
  if (!cost || !dcost || !eq || !iq || !cost_a || !eq_a || !iq_a || !alphas || !alpha_out) return TMPC_EBADARG;
  ChooseArgs<R> a{};
  a.B = B;
  a.A = A;
  a.cost = cost; a.dcost = dcost; a.eq = eq; a.iq = iq;
  a.cost_a = cost_a; a.eq_a = eq_a; a.iq_a = iq_a;
  for (int j = 0; j < A; ++j) {
    a.alpha[j] = (R)alphas[j];
    a.eta_alpha[j] = (R)(eta * alphas[j]);  // the double product, then rounded, as a Python scalar
  }
  a.mu_min = (R)mu_min;
  a.mu_max = (R)mu_max;
  a.floor_ = (R)floor_;
  a.alpha_out = alpha_out;
  a.mu_out = mu_out;
  hipLaunchKernelGGL((linesearch_choose_kernel<R>), dim3((unsigned)((B + 255) / 256)), dim3(256), 0, s, a);
  return launch_status();
}

// ----------------------------------------------------------- KKT state ----
template <typename R>
int kkt_active_sets_impl(hipStream_t s, int64_t count, const R* g, const R* l, const R* u, const R* y,
                         double eps_abs, double eps_rel, double dual_tol, uint8_t* lower, uint8_t* upper) {
  if (count < 0) return TMPC_EBADSHAPE;
  if (count == 0) return TMPC_OK;
  if (!g || !l || !u || !lower || !upper) return TMPC_EBADARG;
  const long long grid = (count + 255) / 256;
  if (grid > 0x7fffffffLL) return TMPC_EBADSHAPE;
  // the scalars rounded to R, as torch rounds a Python scalar to the tensor's type
  hipLaunchKernelGGL((kkt_active_sets_kernel<R>), dim3((unsigned)grid), dim3(256), 0, s, (long long)count, g, l, u,
                     y, (R)eps_abs, (R)eps_rel, (R)dual_tol, lower, upper);
  return launch_status();
}

extern "C" {

const char* tmpc_status_string(int status) {
  switch (status) {
    case TMPC_OK: return "ok";
    case TMPC_EBADSHAPE: return "unsupported dimensions";
    case TMPC_EBADARG: return "invalid argument";
    case TMPC_EWORKSPACE: return "workspace too small";
    case TMPC_ELAUNCH: return "HIP launch failed";
    case TMPC_ESCRATCH: return "problem needs more than the allocation-free scratch";
    case TMPC_ENONFINITE: return "non-finite values in the solution";
    default: return "unknown status";
  }
}

int tmpc_version(void) { return 100; }

int tmpc_fill_zero(hipStream_t s, void* p, size_t bytes) {
  if (bytes == 0) return TMPC_OK;
  if (!p || (reinterpret_cast<uintptr_t>(p) & 3u) != 0 || (bytes & 3u) != 0) return TMPC_EBADARG;
  const size_t words = bytes / 4;
  const size_t blocks = (words + 255) / 256;
  if (blocks > 0x7fffffffu) return TMPC_EBADARG;
  hipLaunchKernelGGL((fill_kernel<uint32_t>), dim3((unsigned)blocks), dim3(256), 0, s, static_cast<uint32_t*>(p),
                     words, 0u);
  return launch_status();
}

void tmpc_set_timing_events(hipEvent_t before, hipEvent_t after) {
  g_iter_events[0] = before;
  g_iter_events[1] = after;
}

size_t tmpc_admm_direct_workspace_bytes(int elem_bytes, const tmpc_dims* dims) {
  if (!dims_ok(dims)) return 0;
  const Dims d = to_dims(dims);
  return elem_bytes == 8 ? direct_ws_bytes_full<double>(d) : direct_ws_bytes_full<float>(d);
}

int tmpc_admm_direct_f32(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                         tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg, void* ws,
                         size_t wsb) {
  return admm_direct_impl<float>(s, dims, qp, in, out, iters, cfg, ws, wsb);
}
int tmpc_admm_direct_f64(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                         tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg, void* ws,
                         size_t wsb) {
  return admm_direct_impl<double>(s, dims, qp, in, out, iters, cfg, ws, wsb);
}

int tmpc_admm_direct_noalloc(hipStream_t s, int elem_bytes, const tmpc_dims* dims, const tmpc_qp* qp,
                             const tmpc_state* in, tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg) {
  if (elem_bytes == 4) return admm_direct_noalloc_impl<float>(s, dims, qp, in, out, iters, cfg);
  if (elem_bytes == 8) return admm_direct_noalloc_impl<double>(s, dims, qp, in, out, iters, cfg);
  return TMPC_EBADARG;
}

int tmpc_sqp_admm_step_f32(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                           tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg, const tmpc_sqp_step* sqp,
                           void* ws, size_t wsb) {
  if (!sqp) return TMPC_EBADARG;
  return admm_direct_impl<float>(s, dims, qp, in, out, iters, cfg, ws, wsb, sqp);
}
int tmpc_sqp_admm_step_f64(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                           tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg, const tmpc_sqp_step* sqp,
                           void* ws, size_t wsb) {
  if (!sqp) return TMPC_EBADARG;
  return admm_direct_impl<double>(s, dims, qp, in, out, iters, cfg, ws, wsb, sqp);
}

size_t tmpc_blktri_workspace_bytes(int elem_bytes, int32_t B, int32_t T, int32_t n) {
  tmpc_dims td{B, T, n, 1, 1, 0};
  if (!dims_ok(&td)) return 0;
  return align_up((size_t)T * B * th_pitch(n) * (elem_bytes == 8 ? 8 : 4));
}
int tmpc_blktri_factor_f32(hipStream_t s, int32_t B, int32_t T, int32_t n, const float* S, void* ws,
                           size_t wsb) {
  return blktri_factor_impl<float>(s, B, T, n, S, ws, wsb);
}
int tmpc_blktri_factor_f64(hipStream_t s, int32_t B, int32_t T, int32_t n, const double* S, void* ws,
                           size_t wsb) {
  return blktri_factor_impl<double>(s, B, T, n, S, ws, wsb);
}
int tmpc_blktri_solve_f32(hipStream_t s, int32_t B, int32_t T, int32_t n, const float* S,
                          const float* rhs, float* x, const void* ws, size_t wsb) {
  return blktri_solve_impl<float>(s, B, T, n, S, rhs, x, ws, wsb);
}
int tmpc_blktri_solve_f64(hipStream_t s, int32_t B, int32_t T, int32_t n, const double* S,
                          const double* rhs, double* x, const void* ws, size_t wsb) {
  return blktri_solve_impl<double>(s, B, T, n, S, rhs, x, ws, wsb);
}

size_t tmpc_adjoint_kkt_workspace_bytes(int elem_bytes, const tmpc_dims* dims) {
  if (!dims_ok(dims)) return 0;
  const Dims d = to_dims(dims);
  return elem_bytes == 8 ? adjoint_ws_bytes<double>(d) : adjoint_ws_bytes<float>(d);
}
int tmpc_adjoint_kkt_f32(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, float* dz,
                         float* mult, double reg, int32_t refine_steps, uint32_t flags, void* ws,
                         size_t wsb) {
  return adjoint_impl<float>(s, dims, qp, dz, mult, reg, refine_steps, flags, ws, wsb);
}
int tmpc_adjoint_kkt_f64(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, double* dz,
                         double* mult, double reg, int32_t refine_steps, uint32_t flags, void* ws,
                         size_t wsb) {
  return adjoint_impl<double>(s, dims, qp, dz, mult, reg, refine_steps, flags, ws, wsb);
}

size_t tmpc_admm_pcg_workspace_bytes(int elem_bytes, const tmpc_dims* dims) {
  if (!dims_ok(dims)) return 0;
  const Dims d = to_dims(dims);
  return elem_bytes == 8 ? admm_pcg_ws_bytes<double>(d) : admm_pcg_ws_bytes<float>(d);
}
int tmpc_admm_pcg_f32(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                      tmpc_state* out, uint32_t* iters, uint32_t* pcg_iters, const tmpc_admm_cfg* cfg,
                      void* ws, size_t wsb) {
  return admm_pcg_impl<float>(s, dims, qp, in, out, iters, pcg_iters, cfg, ws, wsb);
}
int tmpc_admm_pcg_f64(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                      tmpc_state* out, uint32_t* iters, uint32_t* pcg_iters, const tmpc_admm_cfg* cfg,
                      void* ws, size_t wsb) {
  return admm_pcg_impl<double>(s, dims, qp, in, out, iters, pcg_iters, cfg, ws, wsb);
}

int tmpc_schur_build_f32(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const float* rho,
                         double sigma, double rho_f_factor, float* S, float* Phiinv) {
  return schur_build_impl<float>(s, dims, qp, rho, sigma, rho_f_factor, S, Phiinv);
}
int tmpc_schur_build_f64(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const double* rho,
                         double sigma, double rho_f_factor, double* S, double* Phiinv) {
  return schur_build_impl<double>(s, dims, qp, rho, sigma, rho_f_factor, S, Phiinv);
}

size_t tmpc_schur_pcg_workspace_bytes(int elem_bytes, int32_t B, int32_t T, int32_t n) {
  tmpc_dims td{B, T, n, 1, 1, 0};
  if (!dims_ok(&td)) return 0;
  const Dims d = to_dims(&td);
  return elem_bytes == 8 ? pcg_vec_bytes<double>(d) : pcg_vec_bytes<float>(d);
}
int tmpc_schur_pcg_f32(hipStream_t s, int32_t B, int32_t T, int32_t n, const float* S, const float* Phiinv,
                       const float* rhs, const float* x0, float* x, uint32_t* iters, double eps,
                       int32_t max_iter, void* ws, size_t wsb) {
  return schur_pcg_impl<float>(s, B, T, n, S, Phiinv, rhs, x0, x, iters, eps, max_iter, ws, wsb);
}
int tmpc_schur_pcg_f64(hipStream_t s, int32_t B, int32_t T, int32_t n, const double* S,
                       const double* Phiinv, const double* rhs, const double* x0, double* x,
                       uint32_t* iters, double eps, int32_t max_iter, void* ws, size_t wsb) {
  return schur_pcg_impl<double>(s, B, T, n, S, Phiinv, rhs, x0, x, iters, eps, max_iter, ws, wsb);
}

int tmpc_quadrotor_linearize_f32(hipStream_t s, int32_t B, int32_t N, const float* states,
                                 const float* controls, double dt, const double* params, float* A_minus,
                                 float* c) {
  return quad_impl<float>(s, B, N, states, 13, controls, 4, dt, params, A_minus, c, QuadRecOut<float>{});
}
int tmpc_quadrotor_linearize_f64(hipStream_t s, int32_t B, int32_t N, const double* states,
                                 const double* controls, double dt, const double* params, double* A_minus,
                                 double* c) {
  return quad_impl<double>(s, B, N, states, 13, controls, 4, dt, params, A_minus, c, QuadRecOut<double>{});
}
int tmpc_quadrotor_linearize_strided_f32(hipStream_t s, int32_t B, int32_t N, const float* states,
                                         int64_t states_row_stride, const float* controls,
                                         int64_t controls_row_stride, double dt, const double* params,
                                         float* A_minus, float* c) {
  return quad_impl<float>(s, B, N, states, states_row_stride, controls, controls_row_stride, dt, params, A_minus, c,
                          QuadRecOut<float>{});
}
int tmpc_quadrotor_linearize_strided_f64(hipStream_t s, int32_t B, int32_t N, const double* states,
                                         int64_t states_row_stride, const double* controls,
                                         int64_t controls_row_stride, double dt, const double* params,
                                         double* A_minus, double* c) {
  return quad_impl<double>(s, B, N, states, states_row_stride, controls, controls_row_stride, dt, params, A_minus,
                           c, QuadRecOut<double>{});
}

int tmpc_linear_dynamics_f32(hipStream_t s, int32_t B, int32_t N, int32_t nx, int32_t nu, const float* states,
                             const float* controls, const float* A, const float* Bm, const float* b, float* next) {
  return linear_step_impl<float>(s, B, N, nx, nu, states, controls, A, Bm, b, next);
}
int tmpc_linear_dynamics_f64(hipStream_t s, int32_t B, int32_t N, int32_t nx, int32_t nu, const double* states,
                             const double* controls, const double* A, const double* Bm, const double* b,
                             double* next) {
  return linear_step_impl<double>(s, B, N, nx, nu, states, controls, A, Bm, b, next);
}
int tmpc_quadrotor_dynamics_f32(hipStream_t s, int32_t B, int32_t N, const float* states, const float* controls,
                                double dt, const double* params, float* next) {
  return quad_step_impl<float>(s, B, N, states, controls, dt, params, next);
}
int tmpc_quadrotor_dynamics_f64(hipStream_t s, int32_t B, int32_t N, const double* states, const double* controls,
                                double dt, const double* params, double* next) {
  return quad_step_impl<double>(s, B, N, states, controls, dt, params, next);
}

int tmpc_quadrotor_lagrangian_hessian_f32(hipStream_t s, int32_t B, int32_t N, const float* states,
                                          const float* controls, double dt, const double* params,
                                          const float* lambdas, float* H) {
  return quad_hess_impl<float>(s, B, N, states, controls, dt, params, lambdas, H);
}
int tmpc_quadrotor_lagrangian_hessian_f64(hipStream_t s, int32_t B, int32_t N, const double* states,
                                          const double* controls, double dt, const double* params,
                                          const double* lambdas, double* H) {
  return quad_hess_impl<double>(s, B, N, states, controls, dt, params, lambdas, H);
}

int tmpc_obstacle_linearize_f32(hipStream_t s, int32_t B, int32_t N, int32_t nx, int32_t nu, int32_t dim,
                                int32_t K, const float* states, const float* centers, const float* radii, int32_t m,
                                int32_t row0, float* G, float* l, float* u) {
  return obstacle_lin_impl<float>(s, B, N, nx, nu, dim, K, states, nx, centers, radii, m, row0, G, l, u,
                                 ObsRecOut<float>{});
}
int tmpc_obstacle_linearize_f64(hipStream_t s, int32_t B, int32_t N, int32_t nx, int32_t nu, int32_t dim,
                                int32_t K, const double* states, const double* centers, const double* radii,
                                int32_t m, int32_t row0, double* G, double* l, double* u) {
  return obstacle_lin_impl<double>(s, B, N, nx, nu, dim, K, states, nx, centers, radii, m, row0, G, l, u,
                                 ObsRecOut<double>{});
}
int tmpc_obstacle_lagrangian_hessian_f32(hipStream_t s, int32_t B, int32_t N, int32_t nx, int32_t nu, int32_t dim,
                                         int32_t K, const float* states, const float* centers, const float* radii,
                                         int32_t m, int32_t row0, const float* mus, float* H) {
  return obstacle_hess_impl<float>(s, B, N, nx, nu, dim, K, states, centers, radii, m, row0, mus, H);
}
int tmpc_obstacle_lagrangian_hessian_f64(hipStream_t s, int32_t B, int32_t N, int32_t nx, int32_t nu, int32_t dim,
                                         int32_t K, const double* states, const double* centers,
                                         const double* radii, int32_t m, int32_t row0, const double* mus,
                                         double* H) {
  return obstacle_hess_impl<double>(s, B, N, nx, nu, dim, K, states, centers, radii, m, row0, mus, H);
}

int tmpc_ocp_merit_terms_f32(hipStream_t s, const tmpc_merit_terms* args) { return merit_impl<float>(s, args); }
int tmpc_ocp_merit_terms_f64(hipStream_t s, const tmpc_merit_terms* args) { return merit_impl<double>(s, args); }

int tmpc_linesearch_choose_f32(hipStream_t s, int32_t B, int32_t A, const float* cost, const float* dcost,
                               const float* eq, const float* iq, const float* cost_a, const float* eq_a,
                               const float* iq_a, const double* alphas, double eta, double mu_min, double mu_max,
                               double floor_, float* alpha_out, float* mu_out) {
  return choose_impl<float>(s, B, A, cost, dcost, eq, iq, cost_a, eq_a, iq_a, alphas, eta, mu_min, mu_max, floor_,
                            alpha_out, mu_out);
}
int tmpc_linesearch_choose_f64(hipStream_t s, int32_t B, int32_t A, const double* cost, const double* dcost,
                               const double* eq, const double* iq, const double* cost_a, const double* eq_a,
                               const double* iq_a, const double* alphas, double eta, double mu_min, double mu_max,
                               double floor_, double* alpha_out, double* mu_out) {
  return choose_impl<double>(s, B, A, cost, dcost, eq, iq, cost_a, eq_a, iq_a, alphas, eta, mu_min, mu_max, floor_,
                             alpha_out, mu_out);
}

int tmpc_sqp_admm_step_quadrotor_f32(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                                     tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg,
                                     const tmpc_sqp_step* sqp, double dt, const double* params, void* ws,
                                     size_t wsb) {
  if (!qp || !qp->A_minus || !qp->c || !params || !sqp) return TMPC_EBADARG;
  const QuadLin ql{dt, params};
  return admm_direct_impl<float>(s, dims, qp, in, out, iters, cfg, ws, wsb, sqp, &ql);
}
int tmpc_sqp_admm_step_quadrotor_f64(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                                     tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg,
                                     const tmpc_sqp_step* sqp, double dt, const double* params, void* ws,
                                     size_t wsb) {
  if (!qp || !qp->A_minus || !qp->c || !params || !sqp) return TMPC_EBADARG;
  const QuadLin ql{dt, params};
  return admm_direct_impl<double>(s, dims, qp, in, out, iters, cfg, ws, wsb, sqp, &ql);
}

int tmpc_sqp_admm_step_obstacle_f32(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                                    tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg,
                                    const tmpc_sqp_step* sqp, int32_t dim, int32_t K, const float* centers,
                                    const float* radii, int32_t row0, void* ws, size_t wsb) {
  if (!qp || !qp->G || !qp->l || !qp->u || !sqp || (K > 0 && (!centers || !radii))) return TMPC_EBADARG;
  const ObsLin ol{dim, K, row0, centers, radii};
  return admm_direct_impl<float>(s, dims, qp, in, out, iters, cfg, ws, wsb, sqp, nullptr, &ol);
}
int tmpc_sqp_admm_step_obstacle_f64(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const tmpc_state* in,
                                    tmpc_state* out, uint32_t* iters, const tmpc_admm_cfg* cfg,
                                    const tmpc_sqp_step* sqp, int32_t dim, int32_t K, const double* centers,
                                    const double* radii, int32_t row0, void* ws, size_t wsb) {
  if (!qp || !qp->G || !qp->l || !qp->u || !sqp || (K > 0 && (!centers || !radii))) return TMPC_EBADARG;
  const ObsLin ol{dim, K, row0, centers, radii};
  return admm_direct_impl<double>(s, dims, qp, in, out, iters, cfg, ws, wsb, sqp, nullptr, &ol);
}

int tmpc_kkt_active_sets_f32(hipStream_t s, int64_t count, const float* g, const float* l, const float* u,
                             const float* y, double eps_abs, double eps_rel, double dual_tol, uint8_t* lower,
                             uint8_t* upper) {
  return kkt_active_sets_impl<float>(s, count, g, l, u, y, eps_abs, eps_rel, dual_tol, lower, upper);
}
int tmpc_kkt_active_sets_f64(hipStream_t s, int64_t count, const double* g, const double* l, const double* u,
                             const double* y, double eps_abs, double eps_rel, double dual_tol, uint8_t* lower,
                             uint8_t* upper) {
  return kkt_active_sets_impl<double>(s, count, g, l, u, y, eps_abs, eps_rel, dual_tol, lower, upper);
}

int tmpc_sqp_first_order_f32(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const float* x,
                             const float* y_f0, const float* y_f, const float* y_g, const float* slack,
                             double slack_weight, uint32_t flags, float* conv, float* eq_err, float* ineq_err,
                             float* g_out) {
  return sqp_check_impl<float>(s, dims, qp, x, y_f0, y_f, y_g, slack, slack_weight, flags, conv, eq_err, ineq_err, g_out);
}
int tmpc_sqp_first_order_f64(hipStream_t s, const tmpc_dims* dims, const tmpc_qp* qp, const double* x,
                             const double* y_f0, const double* y_f, const double* y_g, const double* slack,
                             double slack_weight, uint32_t flags, double* conv, double* eq_err, double* ineq_err,
                             double* g_out) {
  return sqp_check_impl<double>(s, dims, qp, x, y_f0, y_f, y_g, slack, slack_weight, flags, conv, eq_err, ineq_err, g_out);
}

}  // extern "C"
