// SQP first-order convergence check on the device.
//
// _compute_first_order_convergence_error (turbompc/solvers/turbompc_solver.py:1158-1225)
// evaluated at x = (states, controls) against the relinearized QP:
//   stationarity  = || P x + q + C^T y_f + G^T y_g ||_inf
//   eq_err        = || C x - c ||_inf
//   ineq_err      = || max(l - g, 0), max(g - u, 0) ||_inf,  g = G x (+ slack)
//   conv          = max(stationarity, eq_err, ineq_err, slack stationarity)
// and g itself (the inequality values the KKT-state active sets are built
// from, :1387-1439).
//
// Every (problem, stage) pair is independent here, so one 64-lane block per
// pair evaluates its stage's rows (lane i = row i, read straight from the QP
// blocks) and folds its maxima into the per-problem outputs with atomicMax
// on the IEEE bit pattern (non-negative values order like unsigned integers).
// sqp_check_init_kernel zeroes the outputs first.
#pragma once
#include "common.hpp"

namespace tmpc {

template <typename R>
struct Bits;
template <>
struct Bits<float> {
  using U = unsigned int;
  __device__ static U of(float v) { return __float_as_uint(v) & 0x7fffffffu; }
};
template <>
struct Bits<double> {
  using U = unsigned long long;
  __device__ static U of(double v) { return (U)__double_as_longlong(v) & 0x7fffffffffffffffull; }
};

template <typename R>
__global__ void sqp_check_init_kernel(int B, R* __restrict__ conv, R* __restrict__ eq, R* __restrict__ iq) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  conv[b] = R(0);
  if (eq) eq[b] = R(0);
  if (iq) iq[b] = R(0);
}

// Broadcast lane `k` of v to the whole wave (v_readlane: the value lands in a
// scalar register, so the dot products below read no LDS for vector operands).
__device__ __forceinline__ float lane_bcast(float v, int k) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}
__device__ __forceinline__ double lane_bcast(double v, int k) {
  const long long u = __builtin_bit_cast(long long, v);
  const int lo = __builtin_amdgcn_readlane((int)u, k), hi = __builtin_amdgcn_readlane((int)(u >> 32), k);
  return __builtin_bit_cast(double, ((long long)hi << 32) | (unsigned)lo);
}

// Row stride of a staged block in LDS: odd, so lane i reading row i hits
// distinct banks.
__host__ __device__ constexpr int check_ld(int n) { return n | 1; }

// A stage block of len (<= K * 64) contiguous elements, loaded into
// registers (K elements per lane) so every load of a stage is in flight
// before the first LDS store; put() writes it as rows of stride ld (n
// columns).  K = 0 (n known only at run time) copies in a plain loop.
template <typename R, int K>
struct StageBlock {
  R r[K > 0 ? K : 1];
  const R* src = nullptr;
  int len = 0;
  __device__ __forceinline__ void get(const R* __restrict__ s, int l) {
    src = s;
    len = l;
    if constexpr (K > 0) {
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const int e = threadIdx.x + j * kWave;
        r[j] = e < l ? s[e] : R(0);
      }
    }
  }
  __device__ __forceinline__ void put(R* __restrict__ dst, int n, int ld) const {
    if constexpr (K > 0) {
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const int e = threadIdx.x + j * kWave;
        if (e < len) dst[(e / n) * ld + e % n] = r[j];
      }
    } else {
      for (int e = threadIdx.x; e < len; e += kWave) dst[(e / n) * ld + e % n] = src[e];
    }
  }
};

// sum_k A[i*ld + k] * bcast(v, k), k < n (A in LDS).
template <typename R, int NC>
__device__ __forceinline__ R row_bdot(const R* A, int i, int ld, int n, R v) {
  if constexpr (NC > 0) {
    R a[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) a[k] = A[i * ld + k];
    __builtin_amdgcn_sched_barrier(0);
    R acc = R(0);
#pragma unroll
    for (int k = 0; k < NC; ++k) acc += a[k] * lane_bcast(v, k);
    return acc;
  } else {
    R acc = R(0);
    for (int k = 0; k < n; ++k) acc += A[i * ld + k] * lane_bcast(v, k);
    return acc;
  }
}

// sum_r A[r*ld + i] * bcast(v, r), r < rows (LDS reads batched four at a time).
template <typename R>
__device__ __forceinline__ R col_bdot(const R* A, int i, int ld, int rows, R v) {
  R acc = R(0);
  int r = 0;
  for (; r + 4 <= rows; r += 4) {
    R a[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = A[(r + j) * ld + i];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += a[j] * lane_bcast(v, r + j);
  }
  for (; r < rows; ++r) acc += A[r * ld + i] * lane_bcast(v, r);
  return acc;
}

// One wave per spw consecutive stages of a problem, one stage after the other
// (check_stages_per_wave: more stages per wave where the batch leaves plenty
// of waves, one where it does not).  D_t, A_minus_t and G_t are staged through LDS; the vectors stay
// in registers (lane k holds element k) and reach the other lanes by
// broadcast.  STD: A_plus_t = [-I 0] and E_t = 0 (neither is read); otherwise
// E and A_plus are read from global memory directly.  The slack weight is
// slack_wp[b] when slack_wp is given, else slack_w.  Each stage's maxima are
// folded over the wave as before; the wave keeps the largest of its stages'
// (as bit patterns of the magnitudes, which is what the per-problem atomicMax
// compares) and issues one atomic per output.
constexpr int kCheckMaxStages = 16;
inline int check_stages_per_wave(long long B, int T) {
  const long long s = B * T / 16384;  // about 16 waves per SIMD at one stage per wave
  return s < 1 ? 1 : (s > kCheckMaxStages ? kCheckMaxStages : (int)s);
}

template <typename R, int NC, bool STD>
__global__ __launch_bounds__(kWave) void sqp_check_stage_kernel(Dims d, QPDev<R> qp, const R* __restrict__ x,
                                                              const R* __restrict__ y0, const R* __restrict__ yf,
                                                              const R* __restrict__ yg, const R* __restrict__ slack,
                                                              R slack_w, const R* __restrict__ slack_wp,
                                                              R* __restrict__ conv, R* __restrict__ eq_err,
                                                              R* __restrict__ ineq_err, R* __restrict__ gout,
                                                              int diag, int spw) {
  extern __shared__ __align__(16) unsigned char check_smem[];
  R* sD = reinterpret_cast<R*>(check_smem);
  using U = typename Bits<R>::U;
  const int T = d.T, nsb = (T + spw - 1) / spw, i = threadIdx.x;
  const int b = blockIdx.x / nsb, t_lo = (blockIdx.x - b * nsb) * spw;
  const int t_hi = t_lo + spw < T ? t_lo + spw : T;
  const int N = d.N, n = NC > 0 ? NC : d.n, nx = d.nx, n0 = d.n0, m = d.m;
  U all_b = 0, eq_b = 0, iq_b = 0;
  for (int t = t_lo; t < t_hi; ++t) {
    if (t > t_lo) wsync();  // the previous stage's reads of the LDS blocks are done
    const int ld = check_ld(n);
    R* sAm = sD + n * ld;
    R* sG = sAm + nx * ld;
    const size_t bt = (size_t)b * T + t, bn = (size_t)b * N;
    const bool has_next = t < N, has_prev = t > 0;
    constexpr int KB = NC > 0 ? (NC * NC + kWave - 1) / kWave : 0;
    constexpr int KG = NC > 0 ? NC : 0;  // m <= 64 rows of NC

    // Every load of the stage is issued before the first use.
    const R xt = i < n ? x[bt * n + i] : R(0);
    const R xn = has_next && i < n ? x[(bt + 1) * n + i] : R(0);
    const R xp = !STD && has_prev && i < n ? x[(bt - 1) * n + i] : R(0);
    const R yc = has_next && i < nx ? yf[(bn + t) * nx + i] : R(0);
    const R yp = has_prev && i < nx ? yf[(bn + t - 1) * nx + i] : R(0);
    const R y0v = t == 0 && i < n0 ? y0[(size_t)b * n0 + i] : R(0);
    const R ygv = i < m ? yg[bt * m + i] : R(0);
    const R qv = i < n ? qp.q[bt * n + i] : R(0);
    const R cv = has_next && i < nx ? qp.c[(bn + t) * nx + i] : R(0);
    const R c0v = t == 0 && i < n0 ? qp.c0[(size_t)b * n0 + i] : R(0);
    const R lv = i < m ? qp.l[bt * m + i] : R(0);
    const R uv = i < m ? qp.u[bt * m + i] : R(0);
    const R slv = slack && i < m ? slack[bt * m + i] : R(0);
    const R dii = diag && i < n ? qp.D[bt * n * n + (size_t)i * (n + 1)] : R(0);  // diagonal D_t
    StageBlock<R, KB> bD, bA;
    StageBlock<R, KG> bG;
    bD.get(qp.D + bt * n * n, diag ? 0 : n * n);
    bA.get(qp.Am + (bn + (has_next ? t : 0)) * nx * n, has_next ? nx * n : 0);
    bG.get(qp.G + bt * m * n, m * n);
    __builtin_amdgcn_sched_barrier(0);
    bD.put(sD, n, ld);
    bA.put(sAm, n, ld);
    bG.put(sG, n, ld);
    wsync();

    // Branches below depend on the stage only (uniform); rows past the block's
    // height are computed on row 0 and dropped, so every lane reaches every
    // broadcast.
    const int in = i < n ? i : 0, ix = i < nx ? i : 0, im = i < m ? i : 0, i0 = i < n0 ? i : 0;
    R px = diag ? dii * xt : row_bdot<R, NC>(sD, in, ld, n, xt);
    R aty = m ? col_bdot(sG, in, ld, m, ygv) : R(0);
    if (has_next) aty += col_bdot(sAm, in, ld, nx, yc);
    if (STD) {
      if (has_prev && i < nx) aty -= yp;
    } else {
      if (has_prev) {
        const R* Ep = qp.E + (bn + t - 1) * n * n + (size_t)in * n;
        const R* Ap = qp.Ap + (bn + t - 1) * nx * n;
        for (int k = 0; k < n; ++k) px += Ep[k] * lane_bcast(xp, k);
        for (int r = 0; r < nx; ++r) aty += Ap[(size_t)r * n + in] * lane_bcast(yp, r);
      }
      if (has_next) {
        const R* En = qp.E + (bn + t) * n * n;
        for (int k = 0; k < n; ++k) px += En[(size_t)k * n + in] * lane_bcast(xn, k);
      }
    }
    if (t == 0) {
      const R* A0 = qp.A0 + (size_t)b * n0 * n;
      for (int r = 0; r < n0; ++r) aty += A0[(size_t)r * n + in] * lane_bcast(y0v, r);
    }
    R st = i < n ? rabs(px + qv + aty) : R(0);
    R eq = 0, iq = 0, sl = 0;
    if (has_next) {
      R cx = row_bdot<R, NC>(sAm, ix, ld, n, xt);
      if (STD) {
        cx -= xn;
      } else {
        const R* Ap = qp.Ap + (bn + t) * nx * n + (size_t)ix * n;
        for (int k = 0; k < n; ++k) cx += Ap[k] * lane_bcast(xn, k);
      }
      if (i < nx) eq = rabs(cx - cv);
    }
    if (t == 0) {
      const R* A0 = qp.A0 + ((size_t)b * n0 + i0) * n;
      R cx = 0;
      for (int k = 0; k < n; ++k) cx += A0[k] * lane_bcast(xt, k);
      if (i < n0) eq = rmax(eq, rabs(cx - c0v));
    }
    if (m) {
      const R gv = row_bdot<R, NC>(sG, im, ld, n, xt) + slv;
      if (i < m) {
        if (slack) sl = rabs((slack_wp ? slack_wp[b] : slack_w) * slv + ygv);
        iq = rmax(rmax(lv - gv, R(0)), rmax(gv - uv, R(0)));
        if (gout) gout[bt * m + i] = gv;
      }
    }
    const R all = wave_max(rmax(rmax(st, eq), rmax(iq, sl)));
    if (eq_err) eq = wave_max(eq);
    if (ineq_err) iq = wave_max(iq);
    all_b = all_b > Bits<R>::of(all) ? all_b : Bits<R>::of(all);
    eq_b = eq_b > Bits<R>::of(eq) ? eq_b : Bits<R>::of(eq);
    iq_b = iq_b > Bits<R>::of(iq) ? iq_b : Bits<R>::of(iq);
  }
  if (i == 0) {
    atomicMax(reinterpret_cast<U*>(conv + b), all_b);
    if (eq_err) atomicMax(reinterpret_cast<U*>(eq_err + b), eq_b);
    if (ineq_err) atomicMax(reinterpret_cast<U*>(ineq_err + b), iq_b);
  }
}

// The SQP activity test of one step: act_out = act_in && conv > tol (a NaN
// error stops the problem, as the reference's `conv > tol` does); with conv
// NULL the activity is given: act_out = act_in.
template <typename R>
__global__ void sqp_activity_kernel(int B, const R* __restrict__ conv, R tol, const uint8_t* __restrict__ act_in,
                                    uint8_t* __restrict__ act_out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  act_out[b] = ((act_in ? act_in[b] != 0 : true) && (conv == nullptr || conv[b] > tol)) ? 1 : 0;
}

// The active sets of the KKT state (one thread per inequality row): proximity
// to a bound, min(g - l, u - g) <= eps_abs + eps_rel |bound| on the nearer
// side (identify_active_inequalities, turbompc/solvers/turbompc_solver.py:269-292),
// then, with y, the dual's sign where it is decided (|y| > dual_tol,
// :1387-1439).  The arithmetic is that of the elementwise torch form, value
// for value: the differences, then eps_rel |bound| and eps_abs + that as two
// rounded operations, the scalars rounded to R first; a NaN difference or
// bound makes the row inactive, as torch.minimum's NaN does.  The product and
// the sum must not contract into an FMA (hipcc contracts by default, and the
// intrinsics __fmul_rn / __fadd_rn do not stop it): a row one ulp from its
// tolerance would flip.
template <typename R>
__device__ __forceinline__ R active_tolerance(R eps_abs, R eps_rel, R bound_abs) {
#pragma clang fp contract(off)
  return eps_abs + eps_rel * bound_abs;
}

template <typename R>
__global__ __launch_bounds__(256) void kkt_active_sets_kernel(long long count, const R* __restrict__ g,
                                                              const R* __restrict__ l, const R* __restrict__ u,
                                                              const R* __restrict__ y, R eps_abs, R eps_rel,
                                                              R dual_tol, uint8_t* __restrict__ lower,
                                                              uint8_t* __restrict__ upper) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const R gv = g[i], lv = l[i], uv = u[i];
  const R dl = gv - lv, du = uv - gv;
  const bool use_upper = du < dl;
  const R tol = active_tolerance(eps_abs, eps_rel, use_upper ? rabs(uv) : rabs(lv));
  const bool nan = dl != dl || du != du;
  const bool active = !nan && (dl < du ? dl : du) <= tol;
  bool lo = active && !use_upper, up = active && use_upper;
  if (y != nullptr) {
    const R yv = y[i];
    const bool ylo = yv < -dual_tol, yup = yv > dual_tol, und = !(ylo || yup);
    lo = ylo || (und && lo);
    up = yup || (und && up);
  }
  lower[i] = lo ? 1 : 0;
  upper[i] = up ? 1 : 0;
}

template <typename R>
constexpr size_t check_smem_bytes(int n, int nx, int m) {
  return (size_t)(n + nx + m) * check_ld(n) * sizeof(R);
}

}  // namespace tmpc
