// Terms of the l1 merit function of the SQP line search, one wavefront per
// problem (turbompc/solvers/linesearch.py:14-178 over the tracking OCP's
// cost, equality_constraints and step_inequality_constraints,
// turbompc/problems/optimal_control_problem.py:413-471, :841-912, :982-1066,
// :1504-1515).
//
// For problem p of P (the line search passes its step candidates as
// k copies of the batch, copy j at p = j B0 + b, so every per-problem input
// of the batch is read at b = p % B0):
//   cost  = sum_t,k w (z - zref)^2                       (+ gamma/2 |s|^2)
//   dcost = sum_t,k 2 w (z - zref) dz                     (+ gamma s . ds)
//   eq    = |x_0 - x0|_1 + sum_t |f(x_t, u_t) - x_{t+1}|_1 (+ |u_0 - u0|_1),
//           each row divided by its variable's scale with rescaling
//   iq    = sum_t,j max(lo_j - g, 0) + max(g - hi_j, 0) over the box rows,
//           g = r_j z[idx_j] (+ s), lo and hi scaled by the same r_j, then
//           over the obstacle rows (when given, OptimalControlProblemObstacle,
//           turbompc/problems/obstacle_avoidance.py:16-52)
//           g = ro (1 - |p_t - c_k| / (r_k + 0.001)) (+ s), bounds ro (-1e9, 0),
//           p_t the first `dim` state coordinates
// with f(x_t, u_t) given (the model's step, evaluated by its own kernel).
// Every term is formed as the elementwise torch form forms it (the product
// (w e) e, the scaled bounds); only the order of the sums differs.
#pragma once
#include "common.hpp"

namespace tmpc {

constexpr int kMeritMaxRows = 32;  // box rows
constexpr int kMeritMaxObstacles = 32;
constexpr int kMeritMaxVars = 64;  // nx and nu (the row scales)

// The per-row constants travel by value in the kernel arguments, so that the
// host validates the box rows' variable indices before the launch.
template <typename R>
struct MeritArgs {
  int P, B0, T, nx, nu, mbox;
  const R* states;    // (P, T, nx)
  const R* controls;  // (P, T, nu)
  const R* next;      // (P, T - 1, nx)
  const R* x0;        // (B0, nx)
  const R* u0;        // (B0, nu) or null: no initial-control rows
  const R* w;         // (B0, T, nx + nu)
  const R* zref;      // (B0, T, nx + nu)
  int scaled;         // equality rows divided by sscale (u0 rows by cscale), box rows scaled
  R sscale[kMeritMaxVars], cscale[kMeritMaxVars];
  int box_idx[kMeritMaxRows];  // variable of each box row, < nx + nu
  R box_lo[kMeritMaxRows], box_hi[kMeritMaxRows], box_scale[kMeritMaxRows];
  int nobs, dim;      // obstacle rows after the box rows (0: none), position coordinates
  const R* centers;   // (B0, nobs, dim)
  const R* radii;     // (B0, nobs)
  R obs_scale;        // ro (1 without rescaling)
  const R* lin_A;     // (B0, nx, nx) or null: f_t = A x_t + Bm u_t + b formed here, next unused
  const R* lin_B;     // (B0, nx, nu)
  const R* lin_b;     // (B0, nx)
  const R* slacks;    // (P, T, mbox + nobs) or null
  R gamma;            // slack penalization weight
  const R* dstates;   // (P, T, nx) or null: no directional derivative
  const R* dcontrols; // (P, T, nu)
  const R* dslacks;   // (P, T, mbox) or null
  R* cost;
  R* dcost;           // may be null
  R* eq;
  R* iq;
};

// clamp(x, min=0) as torch evaluates it: a NaN stays NaN (a candidate with a
// NaN row must not look feasible)
template <typename R>
__device__ __forceinline__ R clamp0(R x) {
  return x < R(0) ? R(0) : x;
}

template <typename R>
__global__ __launch_bounds__(256) void ocp_merit_terms_kernel(MeritArgs<R> a) {
  const int p = (int)(blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave);
  const int lane = (int)(threadIdx.x % kWave);
  if (p >= a.P) return;  // whole wavefronts: the sums below need every lane of one
  const int b = p % a.B0, T = a.T, nx = a.nx, nu = a.nu, n = nx + nu, N = T - 1;
  const R* xs = a.states + (size_t)p * T * nx;
  const R* us = a.controls + (size_t)p * T * nu;
  const R* wb = a.w + (size_t)b * T * n;
  const R* rb = a.zref + (size_t)b * T * n;
  R c = R(0), dc = R(0), e = R(0), q = R(0);
  // cost and its directional derivative over the T n entries
  for (int i = lane; i < T * n; i += kWave) {
    const int t = i / n, k = i - t * n;
    const R z = k < nx ? xs[t * nx + k] : us[t * nu + (k - nx)];
    const R d = z - rb[i];
    const R wd = wb[i] * d;
    c += wd * d;
    if (a.dstates != nullptr) {
      const R dz = k < nx ? a.dstates[(size_t)p * T * nx + t * nx + k]
                          : a.dcontrols[(size_t)p * T * nu + t * nu + (k - nx)];
      dc += (R(2) * wb[i]) * d * dz;
    }
  }
  // equality rows: x_0 - x0, then f(x_t, u_t) - x_{t+1}; f_t is the model's
  // step from next, or for linear dynamics formed here as the linear step
  // kernel forms it: (sum_j A_kj x_j + sum_j Bm_kj u_j) + b_k, each sum in j order
  const R* nb = a.next + (size_t)p * N * nx;
  for (int i = lane; i < T * nx; i += kWave) {
    const int t = i / nx, k = i - t * nx;
    R f = R(0);
    if (t > 0) {
      if (a.lin_A != nullptr) {
        const R* ar = a.lin_A + ((size_t)b * nx + k) * nx;
        const R* br = a.lin_B + ((size_t)b * nx + k) * nu;
        const R* xp = xs + (t - 1) * nx;
        const R* up = us + (t - 1) * nu;
        R ax = R(0), bu = R(0);
        for (int j = 0; j < nx; ++j) ax += ar[j] * xp[j];
        for (int j = 0; j < nu; ++j) bu += br[j] * up[j];
        f = (ax + bu) + a.lin_b[(size_t)b * nx + k];
      } else {
        f = nb[(t - 1) * nx + k];
      }
    }
    R h = t == 0 ? xs[k] - a.x0[(size_t)b * nx + k] : f - xs[t * nx + k];
    if (a.scaled) h = h / a.sscale[k];
    e += rabs(h);
  }
  if (a.u0 != nullptr) {
    for (int k = lane; k < nu; k += kWave) {
      R h = us[k] - a.u0[(size_t)b * nu + k];
      if (a.scaled) h = h / a.cscale[k];
      e += rabs(h);
    }
  }
  // inequality rows (+ slack) against their bounds: the box rows, then the
  // obstacle rows of each stage
  const int mr = a.mbox + a.nobs;
  for (int i = lane; i < T * mr; i += kWave) {
    const int t = i / mr, j = i - t * mr;
    R g, lo, hi;
    if (j < a.mbox) {
      const int v = a.box_idx[j];
      g = v < nx ? xs[t * nx + v] : us[t * nu + (v - nx)];
      lo = a.box_lo[j];
      hi = a.box_hi[j];
      if (a.scaled) {
        const R r = a.box_scale[j];
        g = g * r;
        lo = lo * r;
        hi = hi * r;
      }
    } else {
      const int k = j - a.mbox;
      const R* ck = a.centers + ((size_t)b * a.nobs + k) * a.dim;
      R d2 = R(0);
      for (int c = 0; c < a.dim; ++c) {
        const R dc = xs[t * nx + c] - ck[c];
        d2 += dc * dc;
      }
      g = R(1) - r_sqrt(d2) / (a.radii[(size_t)b * a.nobs + k] + R(0.001));
      lo = R(-1.0e9);
      hi = R(0);
      if (a.scaled) {
        g = g * a.obs_scale;
        lo = lo * a.obs_scale;
        hi = hi * a.obs_scale;
      }
    }
    if (a.slacks != nullptr) g = g + a.slacks[(size_t)p * T * mr + i];
    q += clamp0(lo - g) + clamp0(g - hi);
  }
  if (a.slacks != nullptr) {
    R ss = R(0), sd = R(0);
    for (int i = lane; i < T * mr; i += kWave) {
      const R s = a.slacks[(size_t)p * T * mr + i];
      ss += s * s;
      if (a.dslacks != nullptr) sd += s * a.dslacks[(size_t)p * T * mr + i];
    }
    ss = wave_sum(ss);
    sd = wave_sum(sd);
    c = wave_sum(c) + (R(0.5) * a.gamma) * ss;
    dc = wave_sum(dc) + a.gamma * sd;
  } else {
    c = wave_sum(c);
    dc = wave_sum(dc);
  }
  e = wave_sum(e);
  q = wave_sum(q);
  if (lane == 0) {
    a.cost[p] = c;
    if (a.dcost != nullptr) a.dcost[p] = dc;
    a.eq[p] = e;
    a.iq[p] = q;
  }
}

}  // namespace tmpc

namespace tmpc {

// The step choice of the merit line search (backtracking_linesearch,
// turbompc/solvers/linesearch.py:54-178), one thread per problem, from the
// merit terms of the base point and of the A candidates (candidate j of
// problem b at j B + b):
//   cl1 = eq + iq, mu = clip(nan_to_num(dcost / (0.5 max(cl1, floor))), mu_min, mu_max),
//   merit = cost + mu cl1, slope = dcost - mu cl1,
//   cand_j = cost_j + mu (eq_j + iq_j), dec_j = cand_j - (merit + eta alpha_j slope),
//   the largest j with every value finite and dec_j <= 0, else the finite
//   candidate of least merit (the first of equal ones), else candidate 0.
// Each value is formed as the elementwise torch form forms it: one rounding
// per operation (no contraction), the scalars rounded to R first.
constexpr int kMaxAlphas = 8;

template <typename R>
struct ChooseArgs {
  int B, A;
  const R* cost;    // (B)
  const R* dcost;   // (B)
  const R* eq;      // (B)
  const R* iq;      // (B)
  const R* cost_a;  // (A B)
  const R* eq_a;    // (A B)
  const R* iq_a;    // (A B)
  R alpha[kMaxAlphas];
  R eta_alpha[kMaxAlphas];  // eta alpha_j, rounded from its double product
  R mu_min, mu_max, floor_;
  R* alpha_out;  // (B)
  R* mu_out;     // (B) or null
};

template <typename R>
__device__ __forceinline__ bool finite_(R x) {
  return __builtin_isfinite(x);
}

template <typename R>
__global__ __launch_bounds__(256) void linesearch_choose_kernel(ChooseArgs<R> a) {
#pragma clang fp contract(off)
  const int b = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (b >= a.B) return;
  const R cl1 = a.eq[b] + a.iq[b];
  const R den = R(0.5) * (cl1 < a.floor_ ? a.floor_ : cl1);  // clamp(min=floor): NaN stays NaN
  R mu = a.dcost[b] / den;
  if (mu != mu)
    mu = a.mu_min;
  else if (mu == R(__builtin_huge_val()))
    mu = a.mu_max;
  else if (mu == -R(__builtin_huge_val()))
    mu = a.mu_min;
  mu = mu < a.mu_min ? a.mu_min : (mu > a.mu_max ? a.mu_max : mu);
  const R t = mu * cl1;
  const R merit = a.cost[b] + t;
  const R slope = a.dcost[b] - t;
  int valid = -1, best = -1;
  R best_v = R(0);
  for (int j = 0; j < a.A; ++j) {
    const size_t q = (size_t)j * a.B + b;
    const R cand = a.cost_a[q] + mu * (a.eq_a[q] + a.iq_a[q]);
    const R dec = cand - (merit + a.eta_alpha[j] * slope);
    const bool fin = finite_(a.alpha[j]) && finite_(cand) && finite_(dec);
    if (fin && dec <= R(0)) valid = j;
    if (fin && (best < 0 || cand < best_v)) {
      best = j;
      best_v = cand;
    }
  }
  const int index = valid >= 0 ? valid : (best >= 0 ? best : 0);
  a.alpha_out[b] = a.alpha[index];
  if (a.mu_out != nullptr) a.mu_out[b] = mu;
}

}  // namespace tmpc
