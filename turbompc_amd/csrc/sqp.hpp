// SQP first-order convergence check on the device.
//
// _compute_first_order_convergence_error (turbompc/solvers/turbompc_solver.py:1158-1225)
// evaluated at x = (states, controls) against the relinearized QP:
//   stationarity  = || P x + q + C^T y_f + G^T y_g ||_inf
//   eq_err        = || C x - c ||_inf
//   ineq_err      = || max(l - g, 0), max(g - u, 0) ||_inf,  g = G x (+ slack)
//   conv          = max(stationarity, eq_err, ineq_err, slack stationarity)
// and g itself (the inequality values the KKT-state active sets are built
// from, :1387-1439).  One group of g = max(n, m) lanes per problem walks the
// stages with a three-stage window of x in LDS, like the ADMM residual pass.
#pragma once
#include "admm_direct.hpp"
#include "common.hpp"

namespace tmpc {

template <typename R, int NC>
__global__ __launch_bounds__(kWave) void sqp_check_kernel(Dims d, int g, int P, QPDev<R> qp, const R* __restrict__ x,
                                                          const R* __restrict__ y0, const R* __restrict__ yf,
                                                          const R* __restrict__ yg, const R* __restrict__ slack,
                                                          R slack_w, R* __restrict__ conv, R* __restrict__ eq_err,
                                                          R* __restrict__ ineq_err, R* __restrict__ gout) {
  __shared__ R sv[7][kWave];
  __shared__ R red[4][kWave];
  const int n = NC > 0 ? NC : d.n;
  const int T = d.T, N = d.N, nx = d.nx, n0 = d.n0, m = d.m;
  const Group G = make_group(g, P, d.B);
  const int b = G.prob, i = G.lane, base = G.gid * g;
  R* xp = sv[0] + base;
  R* xc = sv[1] + base;
  R* xn = sv[2] + base;
  R* yp = sv[3] + base;
  R* yc = sv[4] + base;
  R* yy = sv[5] + base;
  R* y00 = sv[6] + base;
  const R* X = x + (size_t)b * T * n;
  R st = 0, eq = 0, iq = 0, sl = 0;
  if (i < n) {
    xp[i] = R(0);
    xc[i] = X[i];
    xn[i] = X[n + i];
  }
  if (i < n0) y00[i] = y0[(size_t)b * n0 + i];
  for (int t = 0; t < T; ++t) {
    if (t < N && i < nx) yc[i] = yf[((size_t)b * N + t) * nx + i];
    if (i < m) yy[i] = yg[((size_t)b * T + t) * m + i];
    wsync();
    if (i < n) {
      R px = row_dot<R, NC>(qp.D + ((size_t)b * T + t) * n * n, i, n, xc);
      if (t > 0) px += row_dot<R, NC>(qp.E + ((size_t)b * N + t - 1) * n * n, i, n, xp);
      if (t < N) {
        const R* Et = qp.E + ((size_t)b * N + t) * n * n;
        R s = 0;
        for (int k = 0; k < n; ++k) s += Et[k * n + i] * xn[k];
        px += s;
      }
      R aty = R(0);
      if (t == 0) aty += col_dot(qp.A0 + (size_t)b * n0 * n, n0, n, i, y00);
      if (t < N) aty += col_dot(qp.Am + ((size_t)b * N + t) * nx * n, nx, n, i, yc);
      if (t > 0) aty += col_dot(qp.Ap + ((size_t)b * N + t - 1) * nx * n, nx, n, i, yp);
      if (m) aty += col_dot(qp.G + ((size_t)b * T + t) * m * n, m, n, i, yy);
      st = rmax(st, rabs(px + qp.q[((size_t)b * T + t) * n + i] + aty));
    }
    if (t < N && i < nx) {
      const R cx = row_dot<R, NC>(qp.Am + ((size_t)b * N + t) * nx * n, i, n, xc) +
                   row_dot<R, NC>(qp.Ap + ((size_t)b * N + t) * nx * n, i, n, xn);
      eq = rmax(eq, rabs(cx - qp.c[((size_t)b * N + t) * nx + i]));
    }
    if (t == 0 && i < n0) eq = rmax(eq, rabs(row_dot<R, NC>(qp.A0 + (size_t)b * n0 * n, i, n, xc) - qp.c0[(size_t)b * n0 + i]));
    if (i < m) {
      const size_t o = ((size_t)b * T + t) * m + i;
      R gv = row_dot<R, NC>(qp.G + ((size_t)b * T + t) * m * n, i, n, xc);
      if (slack) {
        gv += slack[o];
        sl = rmax(sl, rabs(slack_w * slack[o] + yy[i]));
      }
      iq = rmax(iq, rmax(rmax(qp.l[o] - gv, R(0)), rmax(gv - qp.u[o], R(0))));
      if (G.live && gout) gout[o] = gv;
    }
    wsync();
    if (i < n) {
      xp[i] = xc[i];
      xc[i] = xn[i];
    }
    if (t < N && i < nx) yp[i] = yc[i];
    wsync();
    if (i < n) xn[i] = (t + 2 < T) ? X[(size_t)(t + 2) * n + i] : R(0);
  }
  const int tid = threadIdx.x;
  red[0][tid] = i < g ? st : R(0);
  red[1][tid] = i < g ? eq : R(0);
  red[2][tid] = i < g ? iq : R(0);
  red[3][tid] = i < g ? sl : R(0);
  wsync();
  if (G.live && i == 0) {
    R r[4] = {0, 0, 0, 0};
    for (int k = 0; k < 4; ++k)
      for (int l = 0; l < g; ++l) r[k] = rmax(r[k], red[k][base + l]);
    conv[b] = rmax(r[0], rmax(r[1], rmax(r[2], r[3])));
    if (eq_err) eq_err[b] = r[1];
    if (ineq_err) ineq_err[b] = r[2];
  }
}

}  // namespace tmpc
