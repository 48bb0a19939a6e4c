// Fused batched ADMM with an exact block-tridiagonal Schur solve.
//
// Semantics follow the reference's pure-JAX loop, ADMMSolver._solve_jax_loop
// (turbompc/solvers/admm/admm.py:795-1049): per iteration
//   gamma = sigma x - q + C^T(rho_f c - y_f) + G^T(rho z - y_g)     (:157-174)
//   xt    = S^{-1} gamma                                             (:883)
//   Cxt, Gxt on the pre-relaxation xt                                 (:884-887)
//   x     = alpha xt + (1-alpha) x                                    (:891-893)
//   z, xi = box projection / slack update                             (:895-919)
//   y_f  += rho_f (alpha C xt + (1-alpha) c - c)                      (:924-925)
//   y_g  += rho (alpha G xt + (1-alpha) z_old - z)                    (:929-931)
//   residuals + adaptive rho every check_termination_every            (:392-556)
// and termination by cond_fun (:843-851), decided per problem.
//
// Mapping (gfx950, wave64): a wavefront holds P = 64/g problems, g = max(n, m)
// lanes each; lane i owns row i of every stage block.  The forward sweep is
//   w_t = Theta_t^{-1}(gamma_t - phi_{t-1} w_{t-1})
// and the backward sweep
//   xt_t = w_t - Theta_t^{-1} phi_t^T xt_{t+1}
// fused with everything that needs stage t only: C/G products, relaxation,
// projection, dual updates and the next iteration's gamma_t.  phi is never
// stored: phi_t = E_t + rho_f A_plus_t^T A_minus_t is applied from the QP blocks
// (STD = A_plus_t == [-I 0] and E_t == 0, the explicit-integrator case, needs
// A_minus only).  Per stage the kernel streams Theta_t^{-1} (packed) and
// A_minus_t twice and every other block once.
//
// The loop runs in chunks that end at the adaptive-rho points; a rho change
// flags the problem and the host re-launches factor_kernel for the flagged
// problems before the next chunk (no host synchronisation).
#pragma once
#include "common.hpp"

namespace tmpc {

template <typename R>
struct AdmmArgs {
  Dims d;
  QPDev<R> qp;
  StateDev<R> st;    // working state, updated in place
  const R* thinv;    // [T][B][packed n]
  R* w;              // [T][B][n]
  R* gam;            // [T][B][n]
  int32_t* ctl;      // [B][4]: it, done, refactor flag, unused
  R* res;            // [B][8]: rp, rd, np, nd, pn, dn
  uint32_t* iters_out;
  R sigma, alpha, rho_f_factor, eps_abs, eps_rel, rho_min, rho_max, rho_tol;
  int max_iter, check_every, adapt_every, use_slack;
  int it_lo, it_hi, first_chunk;
  int g, P;
  const uint8_t* act;  // (B,) or null: problems with act[b] == 0 run no iteration
};

enum { SB_W, SB_R, SB_U, SB_S, SB_X, SB_C, SB_Z, SB_C0, SB_XP, SB_XN, SB_YP, SB_Y, SB_YG, SB_CP, SB_COUNT };
constexpr int kRed = 12;

template <typename R>
struct Shared {
  R v[SB_COUNT][kWave];
  R red[kRed][kWave];
};

// Theta^{-1} (packed lower) row i times the group vector v.
template <typename R, int NC>
__device__ __forceinline__ R sym_row_dot(const R* __restrict__ Th, int i, int n, const R* v) {
  R acc = R(0);
  const int ri = (i * (i + 1)) >> 1;
#pragma unroll
  for (int k = 0; k < (NC > 0 ? NC : 64); ++k) {
    if (NC == 0 && k >= n) break;
    const int idx = k <= i ? ri + k : ((k * (k + 1)) >> 1) + i;
    acc += Th[idx] * v[k];
  }
  return acc;
}

// row r of a (rows x n) row-major block times v
template <typename R, int NC>
__device__ __forceinline__ R row_dot(const R* __restrict__ A, int r, int n, const R* v) {
  R acc = R(0);
  const R* a = A + r * n;
#pragma unroll
  for (int k = 0; k < (NC > 0 ? NC : 64); ++k) {
    if (NC == 0 && k >= n) break;
    acc += a[k] * v[k];
  }
  return acc;
}

// column j of a (rows x n) row-major block times v (length rows)
template <typename R>
__device__ __forceinline__ R col_dot(const R* __restrict__ A, int rows, int n, int j, const R* v) {
  R acc = R(0);
  for (int r = 0; r < rows; ++r) acc += A[r * n + j] * v[r];
  return acc;
}

// gamma for the current state and rho (compute_gamma, admm.py:157-174).
template <typename R, int NC>
__device__ void gamma_pass(const AdmmArgs<R>& a, const Group& G, Shared<R>& sh, R rho) {
  const Dims& d = a.d;
  const int n = NC > 0 ? NC : d.n;
  const int T = d.T, N = d.N, nx = d.nx, n0 = d.n0, m = d.m, B = d.B;
  const int b = G.prob, i = G.lane, base = G.gid * a.g;
  const R rho_f = rho * a.rho_f_factor;
  R* sc = sh.v[SB_C] + base;
  R* scp = sh.v[SB_CP] + base;
  R* sz = sh.v[SB_Z] + base;
  R* sc0 = sh.v[SB_C0] + base;
  for (int t = 0; t < T; ++t) {
    if (t < N && i < nx) sc[i] = rho_f * a.qp.c[((size_t)b * N + t) * nx + i] - a.st.y_f[((size_t)b * N + t) * nx + i];
    if (i < m)
      sz[i] = rho * a.st.z[((size_t)b * T + t) * m + i] - a.st.y_g[((size_t)b * T + t) * m + i];
    if (t == 0 && i < n0) sc0[i] = rho_f * a.qp.c0[(size_t)b * n0 + i] - a.st.y_f0[(size_t)b * n0 + i];
    wsync();
    if (i < n) {
      R gv = a.sigma * a.st.x[((size_t)b * T + t) * n + i] - a.qp.q[((size_t)b * T + t) * n + i];
      if (t < N) gv += col_dot(a.qp.Am + ((size_t)b * N + t) * nx * n, nx, n, i, sc);
      if (t > 0) gv += col_dot(a.qp.Ap + ((size_t)b * N + t - 1) * nx * n, nx, n, i, scp);
      if (m) gv += col_dot(a.qp.G + ((size_t)b * T + t) * m * n, m, n, i, sz);
      if (t == 0) gv += col_dot(a.qp.A0 + (size_t)b * n0 * n, n0, n, i, sc0);
      if (G.live) a.gam[((size_t)t * B + b) * n + i] = gv;
    }
    wsync();
    if (t < N && i < nx) scp[i] = sc[i];
    wsync();
  }
}

// _compute_residuals (admm.py:266-331) on the current state; returns the six
// group-uniform values rp, rd, np, nd, pn, dn in out[].
template <typename R, int NC>
__device__ void residual_pass(const AdmmArgs<R>& a, const Group& G, Shared<R>& sh, R* out) {
  const Dims& d = a.d;
  const int n = NC > 0 ? NC : d.n;
  const int T = d.T, N = d.N, nx = d.nx, n0 = d.n0, m = d.m;
  const int b = G.prob, i = G.lane, base = G.gid * a.g;
  const bool slack = a.use_slack && m > 0;
  const R gs = (slack && a.qp.slack_w) ? a.qp.slack_w[b] : R(0);
  R* xp = sh.v[SB_XP] + base;
  R* xc = sh.v[SB_X] + base;
  R* xn = sh.v[SB_XN] + base;
  R* yp = sh.v[SB_YP] + base;
  R* yc = sh.v[SB_Y] + base;
  R* yg = sh.v[SB_YG] + base;
  R* y0 = sh.v[SB_C0] + base;
  R rp = 0, nCx = 0, nc = 0, nGx = 0, nz = 0, rd = 0, nPx = 0, nAty = 0, nq = 0, nxi = 0, nyg = 0;
  const R* X = a.st.x + (size_t)b * T * n;
  if (i < n) {
    xc[i] = X[i];
    xn[i] = T > 1 ? X[n + i] : R(0);
  }
  if (i < n0) y0[i] = a.st.y_f0[(size_t)b * n0 + i];
  for (int t = 0; t < T; ++t) {
    if (t < N && i < nx) yc[i] = a.st.y_f[((size_t)b * N + t) * nx + i];
    if (i < m) yg[i] = a.st.y_g[((size_t)b * T + t) * m + i];
    wsync();
    if (i < n) {
      R px = row_dot<R, NC>(a.qp.D + ((size_t)b * T + t) * n * n, i, n, xc);
      if (t > 0) px += row_dot<R, NC>(a.qp.E + ((size_t)b * N + t - 1) * n * n, i, n, xp);
      if (t < N) {
        const R* Et = a.qp.E + ((size_t)b * N + t) * n * n;
        R s = 0;
        for (int k = 0; k < n; ++k) s += Et[k * n + i] * xn[k];
        px += s;
      }
      R aty = R(0);
      if (t == 0) aty += col_dot(a.qp.A0 + (size_t)b * n0 * n, n0, n, i, y0);
      if (t < N) aty += col_dot(a.qp.Am + ((size_t)b * N + t) * nx * n, nx, n, i, yc);
      if (t > 0) aty += col_dot(a.qp.Ap + ((size_t)b * N + t - 1) * nx * n, nx, n, i, yp);
      if (m) aty += col_dot(a.qp.G + ((size_t)b * T + t) * m * n, m, n, i, yg);
      const R qv = a.qp.q[((size_t)b * T + t) * n + i];
      rd = rmax(rd, rabs(px + qv + aty));
      nPx = rmax(nPx, rabs(px));
      nAty = rmax(nAty, rabs(aty));
      nq = rmax(nq, rabs(qv));
    }
    if (t < N && i < nx) {
      const R cx = row_dot<R, NC>(a.qp.Am + ((size_t)b * N + t) * nx * n, i, n, xc) +
                   row_dot<R, NC>(a.qp.Ap + ((size_t)b * N + t) * nx * n, i, n, xn);
      const R cv = a.qp.c[((size_t)b * N + t) * nx + i];
      rp = rmax(rp, rabs(cx - cv));
      nCx = rmax(nCx, rabs(cx));
      nc = rmax(nc, rabs(cv));
    }
    if (t == 0 && i < n0) {
      const R cx = row_dot<R, NC>(a.qp.A0 + (size_t)b * n0 * n, i, n, xc);
      const R cv = a.qp.c0[(size_t)b * n0 + i];
      rp = rmax(rp, rabs(cx - cv));
      nCx = rmax(nCx, rabs(cx));
      nc = rmax(nc, rabs(cv));
    }
    if (i < m) {
      const R gx = row_dot<R, NC>(a.qp.G + ((size_t)b * T + t) * m * n, i, n, xc);
      const R zv = a.st.z[((size_t)b * T + t) * m + i];
      rp = rmax(rp, rabs(gx - zv));
      nGx = rmax(nGx, rabs(gx));
      nz = rmax(nz, rabs(zv));
      if (slack) {
        const R xv = a.st.xi[((size_t)b * T + t) * m + i];
        rd = rmax(rd, rabs(gs * xv + yg[i]));
        nxi = rmax(nxi, rabs(xv));
        nyg = rmax(nyg, rabs(yg[i]));
      }
    }
    wsync();
    // rotate the x window and the y_f history
    if (i < n) {
      xp[i] = xc[i];
      xc[i] = xn[i];
    }
    if (t < N && i < nx) yp[i] = yc[i];
    wsync();
    if (i < n) xn[i] = (t + 2 < T) ? X[(size_t)(t + 2) * n + i] : R(0);
  }
  // group max-reductions
  R vals[11] = {rp, nCx, nc, nGx, nz, rd, nPx, nAty, nq, nxi, nyg};
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 11; ++k) sh.red[k][tid] = (i < a.g) ? vals[k] : R(0);
  wsync();
  R r[11];
#pragma unroll
  for (int k = 0; k < 11; ++k) {
    R mx = R(0);
    for (int l = 0; l < a.g; ++l) mx = rmax(mx, sh.red[k][base + l]);
    r[k] = mx;
  }
  wsync();
  const R np = rmax(rmax(r[1], r[3]), rmax(r[2], r[4]));
  R nd = rmax(rmax(r[6], r[7]), r[8]);
  if (slack) nd = rmax(nd, rmax(gs * r[9], r[10]));
  out[0] = r[0];
  out[1] = r[5];
  out[2] = np;
  out[3] = nd;
  out[4] = r[0] / (R(1e-10) + np);
  out[5] = r[5] / (R(1e-10) + nd);
}

template <typename R, int NC, bool STD>
__global__ __launch_bounds__(kWave) void admm_chunk_kernel(AdmmArgs<R> a) {
  __shared__ Shared<R> sh;
  const Dims d = a.d;
  const int n = NC > 0 ? NC : d.n;
  const int T = d.T, N = d.N, nx = d.nx, n0 = d.n0, m = d.m, B = d.B;
  const int pk = th_pitch(n);
  const Group G = make_group(a.g, a.P, B);
  const int b = G.prob, i = G.lane, base = G.gid * a.g;
  const R alpha = a.alpha, one_m_alpha = R(1) - a.alpha;

  // ---- per-problem control state ------------------------------------------
  int it;
  bool done;
  R res[6];
  if (a.first_chunk) {
    // init_residuals of the reference loop (admm.py:998-1005): infinite
    // residuals and unit norm terms; res[] = {rp, rd, np, nd, pn, dn}
    it = 0;
    done = a.act ? a.act[b] == 0 : false;
    res[0] = res[1] = res[4] = res[5] = rinf<R>();
    res[2] = res[3] = R(1);
    if (G.live && i == 0) a.ctl[b * 4 + 2] = 0;
  } else {
    it = a.ctl[b * 4 + 0];
    done = a.ctl[b * 4 + 1] != 0;
#pragma unroll
    for (int k = 0; k < 6; ++k) res[k] = a.res[b * 8 + k];
  }
  R rho = a.st.rho[b];
  gamma_pass<R, NC>(a, G, sh, rho);

  const R* QAm = a.qp.Am + (size_t)b * N * nx * n;
  const R* QAp = a.qp.Ap + (size_t)b * N * nx * n;
  const R* QE = a.qp.E + (size_t)b * N * n * n;
  const R* QG = a.qp.G + (size_t)b * T * m * n;
  const R* QA0 = a.qp.A0 + (size_t)b * n0 * n;
  R* sw = sh.v[SB_W] + base;
  R* sr = sh.v[SB_R] + base;
  R* su = sh.v[SB_U] + base;
  R* ss = sh.v[SB_S] + base;
  R* sx = sh.v[SB_X] + base;
  R* sc = sh.v[SB_C] + base;
  R* sz = sh.v[SB_Z] + base;
  R* sc0 = sh.v[SB_C0] + base;
  const R gs = (a.use_slack && m > 0 && a.qp.slack_w) ? a.qp.slack_w[b] : R(0);

  for (int iter = a.it_lo; iter < a.it_hi; ++iter) {
    // cond_fun (admm.py:843-851)
    bool active = false;
    if (!done) {
      const bool sc_ = mod_zero(iter, a.check_every);
      const bool tl = (res[0] > a.eps_abs + a.eps_rel * res[2]) || (res[1] > a.eps_abs + a.eps_rel * res[3]);
      active = (iter < a.max_iter) && (!sc_ || tl);
      active = active || iter < 1;
      if (!active) done = true;
    }
    const bool commit = active && G.live;
    if (__ballot(active && G.real) == 0) break;
    const R rho_f = rho * a.rho_f_factor;

    // ---- forward sweep: w_t = Theta_t^{-1} (gamma_t - phi_{t-1} w_{t-1}) ----
    for (int t = 0; t < T; ++t) {
      R r = (i < n) ? a.gam[((size_t)t * B + b) * n + i] : R(0);
      if (t > 0) {
        R v = (i < nx) ? row_dot<R, NC>(QAm + (size_t)(t - 1) * nx * n, i, n, sw) : R(0);
        if (STD) {
          if (i < nx) r += rho_f * v;
        } else {
          if (i < nx) su[i] = v;
          wsync();
          if (i < n) {
            R s = row_dot<R, NC>(QE + (size_t)(t - 1) * n * n, i, n, sw);
            s += rho_f * col_dot(QAp + (size_t)(t - 1) * nx * n, nx, n, i, su);
            r -= s;
          }
        }
      }
      if (i < n) sr[i] = r;
      wsync();
      R wv = R(0);
      if (i < n) {
        wv = sym_row_dot<R, NC>(a.thinv + ((size_t)t * B + b) * pk, i, n, sr);
        if (G.live) a.w[((size_t)t * B + b) * n + i] = wv;
        sw[i] = wv;
      }
      wsync();
    }

    // ---- backward sweep fused with the ADMM updates -------------------------
    R xn = R(0);  // xt_{t+1}[i]
    R gp = R(0);  // gamma_{t+1}[i] awaiting its A_plus_t^T term
    for (int t = T - 1; t >= 0; --t) {
      const R wv = (i < n) ? a.w[((size_t)t * B + b) * n + i] : R(0);
      R xt = wv;
      R u = R(0);  // (A_plus_t xt_{t+1})[i], i < nx
      if (t < N) {
        if (STD) {
          u = (i < nx) ? -xn : R(0);
        } else {
          if (i < n) sx[i] = xn;
          wsync();
          if (i < nx) u = row_dot<R, NC>(QAp + (size_t)t * nx * n, i, n, sx);
        }
        if (i < nx) su[i] = u;
        wsync();
        R s = R(0);
        if (i < n) {
          s = rho_f * col_dot(QAm + (size_t)t * nx * n, nx, n, i, su);
          if (!STD) {
            const R* Et = QE + (size_t)t * n * n;
            for (int k = 0; k < n; ++k) s += Et[k * n + i] * sx[k];
          }
          ss[i] = s;
        }
        wsync();
        if (i < n) xt = wv - sym_row_dot<R, NC>(a.thinv + ((size_t)t * B + b) * pk, i, n, ss);
        wsync();
      }
      if (i < n) sx[i] = xt;
      wsync();
      // C and G products of the pre-relaxation iterate
      R cx = R(0), cx0 = R(0), gx = R(0);
      if (t < N && i < nx) cx = row_dot<R, NC>(QAm + (size_t)t * nx * n, i, n, sx) + u;
      if (t == 0 && i < n0) cx0 = row_dot<R, NC>(QA0, i, n, sx);
      if (i < m) gx = row_dot<R, NC>(QG + (size_t)t * m * n, i, n, sx);
      // over-relaxation
      R xnew = R(0);
      if (i < n) {
        R* xp = a.st.x + ((size_t)b * T + t) * n + i;
        xnew = alpha * xt + one_m_alpha * (*xp);
        if (commit) *xp = xnew;
      }
      // box projection / slack and the inequality dual
      R zeta = R(0);
      if (i < m) {
        const size_t o = ((size_t)b * T + t) * m + i;
        const R zo = a.st.z[o], ygo = a.st.y_g[o];
        const R zt = alpha * gx + one_m_alpha * zo + ygo / rho;
        const R proj = rmin(rmax(zt, a.qp.l[o]), a.qp.u[o]);
        R zn, xin;
        if (a.use_slack) {
          const R frac = gs / (gs + rho);
          zn = (R(1) - frac) * zt + frac * proj;
          xin = (rho / (gs + rho)) * (proj - zt);
        } else {
          zn = proj;
          xin = R(0);
        }
        const R ygn = ygo + rho * (alpha * gx + one_m_alpha * zo - zn);
        if (commit) {
          a.st.z[o] = zn;
          a.st.xi[o] = xin;
          a.st.y_g[o] = ygn;
        }
        zeta = rho * zn - ygn;
      }
      // equality duals
      R ct = R(0), ct0 = R(0);
      if (t < N && i < nx) {
        const size_t o = ((size_t)b * N + t) * nx + i;
        const R cv = a.qp.c[o];
        const R yf = a.st.y_f[o] + rho_f * (alpha * cx + one_m_alpha * cv - cv);
        if (commit) a.st.y_f[o] = yf;
        ct = rho_f * cv - yf;
      }
      if (t == 0 && i < n0) {
        const size_t o = (size_t)b * n0 + i;
        const R cv = a.qp.c0[o];
        const R yf = a.st.y_f0[o] + rho_f * (alpha * cx0 + one_m_alpha * cv - cv);
        if (commit) a.st.y_f0[o] = yf;
        ct0 = rho_f * cv - yf;
      }
      // next iteration's gamma (valid while rho is unchanged)
      if (i < nx) sc[i] = ct;
      if (i < m) sz[i] = zeta;
      if (i < n0) sc0[i] = ct0;
      wsync();
      if (t < N) {
        if (STD) {
          if (i < nx) gp -= sc[i];
        } else if (i < n) {
          gp += col_dot(QAp + (size_t)t * nx * n, nx, n, i, sc);
        }
        if (i < n && commit) a.gam[((size_t)(t + 1) * B + b) * n + i] = gp;
      }
      if (i < n) {
        R gv = a.sigma * xnew - a.qp.q[((size_t)b * T + t) * n + i];
        if (t < N) gv += col_dot(QAm + (size_t)t * nx * n, nx, n, i, sc);
        if (m) gv += col_dot(QG + (size_t)t * m * n, m, n, i, sz);
        if (t == 0) gv += col_dot(QA0, n0, n, i, sc0);
        gp = gv;
      }
      xn = xt;
      wsync();
    }
    if (i < n && commit) a.gam[(size_t)b * n + i] = gp;
    wsync();

    // ---- residuals and adaptive rho (admm.py:392-556) ----------------------
    if (mod_zero(iter, a.check_every)) {
      R rv[6];
      residual_pass<R, NC>(a, G, sh, rv);
      if (active) {
#pragma unroll
        for (int k = 0; k < 6; ++k) res[k] = rv[k];
        const R cand = rmin(rmax(rho * r_sqrt(rv[4] / rv[5]), a.rho_min), a.rho_max);
        const R ratio = rmax(cand / rho, rho / cand);
        const bool conv = !((rv[0] > a.eps_abs + a.eps_rel * rv[2]) || (rv[1] > a.eps_abs + a.eps_rel * rv[3]));
        bool keep = iter < 2 || !mod_zero(iter, a.adapt_every);
        keep = keep || conv;
        keep = keep || ratio < a.rho_tol;
        if (!keep) {
          rho = cand;
          if (G.live && i == 0) {
            a.st.rho[b] = cand;
            a.ctl[b * 4 + 2] = 1;
          }
        }
      }
    }
    if (active) it = iter + 1;
  }
  if (G.live && i == 0) {
    a.ctl[b * 4 + 0] = it;
    a.ctl[b * 4 + 1] = done ? 1 : 0;
#pragma unroll
    for (int k = 0; k < 6; ++k) a.res[b * 8 + k] = res[k];
    a.iters_out[b] = (uint32_t)it;
  }
}

// Schur-only exact solve S x = rhs from the factor of S (phi read from S).
template <typename R, int NC>
__global__ __launch_bounds__(kWave) void blktri_solve_kernel(Dims d, int g, int P, const R* __restrict__ S,
                                                             const R* __restrict__ thinv,
                                                             const R* __restrict__ rhs, R* __restrict__ x) {
  __shared__ R sv[3][kWave];
  const int n = NC > 0 ? NC : d.n;
  const int T = d.T, B = d.B, pk = th_pitch(n), w3 = 3 * n;
  const Group G = make_group(g, P, B);
  const int b = G.prob, i = G.lane, base = G.gid * g;
  R* sw = sv[0] + base;
  R* sr = sv[1] + base;
  for (int t = 0; t < T; ++t) {
    R r = (i < n) ? rhs[((size_t)b * T + t) * n + i] : R(0);
    if (t > 0 && i < n) {
      // phi_{t-1} w_{t-1}: phi_{t-1} is the sub-diagonal block of block row t
      const R* row = S + (((size_t)b * T + t) * n + i) * w3;
      R s = R(0);
      for (int k = 0; k < n; ++k) s += row[k] * sw[k];
      r -= s;
    }
    if (i < n) sr[i] = r;
    wsync();
    if (i < n) {
      const R wv = sym_row_dot<R, NC>(thinv + ((size_t)t * B + b) * pk, i, n, sr);
      if (G.live) x[((size_t)b * T + t) * n + i] = wv;
      sw[i] = wv;
    }
    wsync();
  }
  R xn = R(0);
  for (int t = T - 1; t >= 0; --t) {
    R xt = (i < n) ? x[((size_t)b * T + t) * n + i] : R(0);
    if (t < T - 1) {
      if (i < n) sw[i] = xn;
      wsync();
      R s = R(0);
      if (i < n) {
        // phi_t^T xt_{t+1}: phi_t = sub-diagonal block of block row t+1
        const R* Sn = S + ((size_t)b * T + t + 1) * n * w3;
        for (int k = 0; k < n; ++k) s += Sn[k * w3 + i] * sw[k];
        sr[i] = s;
      }
      wsync();
      if (i < n) xt -= sym_row_dot<R, NC>(thinv + ((size_t)t * B + b) * pk, i, n, sr);
      wsync();
    }
    if (i < n && G.live) x[((size_t)b * T + t) * n + i] = xt;
    xn = xt;
  }
}

}  // namespace tmpc
