// Block-tridiagonal Schur-complement PCG (the reference's iterative Schur path).
//
//   schur_build_kernel   compute_S_Phiinv (turbompc/solvers/admm/admm.py:71-154):
//                        S row t = [phi_{t-1} | theta_t | phi_t^T],
//                        Phiinv row t = [theta_t^{-1} phi_{t-1} theta_{t-1}^{-1} |
//                                        -theta_t^{-1} | theta_t^{-1} phi_t^T theta_{t+1}^{-1}]
//   pcg_device           PCGPrimalOptimalControl.solve_linear_system
//                        (turbompc/solvers/linear_systems_solvers/pcg_primal.py:70-175),
//                        stopping rule |eta| < 1e-12 + eps |eta_0|, at least one
//                        iteration unless |eta_0| <= 1e-12.
//   admm_pcg_chunk_kernel  the ADMM loop of admm_direct.hpp with the exact
//                        solve replaced by PCG warm-started at x (admm.py:882-883).
//
// Mapping: g = max(n, m) lanes per problem (lane i = row i), stages walked in
// order; the three-stage window of the vector being multiplied sits in LDS and
// the dot products are reduced across the group through LDS.
#pragma once
#include "admm_direct.hpp"
#include "common.hpp"
#include "factor.hpp"

namespace tmpc {

// ------------------------------------------------------------ S / Phiinv ----
template <typename R>
__global__ __launch_bounds__(kWave) void schur_build_kernel(Dims d, QPDev<R> qp, const R* __restrict__ rho,
                                                            R sigma, R rho_f_factor,
                                                            int32_t* __restrict__ ctl, R* __restrict__ S,
                                                            R* __restrict__ Phiinv) {
  const int b = blockIdx.x;
  if (b >= d.B) return;
  if (ctl != nullptr && ctl[b * 4 + 2] == 0) return;
  const int tid = threadIdx.x;
  const int T = d.T, N = d.N, n = d.n, nx = d.nx, n0 = d.n0, m = d.m;
  const int nn = n * n, w3 = 3 * n;
  extern __shared__ unsigned char smem_raw[];
  // computed in double like factor_kernel; S and Phiinv are rounded on store
  Cmp* sm = reinterpret_cast<Cmp*>(smem_raw);
  Cmp* A = sm;          // theta_t -> theta_t^{-1}
  Cmp* Ainv = A + nn;   // theta_{t-1}^{-1}
  Cmp* ph = Ainv + nn;  // phi_{t-1}
  Cmp* tmp = ph + nn;
  Cmp* rowk = tmp + nn;
  Cmp* colk = rowk + n;
  Cmp* sG = colk + n;
  Cmp* sAm = sG + m * n;
  Cmp* sAp = sAm + nx * n;
  Cmp* sApp = sAp + nx * n;
  Cmp* sA0 = sApp + nx * n;
  const Cmp rho_i = (Cmp)rho[b];
  const Cmp rho_f = rho_i * (Cmp)rho_f_factor;
  const Cmp sig = (Cmp)sigma;
  for (int e = tid; e < n0 * n; e += kWave) sA0[e] = (Cmp)qp.A0[(size_t)b * n0 * n + e];
  R* Sb = S + (size_t)b * T * n * w3;
  R* Pb = Phiinv + (size_t)b * T * n * w3;
  for (int t = 0; t < T; ++t) {
    for (int e = tid; e < m * n; e += kWave) sG[e] = (Cmp)qp.G[((size_t)b * T + t) * m * n + e];
    if (t < N)
      for (int e = tid; e < nx * n; e += kWave) {
        sAm[e] = (Cmp)qp.Am[((size_t)b * N + t) * nx * n + e];
        sAp[e] = (Cmp)qp.Ap[((size_t)b * N + t) * nx * n + e];
      }
    wsync();
    for (int e = tid; e < nn; e += kWave) {
      const int i = e / n, j = e - (e / n) * n;
      Cmp v = (Cmp)qp.D[((size_t)b * T + t) * nn + e] + (i == j ? sig : Cmp(0));
      Cmp gg = 0;
      for (int r = 0; r < m; ++r) gg += sG[r * n + i] * sG[r * n + j];
      Cmp cc = 0;
      if (t == 0)
        for (int r = 0; r < n0; ++r) cc += sA0[r * n + i] * sA0[r * n + j];
      if (t < N)
        for (int r = 0; r < nx; ++r) cc += sAm[r * n + i] * sAm[r * n + j];
      if (t > 0)
        for (int r = 0; r < nx; ++r) cc += sApp[r * n + i] * sApp[r * n + j];
      const Cmp th = v + rho_i * gg + rho_f * cc;
      A[e] = th;
      Sb[((size_t)t * n + i) * w3 + n + j] = (R)th;                        // theta_t
      Sb[((size_t)t * n + i) * w3 + j] = t > 0 ? (R)ph[e] : R(0);          // phi_{t-1}
    }
    wsync();
    gj_invert_spd(A, rowk, colk, n);  // theta_t^{-1} (theta_t is SPD)
    for (int e = tid; e < nn; e += kWave) {
      const int i = e / n, j = e - (e / n) * n;
      Pb[((size_t)t * n + i) * w3 + n + j] = (R)(-A[e]);
    }
    if (t > 0) {
      // tmp = phi_{t-1} theta_{t-1}^{-1};  prev_t = theta_t^{-1} tmp
      for (int e = tid; e < nn; e += kWave) {
        const int i = e / n, j = e - (e / n) * n;
        Cmp s = 0;
        for (int l = 0; l < n; ++l) s += ph[i * n + l] * Ainv[l * n + j];
        tmp[e] = s;
      }
      wsync();
      for (int e = tid; e < nn; e += kWave) {
        const int i = e / n, j = e - (e / n) * n;
        Cmp s = 0;
        for (int l = 0; l < n; ++l) s += A[i * n + l] * tmp[l * n + j];
        Pb[((size_t)t * n + i) * w3 + j] = (R)s;
      }
      wsync();
      // next_{t-1} = theta_{t-1}^{-1} phi_{t-1}^T theta_t^{-1}; tmp = phi_{t-1}^T theta_t^{-1}
      for (int e = tid; e < nn; e += kWave) {
        const int i = e / n, j = e - (e / n) * n;
        Cmp s = 0;
        for (int l = 0; l < n; ++l) s += ph[l * n + i] * A[l * n + j];
        tmp[e] = s;
      }
      wsync();
      for (int e = tid; e < nn; e += kWave) {
        const int i = e / n, j = e - (e / n) * n;
        Cmp s = 0;
        for (int l = 0; l < n; ++l) s += Ainv[i * n + l] * tmp[l * n + j];
        Pb[((size_t)(t - 1) * n + i) * w3 + 2 * n + j] = (R)s;
      }
      wsync();
    } else {
      for (int e = tid; e < nn; e += kWave) {
        const int i = e / n, j = e - (e / n) * n;
        Pb[((size_t)t * n + i) * w3 + j] = R(0);
      }
    }
    // phi_t, the S super-diagonal block phi_t^T and the carried theta_t^{-1}
    for (int e = tid; e < nn; e += kWave) {
      const int i = e / n, j = e - (e / n) * n;
      Ainv[e] = A[e];
      if (t < N) {
        Cmp s = 0;
        for (int r = 0; r < nx; ++r) s += sAp[r * n + i] * sAm[r * n + j];
        ph[e] = (Cmp)qp.E[((size_t)b * N + t) * nn + e] + rho_f * s;
      }
    }
    wsync();
    for (int e = tid; e < nn; e += kWave) {
      const int i = e / n, j = e - (e / n) * n;
      Sb[((size_t)t * n + i) * w3 + 2 * n + j] = t < N ? (R)ph[j * n + i] : R(0);
      if (t == N) Pb[((size_t)t * n + i) * w3 + 2 * n + j] = R(0);
    }
    if (t < N)
      for (int e = tid; e < nx * n; e += kWave) sApp[e] = sAp[e];
    wsync();
  }
  if (ctl != nullptr && tid == 0) ctl[b * 4 + 2] = 0;
}

// --------------------------------------------------------------- PCG core ----
template <typename R>
struct PcgVecs {
  R *x, *r, *p, *q, *rt;  // problem-major (B,T,n)
};

// out_t = Blk_t [v_{t-1}; v_t; v_{t+1}] for all t; returns the group-uniform
// dot(dv, out) (dv = v when dv == nullptr).
template <typename R, int NC>
__device__ R blk_matvec(const Dims& d, const Group& G, int g, R* sh3, R* red, const R* __restrict__ Blk,
                        const R* v, R* out, const R* dv) {
  const int n = NC > 0 ? NC : d.n;
  const int T = d.T, w3 = 3 * n;
  const int b = G.prob, i = G.lane, base = G.gid * g;
  R* vp = sh3;
  R* vc = sh3 + kWave;
  R* vn = sh3 + 2 * kWave;
  const R* V = v + (size_t)b * T * n;
  if (i < n) {
    vp[base + i] = R(0);
    vc[base + i] = V[i];
    vn[base + i] = T > 1 ? V[n + i] : R(0);
  }
  R acc = R(0);
  for (int t = 0; t < T; ++t) {
    wsync();
    if (i < n) {
      const R* row = Blk + (((size_t)b * T + t) * n + i) * w3;
      R s = R(0);
      for (int k = 0; k < n; ++k) s += row[k] * vp[base + k];
      for (int k = 0; k < n; ++k) s += row[n + k] * vc[base + k];
      for (int k = 0; k < n; ++k) s += row[2 * n + k] * vn[base + k];
      if (G.live) out[((size_t)b * T + t) * n + i] = s;
      const R dvi = dv ? dv[((size_t)b * T + t) * n + i] : vc[base + i];
      acc += dvi * s;
    }
    wsync();
    if (i < n) {
      vp[base + i] = vc[base + i];
      vc[base + i] = vn[base + i];
      vn[base + i] = (t + 2 < T) ? V[(size_t)(t + 2) * n + i] : R(0);
    }
  }
  red[threadIdx.x] = (i < g) ? acc : R(0);
  wsync();
  R tot = R(0);
  for (int l = 0; l < g; ++l) tot += red[base + l];
  wsync();
  return tot;
}

// PCG on S x = gamma from x0 (x0 and x may alias).  Returns the iteration count.
template <typename R, int NC>
__device__ int pcg_device(const Dims& d, const Group& G, int g, R* sh3, R* red, const R* __restrict__ S,
                          const R* __restrict__ Phi, const R* gamma, const R* x0, const PcgVecs<R>& v,
                          R eps, int max_iter, bool commit) {
  const int n = NC > 0 ? NC : d.n;
  const int T = d.T;
  const int b = G.prob, i = G.lane;
  const size_t off = (size_t)b * T * n;
  // r = gamma - S x0 (q holds S x0); x = x0
  blk_matvec<R, NC>(d, G, g, sh3, red, S, x0, v.q, nullptr);
  if (i < n && G.live)
    for (int t = 0; t < T; ++t) {
      const size_t o = off + (size_t)t * n + i;
      v.r[o] = gamma[o] - v.q[o];
      v.x[o] = x0[o];
    }
  wsync();
  R eta = blk_matvec<R, NC>(d, G, g, sh3, red, Phi, v.r, v.rt, nullptr);
  if (i < n && G.live)
    for (int t = 0; t < T; ++t) v.p[off + (size_t)t * n + i] = v.rt[off + (size_t)t * n + i];
  wsync();
  const R eta0 = rabs(eta);
  const R abs_tol = R(1e-12);
  int it = 0;
  // the wave keeps iterating while any of its groups does; finished groups
  // stop committing (the reference's per-problem while_loop under vmap).
  // |eta_0| <= 1e-12 returns the warm start untouched (pcg_primal.py:158-174).
  bool running = commit && !(eta0 <= abs_tol);
  while (true) {
    bool cont = false;
    if (running) {
      const bool conv = rabs(eta) < abs_tol + eps * eta0;
      cont = (!conv && it <= max_iter - 1) || it < 1;
      if (!cont) running = false;
    }
    if (__ballot(cont && G.real) == 0) break;
    const R vv = blk_matvec<R, NC>(d, G, g, sh3, red, S, v.p, v.q, nullptr);
    const R al = eta / vv;
    if (i < n && G.live && cont)
      for (int t = 0; t < T; ++t) {
        const size_t o = off + (size_t)t * n + i;
        v.x[o] += al * v.p[o];
        v.r[o] -= al * v.q[o];
      }
    wsync();
    const R etap = blk_matvec<R, NC>(d, G, g, sh3, red, Phi, v.r, cont ? v.rt : v.q, nullptr);
    const R be = etap / eta;
    if (i < n && G.live && cont)
      for (int t = 0; t < T; ++t) {
        const size_t o = off + (size_t)t * n + i;
        v.p[o] = v.rt[o] + be * v.p[o];
      }
    wsync();
    if (cont) {
      eta = etap;
      ++it;
    }
  }
  return it;
}

template <typename R, int NC>
__global__ __launch_bounds__(kWave) void pcg_kernel(Dims d, int g, int P, const R* __restrict__ S,
                                                    const R* __restrict__ Phi, const R* __restrict__ rhs,
                                                    const R* __restrict__ x0, PcgVecs<R> v,
                                                    uint32_t* __restrict__ iters, R eps, int max_iter) {
  __shared__ R sh3[3 * kWave];
  __shared__ R red[kWave];
  const Group G = make_group(g, P, d.B);
  const int it = pcg_device<R, NC>(d, G, g, sh3, red, S, Phi, rhs, x0, v, eps, max_iter, G.real);
  if (G.live && G.lane == 0) iters[G.prob] = (uint32_t)it;
}

// ---------------------------------------------------- ADMM with PCG solve ----
template <typename R>
struct AdmmPcgArgs {
  AdmmArgs<R> a;       // shared fields (thinv/w unused)
  const R* S;
  const R* Phi;
  PcgVecs<R> v;        // v.x receives xt
  uint32_t* pcg_iters; // (B, max_iter) or null
  R pcg_eps;
  int pcg_max_iter;
};

// Everything of one ADMM iteration after the Schur solve, stage-parallel:
// C/G products of xt, relaxation, projection, duals and the next gamma.
template <typename R, int NC>
__device__ void admm_update_pass(const AdmmArgs<R>& a, const Group& G, Shared<R>& sh, const R* xt_all,
                                 R rho, bool commit) {
  const Dims& d = a.d;
  const int n = NC > 0 ? NC : d.n;
  const int T = d.T, N = d.N, nx = d.nx, n0 = d.n0, m = d.m, B = d.B;
  const int b = G.prob, i = G.lane, base = G.gid * a.g;
  const R alpha = a.alpha, oma = R(1) - a.alpha;
  const R rho_f = rho * a.rho_f_factor;
  const R gs = (a.use_slack && m > 0 && a.qp.slack_w) ? a.qp.slack_w[b] : R(0);
  R* xc = sh.v[SB_X] + base;
  R* xn = sh.v[SB_XN] + base;
  R* sc = sh.v[SB_C] + base;
  R* scp = sh.v[SB_CP] + base;
  R* sz = sh.v[SB_Z] + base;
  R* sc0 = sh.v[SB_C0] + base;
  const R* X = xt_all + (size_t)b * T * n;
  if (i < n) {
    xc[i] = X[i];
    xn[i] = X[n + i];
  }
  for (int t = 0; t < T; ++t) {
    wsync();
    R cx = R(0), cx0 = R(0), gx = R(0);
    if (t < N && i < nx)
      cx = row_dot<R, NC>(a.qp.Am + ((size_t)b * N + t) * nx * n, i, n, xc) +
           row_dot<R, NC>(a.qp.Ap + ((size_t)b * N + t) * nx * n, i, n, xn);
    if (t == 0 && i < n0) cx0 = row_dot<R, NC>(a.qp.A0 + (size_t)b * n0 * n, i, n, xc);
    if (i < m) gx = row_dot<R, NC>(a.qp.G + ((size_t)b * T + t) * m * n, i, n, xc);
    R xnew = R(0);
    if (i < n) {
      R* xp = a.st.x + ((size_t)b * T + t) * n + i;
      xnew = alpha * xc[i] + oma * (*xp);
      if (commit) *xp = xnew;
    }
    R zeta = R(0);
    if (i < m) {
      const size_t o = ((size_t)b * T + t) * m + i;
      const R zo = a.st.z[o], ygo = a.st.y_g[o];
      const R zt = alpha * gx + oma * zo + ygo / rho;
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
      const R ygn = ygo + rho * (alpha * gx + oma * zo - zn);
      if (commit) {
        a.st.z[o] = zn;
        a.st.xi[o] = xin;
        a.st.y_g[o] = ygn;
      }
      zeta = rho * zn - ygn;
    }
    R ct = R(0), ct0 = R(0);
    if (t < N && i < nx) {
      const size_t o = ((size_t)b * N + t) * nx + i;
      const R cv = a.qp.c[o];
      const R yf = a.st.y_f[o] + rho_f * (alpha * cx + oma * cv - cv);
      if (commit) a.st.y_f[o] = yf;
      ct = rho_f * cv - yf;
    }
    if (t == 0 && i < n0) {
      const size_t o = (size_t)b * n0 + i;
      const R cv = a.qp.c0[o];
      const R yf = a.st.y_f0[o] + rho_f * (alpha * cx0 + oma * cv - cv);
      if (commit) a.st.y_f0[o] = yf;
      ct0 = rho_f * cv - yf;
    }
    if (i < nx) sc[i] = ct;
    if (i < m) sz[i] = zeta;
    if (i < n0) sc0[i] = ct0;
    wsync();
    if (i < n) {
      R gv = a.sigma * xnew - a.qp.q[((size_t)b * T + t) * n + i];
      if (t < N) gv += col_dot(a.qp.Am + ((size_t)b * N + t) * nx * n, nx, n, i, sc);
      if (t > 0) gv += col_dot(a.qp.Ap + ((size_t)b * N + t - 1) * nx * n, nx, n, i, scp);
      if (m) gv += col_dot(a.qp.G + ((size_t)b * T + t) * m * n, m, n, i, sz);
      if (t == 0) gv += col_dot(a.qp.A0 + (size_t)b * n0 * n, n0, n, i, sc0);
      if (commit) a.gam[((size_t)t * B + b) * n + i] = gv;
    }
    wsync();
    if (i < nx) scp[i] = sc[i];
    if (i < n) {
      xc[i] = xn[i];
      xn[i] = (t + 2 < T) ? X[(size_t)(t + 2) * n + i] : R(0);
    }
  }
  wsync();
}

template <typename R, int NC>
__global__ __launch_bounds__(kWave) void admm_pcg_chunk_kernel(AdmmPcgArgs<R> pa) {
  __shared__ Shared<R> sh;
  __shared__ R sh3[3 * kWave];
  __shared__ R red[kWave];
  const AdmmArgs<R>& a = pa.a;
  const Dims d = a.d;
  const int n = NC > 0 ? NC : d.n;
  const int T = d.T, B = d.B;
  const Group G = make_group(a.g, a.P, B);
  const int b = G.prob, i = G.lane;
  int it;
  bool done;
  R res[6];
  if (a.first_chunk) {
    it = 0;
    done = false;
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
  for (int iter = a.it_lo; iter < a.it_hi; ++iter) {
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
    // gamma (stage-major) -> problem-major buffer w (sized T*B*n)
    if (i < n && G.live)
      for (int t = 0; t < T; ++t) a.w[((size_t)b * T + t) * n + i] = a.gam[((size_t)t * B + b) * n + i];
    wsync();
    const int pit = pcg_device<R, NC>(d, G, a.g, sh3, red, pa.S, pa.Phi, a.w, a.st.x, pa.v, pa.pcg_eps,
                                      pa.pcg_max_iter, active);
    if (pa.pcg_iters && G.live && i == 0 && active && iter < a.max_iter)
      pa.pcg_iters[(size_t)b * a.max_iter + iter] = (uint32_t)pit;
    admm_update_pass<R, NC>(a, G, sh, pa.v.x, rho, commit);
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

}  // namespace tmpc
