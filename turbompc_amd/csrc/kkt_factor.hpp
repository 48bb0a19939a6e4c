// Rows-in-lanes factorization and solves of the stage-block adjoint KKT
// matrix, reading the QP's own blocks (no assembled matrix).
//
// Block row t of the KKT matrix (adjoint.hpp) is [phi_{t-1} | theta_t | phi_t^T]
// with nb = n + p + m unknowns per stage (z_t, the equality multipliers, the
// inequality multipliers):
//   theta_t   = [[D_t + sI, Chat_t^T, G_t^T], [Chat_t, -sI, 0], [G_t, 0, -sI]]
//   phi_{t-1} = K_{t,t-1} = [[E_{t-1}, 0], [A_minus_{t-1}, 0], [0, 0]]
// with Chat_0 = A0, Chat_t = A_plus_{t-1}, and -1 in place of -s on padding
// rows (multiplier rows past n0 or nx, zero G rows), which decouples them.  A
// lane that computes row i of a stage loads row i of these blocks from the QP
// arrays directly (the z rows take the columns of Chat and G).  The coupling
// block has its nonzeros in its first n columns (the z_{t-1} unknowns).  The
// recursion is factor_kernel's (factor.hpp, SRC_S),
//   Theta_t = theta_t - phi_{t-1} Theta_{t-1}^{-1} phi_{t-1}^T,
// and with those n columns the Schur term only needs Z = Theta_{t-1}^{-1}[0:n, 0:n]:
//   (phi Theta^{-1} phi^T)[i][j] = (phi_i Z) . phi_j,   phi_i = phi_{t-1}[i][0:n].
// The stage blocks are quasi-definite (shifted primal block first), so
// Gauss-Jordan without pivoting in the natural order factors them stably.
//
// Layout: a problem's group of NBC >= nb lanes holds row i of the stage block
// in lane i (rows nb..NBC-1 are unit rows, decoupled and never stored); P
// problems per wavefront.  Pivot rows, phi's rows and Z move through LDS; the
// workgroup is one wavefront, whose LDS instructions execute in issue order.
// Each kernel issues the next stage's loads before it works on the current
// one.  fp64 arithmetic; the symmetric part of each Theta_t^{-1} is stored
// packed, rounded to the storage type, where factor_kernel stores it.
#pragma once
#include "adjoint.hpp"
#include "common.hpp"

namespace tmpc {

// Row ir of theta_t as the QP blocks hold it, without the diagonal terms
// (zero for a unit row, ir >= nb).
template <typename R, int NBC>
__device__ __forceinline__ void kkt_theta_row(const KktDims& k, const QPDev<R>& qp, int b, int t, int ir,
                                              R (&v)[NBC]) {
  const int n = k.n, p = k.p, nb = k.nb;
  const int nlam = t == 0 ? k.n0 : k.nx;
  const R* Dt = qp.D + ((size_t)b * k.T + t) * n * n;
  const R* Ch = t == 0 ? qp.A0 + (size_t)b * k.n0 * n : qp.Ap + ((size_t)b * k.N + t - 1) * k.nx * n;
  const R* Gt = k.m ? qp.G + ((size_t)b * k.T + t) * k.m * n : Dt;  // Dt: never read when m = 0
  const bool z = ir < n, lam = !z && ir < n + p, mu = ir >= n + p && ir < nb;
  const int r = lam ? ir - n : ir - n - p;
  const bool rok = z || (lam && r < nlam) || mu;
  const R* rowp = z ? Dt + ir * n : (lam ? Ch + r * n : Gt + r * n);
#pragma unroll
  for (int j = 0; j < NBC; ++j) {
    R x = R(0);
    if (j < n) {
      if (rok) x = rowp[j];
    } else if (j < n + p) {
      if (z && j - n < nlam) x = Ch[(j - n) * n + ir];
    } else if (j < nb) {
      if (z) x = Gt[(j - n - p) * n + ir];
    }
    v[j] = x;
  }
}

// The diagonal of row ir of theta_t on top of kkt_theta_row's values:
// +shift on z rows, -shift on multiplier rows (shift = 0: the unshifted
// matrix), -1 on padding rows, 1 on unit rows.
template <typename C, int NBC>
__device__ __forceinline__ void kkt_theta_diag(const KktDims& k, int t, int ir, C shift, C (&a)[NBC]) {
  const int n = k.n, p = k.p, nb = k.nb;
  const bool z = ir < n, lam = !z && ir < n + p, mu = ir >= n + p && ir < nb;
  C nrm = C(0);
#pragma unroll
  for (int j = 0; j < NBC; ++j) nrm += j < n ? fabs(a[j]) : C(0);
  const bool pad = (lam && ir - n >= (t == 0 ? k.n0 : k.nx)) || (mu && !(nrm > C(0)));
  const C other = ir >= nb ? C(1) : (pad ? C(-1) : -shift);
#pragma unroll
  for (int j = 0; j < NBC; ++j)
    if (j == ir) a[j] = z ? a[j] + shift : other;
}

// Row ir of phi_{t-1}, its first n columns (zero at t = 0): E_{t-1} on the z
// rows, A_minus_{t-1} on the first nx multiplier rows.
template <typename R, int NC>
__device__ __forceinline__ void kkt_phi_row(const KktDims& k, const QPDev<R>& qp, int b, int t, int ir,
                                            R (&f)[NC]) {
  const int n = k.n;
  const bool z = ir < n, ok = t > 0 && (z || ir < n + k.nx);
  const size_t s = (size_t)b * k.N + (t > 0 ? t - 1 : 0);
  const R* rp = z ? qp.E + s * n * n + ir * n : qp.Am + s * k.nx * n + (ir - n) * n;
#pragma unroll
  for (int c = 0; c < NC; ++c) f[c] = (ok && c < n) ? rp[c] : R(0);
}

// Column ic (< n) of phi_t (t < T - 1; ok false gives zeros): E_t[j][ic] for
// j < n, A_minus_t[j - n][ic] for n <= j < n + nx.
template <typename R, int NBC>
__device__ __forceinline__ void kkt_phi_col(const KktDims& k, const QPDev<R>& qp, int b, int t, int ic, bool ok,
                                            R (&g)[NBC]) {
  const int n = k.n, nx = k.nx;
  const size_t s = (size_t)b * k.N + (ok ? t : 0);
  const R* Ec = qp.E + s * n * n + ic;
  const R* Ac = qp.Am + s * nx * n + ic;
#pragma unroll
  for (int j = 0; j < NBC; ++j) g[j] = !ok ? R(0) : (j < n ? Ec[j * n] : (j < n + nx ? Ac[(j - n) * n] : R(0)));
}


// NC >= n, NBC >= nb, P problems per wavefront (groups at a stride of 64 / P lanes).
template <typename R, int NC, int NBC, int P>
__global__ __launch_bounds__(kWave) void factor_kkt_rows_kernel(KktDims k, QPDev<R> qp,
                                                                const R* __restrict__ shift,
                                                                R* __restrict__ thinv) {
  static_assert(NBC * P <= kWave, "a problem's rows must fit its group");
  using C = double;
  const int nb = k.nb, n = k.n, T = k.T, B = k.B, pk = th_pitch(nb);
  const Group G = make_group_strided(NBC, P, B);
  const int b = G.prob, i = G.lane, p = G.gid;
  const int ir = min(i, NBC - 1);     // the group row this lane computes (idle lanes repeat the last)
  const bool row = ir < nb;           // a row of the block (else a unit row)
  __shared__ C Zs[P][NC][NC];          // Theta_{t-1}^{-1}[0:n, 0:n]
  __shared__ C Ph[P][NBC][NC];         // phi_{t-1}[:, 0:n]
  __shared__ C Pv[P][2][NBC];          // pivot rows
  __shared__ C Sy[P][NBC][NBC + 1];    // the inverse, for its symmetric part
  const bool wr = i < NBC;             // lanes that write the group's LDS rows
  const C sh = (C)shift[b];

  // the next stage's loads wait in registers while a stage is factored where
  // they fit (NBC <= 18; the larger blocks would spill)
  constexpr bool PF = NBC <= 18;
  R va[NBC], vf[NC];
  if constexpr (PF) {
    kkt_theta_row(k, qp, b, 0, ir, va);
    kkt_phi_row(k, qp, b, 0, ir, vf);  // zeros
  }
  C a[NBC];
  for (int t = 0; t < T; ++t) {
    // theta_t row i (rows past nb: unit rows) and phi_{t-1} row i, its first
    // n columns
    if constexpr (!PF) {
      kkt_theta_row(k, qp, b, t, ir, va);
      kkt_phi_row(k, qp, b, t, ir, vf);
    }
#pragma unroll
    for (int j = 0; j < NBC; ++j) a[j] = (C)va[j];
    C f[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) f[c] = (C)vf[c];
    if (PF && t + 1 < T) {
      kkt_theta_row(k, qp, b, t + 1, ir, va);
      kkt_phi_row(k, qp, b, t + 1, ir, vf);
    }
    kkt_theta_diag(k, t, ir, sh, a);
    if (t > 0) {
      if (wr)
#pragma unroll
        for (int c = 0; c < NC; ++c) Ph[p][i][c] = f[c];
      lds_order();
      // u = phi_i Z
      C u[NC];
#pragma unroll
      for (int l = 0; l < NC; ++l) u[l] = C(0);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        C z[NC];
#pragma unroll
        for (int l = 0; l < NC; ++l) z[l] = Zs[p][c][l];
#pragma unroll
        for (int l = 0; l < NC; ++l) u[l] += f[c] * z[l];
      }
      // a[j] -= u . phi_j
#pragma unroll
      for (int j = 0; j < NBC; ++j) {
        C q[NC];
#pragma unroll
        for (int l = 0; l < NC; ++l) q[l] = Ph[p][j][l];
        C s = C(0);
#pragma unroll
        for (int l = 0; l < NC; ++l) s += u[l] * q[l];
        a[j] -= s;
      }
    }
    // Gauss-Jordan, two pivots per LDS round trip: rows k and k+1 are
    // broadcast together and every lane replays the two single-pivot steps,
    // forming row k+1 after step k itself.  A pivot row is not normalized at
    // its step (its lane keeps 1/pivot and scales at the end), so every lane
    // runs the same instructions.
    C myip = C(1);
#pragma unroll
    for (int kp = 0; kp < NBC; kp += 2) {
      const bool pair = kp + 1 < NBC;
      lds_order();
      if (wr && (ir == kp || (pair && ir == kp + 1)))
#pragma unroll
        for (int j = 0; j < NBC; ++j) Pv[p][ir - kp][j] = a[j];
      lds_order();
      C p1[NBC], p2[NBC];
#pragma unroll
      for (int j = 0; j < NBC; ++j) {
        p1[j] = Pv[p][0][j];
        p2[j] = pair ? Pv[p][1][j] : C(0);
      }
      const bool m0 = ir == kp, m1 = pair && ir == kp + 1;
      const C ip = C(1) / p1[kp];
      myip = m0 ? ip : myip;
      const C g = m0 ? C(0) : a[kp] * ip;
#pragma unroll
      for (int j = 0; j < NBC; ++j) a[j] = (j == kp) ? (m0 ? C(1) : -g) : a[j] - g * p1[j];
      if (pair) {
        const C gq = p2[kp] * ip;
#pragma unroll
        for (int j = 0; j < NBC; ++j) p2[j] = (j == kp) ? -gq : p2[j] - gq * p1[j];
        const C ip2 = C(1) / p2[kp + 1];
        myip = m1 ? ip2 : myip;
        const C g2 = m1 ? C(0) : a[kp + 1] * ip2;
#pragma unroll
        for (int j = 0; j < NBC; ++j) a[j] = (j == kp + 1) ? (m1 ? C(1) : -g2) : a[j] - g2 * p2[j];
      }
    }
#pragma unroll
    for (int j = 0; j < NBC; ++j) a[j] *= myip;
    // symmetric part (row i averaged with column i), as factor_kernel keeps
    lds_order();
    if (wr)
#pragma unroll
      for (int j = 0; j < NBC; ++j) Sy[p][i][j] = a[j];
    lds_order();
#pragma unroll
    for (int j = 0; j < NBC; ++j) a[j] = C(0.5) * (a[j] + Sy[p][j][ir]);
    if (G.live && row) {
      R* out = thinv + ((size_t)t * B + b) * pk + ((ir * (ir + 1)) >> 1);
#pragma unroll
      for (int j = 0; j < NBC; ++j)
        if (j <= ir) out[j] = (R)a[j];
    }
    // Z for the next stage
    lds_order();
    if (wr && ir < NC)
#pragma unroll
      for (int l = 0; l < NC; ++l) Zs[p][ir][l] = (ir < n && l < n) ? a[l] : C(0);
    lds_order();
  }
}

// x = K^{-1} rhs from the factor above (the coupling blocks read from the QP,
// their first n columns only): the forward sweep
//   w_t = Theta_t^{-1} (rhs_t - phi_{t-1} w_{t-1}),  phi_{t-1} w_{t-1} = phi_{t-1}[:, 0:n] w_{t-1}[0:n],
// then the backward sweep
//   x_t = w_t - Theta_t^{-1} phi_t^T x_{t+1},  (phi_t^T x_{t+1}) nonzero in its first n entries,
// as blktri_solve_kernel computes it, with the same lane layout as the
// factorization (row i of a stage in lane i, P problems per wavefront); the
// loads of stage t +- 1 are in flight while stage t is solved.  Vectors move
// through LDS.  rhs null: the KKT system's own right-hand side [-q_t | 0 | 0].
template <typename R, int NC, int NBC, int P>
__global__ __launch_bounds__(kWave) void kkt_solve_rows_kernel(KktDims k, QPDev<R> qp,
                                                               const R* __restrict__ thinv,
                                                               const R* __restrict__ rhs, R* __restrict__ x) {
  static_assert(NBC * P <= kWave, "a problem's rows must fit its group");
  const int nb = k.nb, n = k.n, T = k.T, B = k.B, pk = th_pitch(nb);
  const Group G = make_group_strided(NBC, P, B);
  const int b = G.prob, i = G.lane, p = G.gid;
  const int ir = min(i, NBC - 1);
  const bool row = ir < nb;
  const int ic = row ? ir : 0;
  const int icn = min(ir, NC - 1);  // a column < n of the coupling block
  const bool wr = i < NBC;
  __shared__ R sv[P][2][NBC];
  R* X = x + (size_t)b * T * nb;
  // Theta_t^{-1} row i (packed symmetric; zero past nb)
  auto th_row = [&](int t, R (&h)[NBC]) {
    const R* Th = thinv + ((size_t)t * B + b) * pk;
    const int ri = (ic * (ic + 1)) >> 1;
#pragma unroll
    for (int c = 0; c < NBC; ++c) h[c] = (row && c < nb) ? Th[c <= ic ? ri + c : ((c * (c + 1)) >> 1) + ic] : R(0);
  };
  auto rhs_at = [&](int t) -> R {
    if (rhs) return row ? rhs[((size_t)b * T + t) * nb + ic] : R(0);
    return ir < n ? -qp.q[((size_t)b * T + t) * n + ir] : R(0);
  };
  // forward sweep
  R h[NBC], f[NC], rr;
  th_row(0, h);
  kkt_phi_row(k, qp, b, 0, ir, f);  // zeros
  rr = rhs_at(0);
  R wprev = R(0);  // w_{t-1}[i]
  for (int t = 0; t < T; ++t) {
    R hc[NBC], fc[NC];
#pragma unroll
    for (int c = 0; c < NBC; ++c) hc[c] = h[c];
#pragma unroll
    for (int c = 0; c < NC; ++c) fc[c] = f[c];
    R r = rr;
    if (t + 1 < T) {
      th_row(t + 1, h);
      kkt_phi_row(k, qp, b, t + 1, ir, f);
      rr = rhs_at(t + 1);
    }
    lds_order();
    if (wr) sv[p][0][i] = wprev;  // w_{t-1}
    lds_order();
    R s = R(0);
#pragma unroll
    for (int c = 0; c < NC; ++c) s += fc[c] * sv[p][0][c];
    r -= s;
    lds_order();
    if (wr) sv[p][1][i] = r;
    lds_order();
    R wv = R(0);
#pragma unroll
    for (int c = 0; c < NBC; ++c) wv += hc[c] * sv[p][1][c];
    if (G.live && row) X[(size_t)t * nb + ic] = wv;
    wprev = row ? wv : R(0);
  }
  // backward sweep: x_{T-1} = w_{T-1}; lane i keeps x_t[i]
  R xn = wprev;
  R g[NBC], wn = R(0);
  if (T >= 2) {
    th_row(T - 2, h);
    kkt_phi_col(k, qp, b, T - 2, icn, ir < n, g);  // column icn of phi_{T-2}
    wn = row ? X[(size_t)(T - 2) * nb + ic] : R(0);
  }
  for (int t = T - 2; t >= 0; --t) {
    R hc[NBC], gc[NBC];
#pragma unroll
    for (int c = 0; c < NBC; ++c) hc[c] = h[c];
#pragma unroll
    for (int j = 0; j < NBC; ++j) gc[j] = g[j];
    const R wt = wn;
    if (t >= 1) {
      th_row(t - 1, h);
      kkt_phi_col(k, qp, b, t - 1, icn, ir < n, g);
      wn = row ? X[(size_t)(t - 1) * nb + ic] : R(0);
    }
    lds_order();
    if (wr) sv[p][0][i] = xn;  // x_{t+1}
    lds_order();
    R q = R(0);
#pragma unroll
    for (int j = 0; j < NBC; ++j) q += gc[j] * sv[p][0][j];
    lds_order();
    if (wr) sv[p][1][i] = ir < n ? q : R(0);  // (phi_t^T x_{t+1})[i], zero past n
    lds_order();
    R d = R(0);
#pragma unroll
    for (int c = 0; c < NC; ++c) d += hc[c] * sv[p][1][c];
    const R xt = wt - d;
    if (G.live && row) X[(size_t)t * nb + ic] = xt;
    xn = row ? xt : R(0);
  }
}

// r = rhs - K x with the unshifted matrix (-1 on padding rows, as in the
// shifted one) and the KKT system's own right-hand side [-q_t | 0 | 0], as
// kkt_residual_kernel computes it.  A stage's residual needs only x_{t-1},
// x_t and x_{t+1}, so every (problem, stage) is an independent unit: P units
// per wavefront, row i of a unit's block row in lane i of its group (the
// sub-diagonal block's nonzeros in columns < n, the super-diagonal block
// phi_t^T's in rows < n), the three x blocks through LDS.
template <typename R, int NC, int NBC, int P>
__global__ __launch_bounds__(kWave) void kkt_residual_rows_kernel(KktDims k, QPDev<R> qp,
                                                                  const R* __restrict__ x, R* __restrict__ r) {
  static_assert(NBC * P <= kWave, "a unit's rows must fit its group");
  const int nb = k.nb, n = k.n, T = k.T;
  const Group G = make_group_strided(NBC, P, k.B * T);  // groups over (problem, stage) units
  const int b = G.prob / T, t = G.prob - b * T, i = G.lane, p = G.gid;
  const int ir = min(i, NBC - 1);
  const bool row = ir < nb;
  const int ic = row ? ir : 0;
  const int icn = min(ir, NC - 1);
  __shared__ R xw[P][3][NBC];  // x_{t-1}, x_t, x_{t+1}
  const size_t o = ((size_t)b * T + t) * nb;
  R sub[NC], dia[NBC], sup[NBC];
  kkt_phi_row(k, qp, b, t, ir, sub);
  kkt_theta_row(k, qp, b, t, ir, dia);
  kkt_phi_col(k, qp, b, t, icn, ir < n && t + 1 < T, sup);  // row ir of phi_t^T
  const R qn = ir < n ? qp.q[((size_t)b * T + t) * n + ir] : R(0);
  if (i < NBC) {
    xw[p][0][i] = (row && t > 0) ? x[o - nb + ic] : R(0);
    xw[p][1][i] = row ? x[o + ic] : R(0);
    xw[p][2][i] = (row && t + 1 < T) ? x[o + nb + ic] : R(0);
  }
  kkt_theta_diag(k, t, ir, R(0), dia);
  lds_order();
  R s = R(0);
#pragma unroll
  for (int c = 0; c < NC; ++c) s += sub[c] * xw[p][0][c];
#pragma unroll
  for (int c = 0; c < NBC; ++c) s += dia[c] * xw[p][1][c];
#pragma unroll
  for (int c = 0; c < NBC; ++c) s += sup[c] * xw[p][2][c];
  if (G.live && row) r[o + ic] = -qn - s;
}

}  // namespace tmpc
