// Rows-in-lanes factorization of the stage-block adjoint KKT matrix.
//
// The blocks are those of kkt_assemble_kernel (adjoint.hpp): block row t holds
// [phi_{t-1} | theta_t | phi_t^T] with nb = n + p + m unknowns per stage
// (z_t, the equality multipliers, the inequality multipliers), and the
// coupling block phi_{t-1} = K_{t,t-1} = [[E_{t-1}, 0], [A_minus_{t-1}, 0], [0, 0]]
// has its nonzeros in the first n columns (the z_{t-1} unknowns).  The
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
// fp64 arithmetic; the symmetric part of each Theta_t^{-1} is stored packed,
// rounded to the storage type, where factor_kernel stores it.
#pragma once
#include "adjoint.hpp"
#include "common.hpp"

namespace tmpc {

// NC >= n, NBC >= nb, P problems per wavefront (groups at a stride of 64 / P lanes).
template <typename R, int NC, int NBC, int P>
__global__ __launch_bounds__(kWave) void factor_kkt_rows_kernel(KktDims k, const R* __restrict__ K,
                                                                R* __restrict__ thinv) {
  static_assert(NBC * P <= kWave, "a problem's rows must fit its group");
  using C = double;
  const int nb = k.nb, n = k.n, T = k.T, B = k.B, w3 = 3 * nb, pk = th_pitch(nb);
  const Group G = make_group_strided(NBC, P, B);
  const int b = G.prob, i = G.lane, p = G.gid;
  const int ir = min(i, NBC - 1);     // the group row this lane computes (idle lanes repeat the last)
  const bool row = ir < nb;           // a row of the block (else a unit row)
  const int ic = row ? ir : 0;        // clamped row for loads
  __shared__ C Zs[P][NC][NC];          // Theta_{t-1}^{-1}[0:n, 0:n]
  __shared__ C Ph[P][NBC][NC];         // phi_{t-1}[:, 0:n]
  __shared__ C Pv[P][2][NBC];          // pivot rows
  __shared__ C Sy[P][NBC][NBC + 1];    // the inverse, for its symmetric part
  const bool wr = i < NBC;             // lanes that write the group's LDS rows

  C a[NBC];
  for (int t = 0; t < T; ++t) {
    const R* Kr = K + (((size_t)b * T + t) * nb + ic) * w3;
    // theta_t row i (rows past nb: unit rows)
#pragma unroll
    for (int j = 0; j < NBC; ++j) a[j] = (row && j < nb) ? (C)Kr[nb + j] : (j == ir ? C(1) : C(0));
    if (t > 0) {
      // phi_{t-1} row i, its first n columns
      C f[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) f[c] = (row && c < n) ? (C)Kr[c] : C(0);
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

// x = K^{-1} rhs from the factor above (K's coupling blocks read from the
// S-form blocks, their first n columns only): the forward sweep
//   w_t = Theta_t^{-1} (rhs_t - phi_{t-1} w_{t-1}),  phi_{t-1} w_{t-1} = phi_{t-1}[:, 0:n] w_{t-1}[0:n],
// then the backward sweep
//   x_t = w_t - Theta_t^{-1} phi_t^T x_{t+1},  (phi_t^T x_{t+1}) nonzero in its first n entries,
// as blktri_solve_kernel computes it, with the same lane layout as the
// factorization (row i of a stage in lane i, P problems per wavefront) and
// every load of a stage issued at once.  Vectors move through LDS.
template <typename R, int NC, int NBC, int P>
__global__ __launch_bounds__(kWave) void kkt_solve_rows_kernel(KktDims k, const R* __restrict__ K,
                                                               const R* __restrict__ thinv,
                                                               const R* __restrict__ rhs, R* __restrict__ x) {
  static_assert(NBC * P <= kWave, "a problem's rows must fit its group");
  const int nb = k.nb, n = k.n, T = k.T, B = k.B, w3 = 3 * nb, pk = th_pitch(nb);
  const Group G = make_group_strided(NBC, P, B);
  const int b = G.prob, i = G.lane, p = G.gid;
  const int ir = min(i, NBC - 1);
  const bool row = ir < nb;
  const int ic = row ? ir : 0;
  const int icn = min(ir, NC - 1);  // a column < n of the coupling block
  const bool wr = i < NBC;
  __shared__ R sv[P][2][NBC];
  R* X = x + (size_t)b * T * nb;
  const R* Rh = rhs + (size_t)b * T * nb;
  // Theta_t^{-1} row i (packed symmetric; zero past nb)
  auto th_row = [&](int t, R (&h)[NBC]) {
    const R* Th = thinv + ((size_t)t * B + b) * pk;
    const int ri = (ic * (ic + 1)) >> 1;
#pragma unroll
    for (int c = 0; c < NBC; ++c) h[c] = (row && c < nb) ? Th[c <= ic ? ri + c : ((c * (c + 1)) >> 1) + ic] : R(0);
  };
  // forward sweep
  R wprev = R(0);  // w_{t-1}[i]
  for (int t = 0; t < T; ++t) {
    R h[NBC], f[NC];
    th_row(t, h);
    const R* Kr = K + (((size_t)b * T + t) * nb + ic) * w3;
#pragma unroll
    for (int c = 0; c < NC; ++c) f[c] = (t > 0 && row && c < n) ? Kr[c] : R(0);
    R r = row ? Rh[(size_t)t * nb + ic] : R(0);
    lds_order();
    if (wr) sv[p][0][i] = wprev;  // w_{t-1}
    lds_order();
    R s = R(0);
#pragma unroll
    for (int c = 0; c < NC; ++c) s += f[c] * sv[p][0][c];
    r -= s;
    lds_order();
    if (wr) sv[p][1][i] = r;
    lds_order();
    R wv = R(0);
#pragma unroll
    for (int c = 0; c < NBC; ++c) wv += h[c] * sv[p][1][c];
    if (G.live && row) X[(size_t)t * nb + ic] = wv;
    wprev = row ? wv : R(0);
  }
  // backward sweep: x_{T-1} = w_{T-1}; lane i keeps x_t[i]
  R xn = wprev;
  for (int t = T - 2; t >= 0; --t) {
    R h[NBC], g[NBC];
    th_row(t, h);
    // column icn (< n) of phi_t = the coupling block of block row t + 1
    const R* Kn = K + ((size_t)b * T + t + 1) * nb * w3;
#pragma unroll
    for (int j = 0; j < NBC; ++j) g[j] = (j < nb) ? Kn[(size_t)j * w3 + icn] : R(0);
    const R wt = row ? X[(size_t)t * nb + ic] : R(0);
    lds_order();
    if (wr) sv[p][0][i] = xn;  // x_{t+1}
    lds_order();
    R q = R(0);
#pragma unroll
    for (int j = 0; j < NBC; ++j) q += g[j] * sv[p][0][j];
    lds_order();
    if (wr) sv[p][1][i] = ir < n ? q : R(0);  // (phi_t^T x_{t+1})[i], zero past n
    lds_order();
    R d = R(0);
#pragma unroll
    for (int c = 0; c < NC; ++c) d += h[c] * sv[p][1][c];
    const R xt = wt - d;
    if (G.live && row) X[(size_t)t * nb + ic] = xt;
    xn = row ? xt : R(0);
  }
}

}  // namespace tmpc
