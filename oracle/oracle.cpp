// TEST INFRASTRUCTURE ONLY — CPU oracle (see oracle.h for the contract).
//
// A plain restatement of the reference's pure-JAX solver path, one problem per
// OpenMP iteration.  Every function names the reference lines it follows.
// Reference paths are relative to the TurboMPC repository root.
//
// Parity pins (tests/test_oracle_*.py):
//   schur_build      closed form S = P + sigma I + rho_f C^T C + rho G^T G and the
//                    Phiinv block formula, checked against dense numpy assembly.
//   blktri_solve     dense numpy.linalg.solve on the assembled S.
//   pcg              converges to the dense solve; stops after exactly r + 1
//                    iterations when M^{-1} S has r + 1 distinct eigenvalues;
//                    every fixed-count iterate is the Galerkin solution on its
//                    Krylov space (tests/test_oracle_pcg_pins.py).
//   admm_solve       (a) one iteration against a hand-assembled dense
//                    restatement in numpy; (b) at convergence: primal
//                    feasibility, stationarity, complementarity; (c) brute-force
//                    active-set enumeration on tiny QPs; (d) max_iter/check
//                    oracle (re-running to the stopping iteration reproduces it).
//   adjoint_kkt      numpy dense solve of the KKT; central finite differences of
//                    the converged forward QP solution.
//   quadrotor_rk4_jac  central finite differences and the analytic hover trim.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <complex>
#include <cstring>
#include <limits>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

template <typename R>
using Vec = std::vector<R>;

// ---------------------------------------------------------------- dims ----
struct Dims {
  int B, T, N, n, nx, n0, m;
  explicit Dims(const ora_dims& d)
      : B(d.B), T(d.T), N(d.T - 1), n(d.n), nx(d.nx), n0(d.n0), m(d.m) {}
};

template <typename R>
struct QP {  // one problem's view
  const R *D, *E, *q, *A0, *Am, *Ap, *G, *l, *u, *c0, *c;
  R slack_w;
  bool use_slack;
};

template <typename R>
QP<R> qp_view(const ora_qp& qp, const Dims& d, int b) {
  QP<R> v;
  const int T = d.T, N = d.N, n = d.n, nx = d.nx, n0 = d.n0, m = d.m;
  v.D = static_cast<const R*>(qp.D) + (size_t)b * T * n * n;
  v.E = static_cast<const R*>(qp.E) + (size_t)b * N * n * n;
  v.q = static_cast<const R*>(qp.q) + (size_t)b * T * n;
  v.A0 = static_cast<const R*>(qp.A0) + (size_t)b * n0 * n;
  v.Am = static_cast<const R*>(qp.A_minus) + (size_t)b * N * nx * n;
  v.Ap = static_cast<const R*>(qp.A_plus) + (size_t)b * N * nx * n;
  v.G = m ? static_cast<const R*>(qp.G) + (size_t)b * T * m * n : nullptr;
  v.l = m ? static_cast<const R*>(qp.l) + (size_t)b * T * m : nullptr;
  v.u = m ? static_cast<const R*>(qp.u) + (size_t)b * T * m : nullptr;
  v.c0 = static_cast<const R*>(qp.c0) + (size_t)b * n0;
  v.c = static_cast<const R*>(qp.c) + (size_t)b * N * nx;
  v.slack_w = (R)qp.slack_weight;
  v.use_slack = qp.use_slack != 0;
  return v;
}

// ------------------------------------------------------- state (local) ----
template <typename R>
struct State {
  Vec<R> x, z, y_g, y_f0, y_f, xi;
  R rho;
  explicit State(const Dims& d)
      : x(d.T * d.n), z(d.T * d.m), y_g(d.T * d.m), y_f0(d.n0), y_f(d.N * d.nx),
        xi(d.T * d.m), rho(0) {}
};

template <typename R>
void load_state(State<R>& s, const ora_state& st, const Dims& d, int b) {
  auto cp = [](Vec<R>& dst, const void* src, size_t off) {
    if (!dst.empty())
      std::memcpy(dst.data(), static_cast<const R*>(src) + off * dst.size(),
                  dst.size() * sizeof(R));
  };
  cp(s.x, st.x, b);
  cp(s.z, st.z_g, b);
  cp(s.y_g, st.y_g, b);
  cp(s.y_f0, st.y_f0, b);
  cp(s.y_f, st.y_f, b);
  cp(s.xi, st.xi_g, b);
  s.rho = static_cast<const R*>(st.rho)[b];
}

template <typename R>
void store_state(const State<R>& s, ora_state& st, const Dims& d, int b) {
  auto cp = [](const Vec<R>& src, void* dst, size_t off) {
    if (!src.empty())
      std::memcpy(static_cast<R*>(dst) + off * src.size(), src.data(),
                  src.size() * sizeof(R));
  };
  cp(s.x, st.x, b);
  cp(s.z, st.z_g, b);
  cp(s.y_g, st.y_g, b);
  cp(s.y_f0, st.y_f0, b);
  cp(s.y_f, st.y_f, b);
  cp(s.xi, st.xi_g, b);
  static_cast<R*>(st.rho)[b] = s.rho;
}

// --------------------------------------------------- small dense algebra ----
// y[r] (+)= sum_k A[r*lda + k] * x[k]
template <typename R>
void matvec(const R* A, int rows, int cols, const R* x, R* y, bool accumulate) {
  for (int r = 0; r < rows; ++r) {
    R s = 0;
    for (int k = 0; k < cols; ++k) s += A[r * cols + k] * x[k];
    y[r] = accumulate ? y[r] + s : s;
  }
}
// y[c] (+)= sum_r A[r*cols + c] * x[r]
template <typename R>
void matTvec(const R* A, int rows, int cols, const R* x, R* y, bool accumulate) {
  for (int c = 0; c < cols; ++c) {
    R s = 0;
    for (int r = 0; r < rows; ++r) s += A[r * cols + c] * x[r];
    y[c] = accumulate ? y[c] + s : s;
  }
}

// LU with partial pivoting (row-major, in place), the textbook algorithm
// (Golub & Van Loan, Alg. 3.4.1).  Returns false on an exact zero pivot.
template <typename R>
bool lu_factor(R* A, int n, int* piv) {
  for (int k = 0; k < n; ++k) {
    int p = k;
    R best = std::abs(A[k * n + k]);
    for (int i = k + 1; i < n; ++i) {
      R v = std::abs(A[i * n + k]);
      if (v > best) { best = v; p = i; }
    }
    piv[k] = p;
    if (best == R(0)) return false;
    if (p != k)
      for (int j = 0; j < n; ++j) std::swap(A[k * n + j], A[p * n + j]);
    const R inv = R(1) / A[k * n + k];
    for (int i = k + 1; i < n; ++i) {
      R f = A[i * n + k] * inv;
      A[i * n + k] = f;
      if (f != R(0))
        for (int j = k + 1; j < n; ++j) A[i * n + j] -= f * A[k * n + j];
    }
  }
  return true;
}
template <typename R>
void lu_solve(const R* LU, int n, const int* piv, R* b) {
  for (int k = 0; k < n; ++k)
    if (piv[k] != k) std::swap(b[k], b[piv[k]]);
  for (int i = 0; i < n; ++i) {
    R s = b[i];
    for (int j = 0; j < i; ++j) s -= LU[i * n + j] * b[j];
    b[i] = s;
  }
  for (int i = n - 1; i >= 0; --i) {
    R s = b[i];
    for (int j = i + 1; j < n; ++j) s -= LU[i * n + j] * b[j];
    b[i] = s / LU[i * n + i];
  }
}
// inverse through LU (what jnp.linalg.inv does: solve(A, I)).
template <typename R>
void inverse(const R* A, int n, R* Ainv) {
  Vec<R> LU(A, A + n * n);
  std::vector<int> piv(n);
  lu_factor(LU.data(), n, piv.data());
  Vec<R> col(n);
  for (int j = 0; j < n; ++j) {
    std::fill(col.begin(), col.end(), R(0));
    col[j] = R(1);
    lu_solve(LU.data(), n, piv.data(), col.data());
    for (int i = 0; i < n; ++i) Ainv[i * n + j] = col[i];
  }
}

// Cholesky A = L L^T (lower, row-major, in place; upper part zeroed).
template <typename R>
void cholesky(R* A, int n) {
  for (int j = 0; j < n; ++j) {
    R s = A[j * n + j];
    for (int k = 0; k < j; ++k) s -= A[j * n + k] * A[j * n + k];
    const R d = std::sqrt(s);
    A[j * n + j] = d;
    for (int i = j + 1; i < n; ++i) {
      R t = A[i * n + j];
      for (int k = 0; k < j; ++k) t -= A[i * n + k] * A[j * n + k];
      A[i * n + j] = t / d;
    }
    for (int k = j + 1; k < n; ++k) A[j * n + k] = R(0);
  }
}
// solve L y = b (in place)
template <typename R>
void trsv_lower(const R* L, int n, R* b) {
  for (int i = 0; i < n; ++i) {
    R s = b[i];
    for (int k = 0; k < i; ++k) s -= L[i * n + k] * b[k];
    b[i] = s / L[i * n + i];
  }
}
// solve L^T x = b (in place)
template <typename R>
void trsv_lower_T(const R* L, int n, R* b) {
  for (int i = n - 1; i >= 0; --i) {
    R s = b[i];
    for (int k = i + 1; k < n; ++k) s -= L[k * n + i] * b[k];
    b[i] = s / L[i * n + i];
  }
}

template <typename R>
R inf_norm(const R* v, size_t len) {
  R m = 0;
  for (size_t i = 0; i < len; ++i) m = std::max(m, std::abs(v[i]));
  return m;
}

// ------------------------------------------------ QP operator restatement ----
// theta_t / phi_t of compute_S_Phiinv (turbompc/solvers/admm/admm.py:88-101).
template <typename R>
void assemble_theta_phi(const QP<R>& qp, const Dims& d, R rho_f, R sigma, R rho_ineq,
                        Vec<R>& theta, Vec<R>& phi) {
  const int T = d.T, N = d.N, n = d.n, nx = d.nx, n0 = d.n0, m = d.m;
  theta.assign((size_t)T * n * n, R(0));
  phi.assign((size_t)N * n * n, R(0));
  for (int t = 0; t < T; ++t) {
    R* th = theta.data() + (size_t)t * n * n;
    const R* Dt = qp.D + (size_t)t * n * n;
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < n; ++j) {
        R v = Dt[i * n + j] + (i == j ? sigma : R(0));
        R gtg = 0;
        for (int r = 0; r < m; ++r) {
          const R* Gt = qp.G + (size_t)t * m * n;
          gtg += Gt[r * n + i] * Gt[r * n + j];
        }
        v += rho_ineq * gtg;
        R cc = 0;
        if (t == 0)
          for (int r = 0; r < n0; ++r) cc += qp.A0[r * n + i] * qp.A0[r * n + j];
        if (t < N) {
          const R* A = qp.Am + (size_t)t * nx * n;
          for (int r = 0; r < nx; ++r) cc += A[r * n + i] * A[r * n + j];
        }
        if (t > 0) {
          const R* A = qp.Ap + (size_t)(t - 1) * nx * n;
          for (int r = 0; r < nx; ++r) cc += A[r * n + i] * A[r * n + j];
        }
        th[i * n + j] = v + rho_f * cc;
      }
  }
  for (int t = 0; t < N; ++t) {  // phi_t = E_t + rho_f A_plus_t^T A_minus_t
    R* ph = phi.data() + (size_t)t * n * n;
    const R* Et = qp.E + (size_t)t * n * n;
    const R* Am = qp.Am + (size_t)t * nx * n;
    const R* Ap = qp.Ap + (size_t)t * nx * n;
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < n; ++j) {
        R s = 0;
        for (int r = 0; r < nx; ++r) s += Ap[r * n + i] * Am[r * n + j];
        ph[i * n + j] = Et[i * n + j] + rho_f * s;
      }
  }
}

// S and Phiinv blocks (admm.py:103-154).
template <typename R>
void build_S_Phiinv(const Vec<R>& theta, const Vec<R>& phi, const Dims& d, R* S,
                    R* Phiinv) {
  const int T = d.T, N = d.N, n = d.n, w = 3 * n;
  Vec<R> thinv((size_t)T * n * n);
  for (int t = 0; t < T; ++t)
    inverse(theta.data() + (size_t)t * n * n, n, thinv.data() + (size_t)t * n * n);
  Vec<R> tmp(n * n), prod(n * n);
  for (int t = 0; t < T; ++t) {
    R* St = S + (size_t)t * n * w;
    R* Pt = Phiinv + (size_t)t * n * w;
    const R* thi = thinv.data() + (size_t)t * n * n;
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < n; ++j) {
        St[i * w + j] = t > 0 ? phi[(size_t)(t - 1) * n * n + i * n + j] : R(0);
        St[i * w + n + j] = theta[(size_t)t * n * n + i * n + j];
        St[i * w + 2 * n + j] = t < N ? phi[(size_t)t * n * n + j * n + i] : R(0);
        Pt[i * w + n + j] = -thi[i * n + j];
      }
    // prev: theta_t^-1 phi_{t-1} theta_{t-1}^-1 (zero block at t = 0)
    if (t == 0) {
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) Pt[i * w + j] = 0;
    } else {
      const R* ph = phi.data() + (size_t)(t - 1) * n * n;
      const R* thp = thinv.data() + (size_t)(t - 1) * n * n;
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
          R s = 0;
          for (int k = 0; k < n; ++k) s += thi[i * n + k] * ph[k * n + j];
          tmp[i * n + j] = s;
        }
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
          R s = 0;
          for (int k = 0; k < n; ++k) s += tmp[i * n + k] * thp[k * n + j];
          Pt[i * w + j] = s;
        }
    }
    // next: theta_t^-1 phi_t^T theta_{t+1}^-1
    if (t < N) {
      const R* ph = phi.data() + (size_t)t * n * n;
      const R* thn = thinv.data() + (size_t)(t + 1) * n * n;
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
          R s = 0;
          for (int k = 0; k < n; ++k) s += thi[i * n + k] * ph[j * n + k];
          tmp[i * n + j] = s;
        }
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
          R s = 0;
          for (int k = 0; k < n; ++k) s += tmp[i * n + k] * thn[k * n + j];
          Pt[i * w + 2 * n + j] = s;
        }
    } else {
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) Pt[i * w + 2 * n + j] = 0;
    }
  }
}

// _apply_C_parts (admm.py:209-221)
template <typename R>
void apply_C(const QP<R>& qp, const Dims& d, const R* x, R* Cx0, R* Cx) {
  const int N = d.N, n = d.n, nx = d.nx, n0 = d.n0;
  matvec(qp.A0, n0, n, x, Cx0, false);
  for (int t = 0; t < N; ++t) {
    matvec(qp.Am + (size_t)t * nx * n, nx, n, x + (size_t)t * n, Cx + (size_t)t * nx, false);
    matvec(qp.Ap + (size_t)t * nx * n, nx, n, x + (size_t)(t + 1) * n, Cx + (size_t)t * nx,
           true);
  }
}
// _apply_Ct (admm.py:229-249)
template <typename R>
void apply_Ct(const QP<R>& qp, const Dims& d, const R* y0, const R* y, R* out) {
  const int T = d.T, N = d.N, n = d.n, nx = d.nx, n0 = d.n0;
  std::fill(out, out + (size_t)T * n, R(0));
  matTvec(qp.A0, n0, n, y0, out, true);
  for (int t = 0; t < N; ++t) {
    matTvec(qp.Am + (size_t)t * nx * n, nx, n, y + (size_t)t * nx, out + (size_t)t * n, true);
    matTvec(qp.Ap + (size_t)t * nx * n, nx, n, y + (size_t)t * nx, out + (size_t)(t + 1) * n,
            true);
  }
}
// _apply_G / _apply_Gt (admm.py:252-263)
template <typename R>
void apply_G(const QP<R>& qp, const Dims& d, const R* x, R* Gx) {
  for (int t = 0; t < d.T; ++t)
    matvec(qp.G + (size_t)t * d.m * d.n, d.m, d.n, x + (size_t)t * d.n, Gx + (size_t)t * d.m,
           false);
}
template <typename R>
void apply_Gt(const QP<R>& qp, const Dims& d, const R* y, R* out, bool accumulate) {
  for (int t = 0; t < d.T; ++t)
    matTvec(qp.G + (size_t)t * d.m * d.n, d.m, d.n, y + (size_t)t * d.m, out + (size_t)t * d.n,
            accumulate);
}
// _apply_P (admm.py:185-206): row t = E_{t-1} x_{t-1} + D_t x_t + E_t^T x_{t+1}
template <typename R>
void apply_P(const QP<R>& qp, const Dims& d, const R* x, R* out) {
  const int T = d.T, N = d.N, n = d.n;
  for (int t = 0; t < T; ++t) {
    R* o = out + (size_t)t * n;
    matvec(qp.D + (size_t)t * n * n, n, n, x + (size_t)t * n, o, false);
    if (t > 0) matvec(qp.E + (size_t)(t - 1) * n * n, n, n, x + (size_t)(t - 1) * n, o, true);
    if (t < N) matTvec(qp.E + (size_t)t * n * n, n, n, x + (size_t)(t + 1) * n, o, true);
  }
}

// ---------------------------------------------------------- Schur solvers ----
// Exact block-tridiagonal solve by block Cholesky: S = L L^T with L_t lower
// triangular on the diagonal and M_t = phi_{t-1} L_{t-1}^{-T} below it.  The
// reference CPU path solves the same system densely (linear_solve.py:85-112).
template <typename R>
struct BlockChol {
  int T, n;
  Vec<R> L, M;  // L (T,n,n) lower; M (T,n,n) with M_0 unused
  void factor(const R* theta, const R* phi, int T_, int n_) {
    T = T_;
    n = n_;
    L.assign((size_t)T * n * n, R(0));
    M.assign((size_t)T * n * n, R(0));
    std::memcpy(L.data(), theta, sizeof(R) * n * n);
    cholesky(L.data(), n);
    Vec<R> row(n);
    for (int t = 1; t < T; ++t) {
      const R* Lp = L.data() + (size_t)(t - 1) * n * n;
      R* Mt = M.data() + (size_t)t * n * n;
      // row i of M_t solves L_{t-1} m_i = phi_{t-1}[i,:]^T
      for (int i = 0; i < n; ++i) {
        for (int k = 0; k < n; ++k) row[k] = phi[(size_t)(t - 1) * n * n + i * n + k];
        trsv_lower(Lp, n, row.data());
        for (int k = 0; k < n; ++k) Mt[i * n + k] = row[k];
      }
      R* Lt = L.data() + (size_t)t * n * n;
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
          R s = theta[(size_t)t * n * n + i * n + j];
          for (int k = 0; k < n; ++k) s -= Mt[i * n + k] * Mt[j * n + k];
          Lt[i * n + j] = s;
        }
      cholesky(Lt, n);
    }
  }
  void solve(const R* rhs, R* x) const {
    Vec<R> y((size_t)T * n);
    for (int t = 0; t < T; ++t) {
      R* yt = y.data() + (size_t)t * n;
      for (int i = 0; i < n; ++i) yt[i] = rhs[(size_t)t * n + i];
      if (t > 0) {
        const R* Mt = M.data() + (size_t)t * n * n;
        const R* yp = y.data() + (size_t)(t - 1) * n;
        for (int i = 0; i < n; ++i) {
          R s = 0;
          for (int k = 0; k < n; ++k) s += Mt[i * n + k] * yp[k];
          yt[i] -= s;
        }
      }
      trsv_lower(L.data() + (size_t)t * n * n, n, yt);
    }
    for (int t = T - 1; t >= 0; --t) {
      R* xt = x + (size_t)t * n;
      for (int i = 0; i < n; ++i) xt[i] = y[(size_t)t * n + i];
      if (t < T - 1) {
        const R* Mn = M.data() + (size_t)(t + 1) * n * n;
        const R* xn = x + (size_t)(t + 1) * n;
        for (int i = 0; i < n; ++i) {
          R s = 0;
          for (int k = 0; k < n; ++k) s += Mn[k * n + i] * xn[k];
          xt[i] -= s;
        }
      }
      trsv_lower_T(L.data() + (size_t)t * n * n, n, xt);
    }
  }
};

// v = blocks (T,n,3n) applied to [v_{t-1}, v_t, v_{t+1}] with zero padding.
template <typename R>
void blk_apply(const R* Blk, int T, int n, const R* v, R* out) {
  const int w = 3 * n;
  for (int t = 0; t < T; ++t)
    for (int i = 0; i < n; ++i) {
      const R* row = Blk + (size_t)t * n * w + (size_t)i * w;
      R s = 0;
      if (t > 0)
        for (int k = 0; k < n; ++k) s += row[k] * v[(size_t)(t - 1) * n + k];
      for (int k = 0; k < n; ++k) s += row[n + k] * v[(size_t)t * n + k];
      if (t < T - 1)
        for (int k = 0; k < n; ++k) s += row[2 * n + k] * v[(size_t)(t + 1) * n + k];
      out[(size_t)t * n + i] = s;
    }
}

// PCGPrimalOptimalControl.solve_linear_system (pcg_primal.py:70-175).
template <typename R>
int pcg_solve(const R* S, const R* Phiinv, int T, int n, const R* gamma, const R* x0,
              R* x, R eps, int max_iter) {
  const size_t L = (size_t)T * n;
  Vec<R> r(L), rt(L), p(L), Up(L);
  blk_apply(S, T, n, x0, Up.data());
  for (size_t i = 0; i < L; ++i) r[i] = gamma[i] - Up[i];
  blk_apply(Phiinv, T, n, r.data(), rt.data());
  p = rt;
  R eta = 0;
  for (size_t i = 0; i < L; ++i) eta += r[i] * rt[i];
  const R eta0 = std::abs(eta);
  for (size_t i = 0; i < L; ++i) x[i] = x0[i];
  const R abs_tol = R(1e-12);
  if (eta0 <= abs_tol) return 0;
  int it = 0;
  while (true) {
    const bool converged = std::abs(eta) < abs_tol + eps * eta0;
    bool cont = (!converged) && (it <= max_iter - 1);
    cont = cont || (it < 1);
    if (!cont) break;
    blk_apply(S, T, n, p.data(), Up.data());
    R v = 0;
    for (size_t i = 0; i < L; ++i) v += p[i] * Up[i];
    const R a = eta / v;
    for (size_t i = 0; i < L; ++i) {
      x[i] += a * p[i];
      r[i] -= a * Up[i];
    }
    blk_apply(Phiinv, T, n, r.data(), rt.data());
    R etap = 0;
    for (size_t i = 0; i < L; ++i) etap += r[i] * rt[i];
    const R beta = etap / eta;
    for (size_t i = 0; i < L; ++i) p[i] = rt[i] + beta * p[i];
    eta = etap;
    ++it;
  }
  return it;
}

// ------------------------------------------------------------- residuals ----
template <typename R>
struct Residuals {
  R rp, rd, pn, dn, np, nd;
};

// _compute_residuals (admm.py:266-331)
template <typename R>
Residuals<R> compute_residuals(const QP<R>& qp, const Dims& d, const State<R>& s) {
  const int T = d.T, N = d.N, n = d.n, nx = d.nx, n0 = d.n0, m = d.m;
  Vec<R> Cx0(n0), Cx((size_t)N * nx), Gx((size_t)T * m);
  apply_C(qp, d, s.x.data(), Cx0.data(), Cx.data());
  if (m) apply_G(qp, d, s.x.data(), Gx.data());
  R rp = 0, nCx = 0, nc = 0;
  for (int i = 0; i < n0; ++i) {
    rp = std::max(rp, std::abs(Cx0[i] - qp.c0[i]));
    nCx = std::max(nCx, std::abs(Cx0[i]));
    nc = std::max(nc, std::abs(qp.c0[i]));
  }
  for (size_t i = 0; i < (size_t)N * nx; ++i) {
    rp = std::max(rp, std::abs(Cx[i] - qp.c[i]));
    nCx = std::max(nCx, std::abs(Cx[i]));
    nc = std::max(nc, std::abs(qp.c[i]));
  }
  R nGx = 0, nz = 0;
  if (m) {
    for (size_t i = 0; i < (size_t)T * m; ++i)
      rp = std::max(rp, std::abs(Gx[i] - s.z[i]));
    nGx = inf_norm(Gx.data(), Gx.size());
    nz = inf_norm(s.z.data(), s.z.size());
  }
  const R np = std::max(std::max(nCx, nGx), std::max(nc, nz));
  Vec<R> Px((size_t)T * n), Aty((size_t)T * n);
  apply_P(qp, d, s.x.data(), Px.data());
  apply_Ct(qp, d, s.y_f0.data(), s.y_f.data(), Aty.data());
  if (m) apply_Gt(qp, d, s.y_g.data(), Aty.data(), true);
  R rd = 0;
  for (size_t i = 0; i < (size_t)T * n; ++i)
    rd = std::max(rd, std::abs(Px[i] + qp.q[i] + Aty[i]));
  const bool slack = qp.use_slack && m > 0;
  if (slack)
    for (size_t i = 0; i < (size_t)T * m; ++i)
      rd = std::max(rd, std::abs(qp.slack_w * s.xi[i] + s.y_g[i]));
  R nd = std::max(std::max(inf_norm(Px.data(), Px.size()), inf_norm(Aty.data(), Aty.size())),
                  inf_norm(qp.q, (size_t)T * n));
  if (slack)
    nd = std::max(nd, std::max(qp.slack_w * inf_norm(s.xi.data(), s.xi.size()),
                               inf_norm(s.y_g.data(), s.y_g.size())));
  Residuals<R> r;
  r.rp = rp;
  r.rd = rd;
  r.np = np;
  r.nd = nd;
  r.pn = rp / (R(1e-10) + np);
  r.dn = rd / (R(1e-10) + nd);
  return r;
}

// `it % k == 0` with XLA's integer-remainder convention (x % 0 == x).
inline bool mod_zero(int it, int k) { return k > 0 ? (it % k) == 0 : it == 0; }

template <typename R>
bool too_large(const Residuals<R>& r, R eps_abs, R eps_rel) {  // admm.py:347-355
  return (r.rp > eps_abs + eps_rel * r.np) || (r.rd > eps_abs + eps_rel * r.nd);
}

// --------------------------------------------------------------- ADMM ----
// ADMMSolver._solve_jax_loop (admm.py:795-1049) for one problem.
template <typename R>
void admm_one(const QP<R>& qp, const Dims& d, State<R>& s, const ora_cfg& cfg, int schur,
              int* iters_out, int* pcg_total) {
  const int T = d.T, N = d.N, n = d.n, nx = d.nx, n0 = d.n0, m = d.m;
  const R sigma = (R)cfg.sigma, alpha = (R)cfg.alpha;
  const R eps_abs = (R)cfg.eps_abs, eps_rel = (R)cfg.eps_rel;
  Vec<R> theta, phi, S, Phi;
  BlockChol<R> chol;
  auto build = [&](R rho) {  // compute_S_Phiinv (admm.py:827-832, :513-518)
    assemble_theta_phi(qp, d, rho * (R)cfg.rho_f_factor, sigma, rho, theta, phi);
    if (schur == 0) {
      chol.factor(theta.data(), phi.data(), T, n);
    } else {
      S.resize((size_t)T * n * 3 * n);
      Phi.resize((size_t)T * n * 3 * n);
      build_S_Phiinv(theta, phi, d, S.data(), Phi.data());
    }
  };
  build(s.rho);
  const R inf = std::numeric_limits<R>::infinity();
  Residuals<R> res_prev{inf, inf, inf, inf, R(1), R(1)};
  Vec<R> gam((size_t)T * n), xt((size_t)T * n), tmp((size_t)T * n), c0t(n0), ct((size_t)N * nx),
      zy((size_t)T * m), Cx0(n0), Cx((size_t)N * nx), Gx((size_t)T * m), zn((size_t)T * m);
  int it = 0, pcg_sum = 0;
  while (true) {
    // cond_fun (admm.py:843-851)
    const bool sc = mod_zero(it, cfg.check_every);
    const bool tl = too_large(res_prev, eps_abs, eps_rel);
    bool cont = (it < cfg.max_iter) && (!sc || tl);
    cont = cont || it < 1;
    if (!cont) break;
    // body_fun (admm.py:853-995)
    const R rho = s.rho;
    const R rho_f = rho * (R)cfg.rho_f_factor;
    // compute_gamma (admm.py:157-174)
    for (int i = 0; i < n0; ++i) c0t[i] = rho_f * qp.c0[i] - s.y_f0[i];
    for (size_t i = 0; i < (size_t)N * nx; ++i) ct[i] = rho_f * qp.c[i] - s.y_f[i];
    apply_Ct(qp, d, c0t.data(), ct.data(), tmp.data());
    for (size_t i = 0; i < (size_t)T * n; ++i) gam[i] = sigma * s.x[i] - qp.q[i] + tmp[i];
    if (m) {
      for (size_t i = 0; i < (size_t)T * m; ++i) zy[i] = rho * s.z[i] - s.y_g[i];
      apply_Gt(qp, d, zy.data(), gam.data(), true);
    }
    // Schur solve (admm.py:882-883)
    if (schur == 0) {
      chol.solve(gam.data(), xt.data());
    } else {
      pcg_sum += pcg_solve(S.data(), Phi.data(), T, n, gam.data(), s.x.data(), xt.data(),
                           (R)cfg.pcg_eps, cfg.pcg_max_iter);
    }
    apply_C(qp, d, xt.data(), Cx0.data(), Cx.data());
    if (m) apply_G(qp, d, xt.data(), Gx.data());
    // over-relaxation, slack and dual updates (admm.py:891-931)
    if (m) {
      const R gs = qp.slack_w;
      for (size_t i = 0; i < (size_t)T * m; ++i) {
        const R zt = alpha * Gx[i] + (R(1) - alpha) * s.z[i] + s.y_g[i] / rho;
        const R proj = std::min(std::max(zt, qp.l[i]), qp.u[i]);
        if (qp.use_slack) {
          const R frac = gs / (gs + rho);
          zn[i] = (R(1) - frac) * zt + frac * proj;
          s.xi[i] = (rho / (gs + rho)) * (proj - zt);
        } else {
          zn[i] = proj;
          s.xi[i] = R(0);
        }
      }
    }
    for (int i = 0; i < n0; ++i)
      s.y_f0[i] += rho_f * (alpha * Cx0[i] + (R(1) - alpha) * qp.c0[i] - qp.c0[i]);
    for (size_t i = 0; i < (size_t)N * nx; ++i)
      s.y_f[i] += rho_f * (alpha * Cx[i] + (R(1) - alpha) * qp.c[i] - qp.c[i]);
    if (m)
      for (size_t i = 0; i < (size_t)T * m; ++i) {
        s.y_g[i] += rho * (alpha * Gx[i] + (R(1) - alpha) * s.z[i] - zn[i]);
        s.z[i] = zn[i];
      }
    for (size_t i = 0; i < (size_t)T * n; ++i)
      s.x[i] = alpha * xt[i] + (R(1) - alpha) * s.x[i];
    // _update_residuals_and_rho (admm.py:392-556)
    if (mod_zero(it, cfg.check_every)) {
      const Residuals<R> r = compute_residuals(qp, d, s);
      res_prev = r;
      const R cand = std::min(std::max(rho * std::sqrt(r.pn / r.dn), (R)cfg.rho_min),
                              (R)cfg.rho_max);
      const R ratio = std::max(cand / rho, rho / cand);
      const bool converged = !too_large(r, eps_abs, eps_rel);
      bool keep = it < 2 || !mod_zero(it, cfg.adapt_rho_every);
      keep = keep || converged;
      keep = keep || ratio < (R)cfg.adaptive_rho_tolerance;
      if (!keep) {
        s.rho = cand;
        build(cand);
      }
    }
    ++it;
  }
  *iters_out = it;
  if (pcg_total) *pcg_total = pcg_sum;
}

template <typename R>
int admm_solve_t(int schur, const ora_dims* dd, const ora_qp* qp, const ora_state* in,
                 ora_state* out, int32_t* iters, int32_t* pcg_iters, const ora_cfg* cfg,
                 int nthreads) {
  const Dims d(*dd);
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (int b = 0; b < d.B; ++b) {
    State<R> s(d);
    load_state(s, *in, d, b);
    const QP<R> v = qp_view<R>(*qp, d, b);
    int it = 0, pc = 0;
    admm_one(v, d, s, *cfg, schur, &it, &pc);
    ora_state o = *out;
    store_state(s, o, d, b);
    iters[b] = it;
    if (pcg_iters) pcg_iters[b] = pc;
  }
  return 0;
}

template <typename R>
int schur_build_t(const ora_dims* dd, const ora_qp* qp, const void* rho, double sigma,
                  double rho_f_factor, void* S, void* Phiinv, int nthreads) {
  const Dims d(*dd);
  const size_t blk = (size_t)d.T * d.n * 3 * d.n;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (int b = 0; b < d.B; ++b) {
    const QP<R> v = qp_view<R>(*qp, d, b);
    const R r = static_cast<const R*>(rho)[b];
    Vec<R> theta, phi;
    assemble_theta_phi(v, d, r * (R)rho_f_factor, (R)sigma, r, theta, phi);
    build_S_Phiinv(theta, phi, d, static_cast<R*>(S) + b * blk, static_cast<R*>(Phiinv) + b * blk);
  }
  return 0;
}

template <typename R>
int pcg_t(int B, int T, int n, const void* S, const void* Phiinv, const void* rhs,
          const void* x0, void* x, int32_t* iters, double eps, int32_t max_iter, int nthreads) {
  const size_t blk = (size_t)T * n * 3 * n, vec = (size_t)T * n;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (int b = 0; b < B; ++b)
    iters[b] = pcg_solve(static_cast<const R*>(S) + b * blk, static_cast<const R*>(Phiinv) + b * blk,
                         T, n, static_cast<const R*>(rhs) + b * vec,
                         static_cast<const R*>(x0) + b * vec, static_cast<R*>(x) + b * vec, (R)eps,
                         max_iter);
  return 0;
}

template <typename R>
int blktri_t(int B, int T, int n, const void* S, const void* rhs, void* x, int nthreads) {
  const size_t blk = (size_t)T * n * 3 * n, vec = (size_t)T * n;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (int b = 0; b < B; ++b) {
    const R* Sb = static_cast<const R*>(S) + b * blk;
    Vec<R> theta((size_t)T * n * n), phi((size_t)std::max(T - 1, 0) * n * n);
    for (int t = 0; t < T; ++t)
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
          theta[(size_t)t * n * n + i * n + j] = Sb[(size_t)t * n * 3 * n + i * 3 * n + n + j];
          if (t > 0)
            phi[(size_t)(t - 1) * n * n + i * n + j] = Sb[(size_t)t * n * 3 * n + i * 3 * n + j];
        }
    BlockChol<R> ch;
    ch.factor(theta.data(), phi.data(), T, n);
    ch.solve(static_cast<const R*>(rhs) + b * vec, static_cast<R*>(x) + b * vec);
  }
  return 0;
}

// assemble_backward_kkt_system + solve_backward_kkt
// (turbompc/solvers/backward/backward_kkt_jax.py:10-211), dense LU.
template <typename R>
int adjoint_t(const ora_dims* dd, const ora_qp* qp, void* dz, void* mult, int nthreads) {
  const Dims d(*dd);
  const int T = d.T, N = d.N, n = d.n, nx = d.nx, n0 = d.n0, m = d.m;
  const int nt = T * n, meq = n0 + N * nx, mi = T * m, K = nt + meq + mi;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
  for (int b = 0; b < d.B; ++b) {
    const QP<R> v = qp_view<R>(*qp, d, b);
    Vec<R> A((size_t)K * K, R(0)), rhs(K, R(0));
    auto at = [&](int i, int j) -> R& { return A[(size_t)i * K + j]; };
    for (int t = 0; t < T; ++t)
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
          at(t * n + i, t * n + j) = v.D[(size_t)t * n * n + i * n + j];
          if (t < N) at(t * n + i, (t + 1) * n + j) = v.E[(size_t)t * n * n + j * n + i];
          if (t > 0) at(t * n + i, (t - 1) * n + j) = v.E[(size_t)(t - 1) * n * n + i * n + j];
        }
    // C = [A0 rows; dynamics rows; G rows] placed symmetric.
    auto put = [&](int row, int col, R val) {
      at(nt + row, col) = val;
      at(col, nt + row) = val;
    };
    for (int r = 0; r < n0; ++r)
      for (int j = 0; j < n; ++j) put(r, j, v.A0[r * n + j]);
    for (int t = 0; t < N; ++t)
      for (int r = 0; r < nx; ++r)
        for (int j = 0; j < n; ++j) {
          put(n0 + t * nx + r, t * n + j, v.Am[(size_t)t * nx * n + r * n + j]);
          put(n0 + t * nx + r, (t + 1) * n + j, v.Ap[(size_t)t * nx * n + r * n + j]);
        }
    for (int t = 0; t < T; ++t)
      for (int r = 0; r < m; ++r) {
        R nrm = 0;
        for (int j = 0; j < n; ++j) {
          const R g = v.G[(size_t)t * m * n + r * n + j];
          put(meq + t * m + r, t * n + j, g);
          nrm += g * g;
        }
        if (nrm == R(0)) at(nt + meq + t * m + r, nt + meq + t * m + r) = R(-1e-12);
      }
    for (int i = 0; i < nt; ++i) rhs[i] = -v.q[i];
    std::vector<int> piv(K);
    lu_factor(A.data(), K, piv.data());
    lu_solve(A.data(), K, piv.data(), rhs.data());
    std::memcpy(static_cast<R*>(dz) + (size_t)b * nt, rhs.data(), sizeof(R) * nt);
    std::memcpy(static_cast<R*>(mult) + (size_t)b * (meq + mi), rhs.data() + nt,
                sizeof(R) * (meq + mi));
  }
  return 0;
}

// --------------------------------------------------------- quadrotor ----
// Rotor-thrust quadrotor used for the B=4096 SQP workload (the reference's own
// quadrotor model uses thrust/torque inputs; this model is specified in the
// build's design notes).  State [p(3), q(4) (w,x,y,z), v(3), omega(3)], input
// four rotor thrusts in an x-configuration.  params: mass, Jxx, Jyy, Jzz, arm,
// yaw coefficient, g.
template <typename S>
void quad_xdot(const S* x, const S* f, const double* P, S* xd) {
  const double mass = P[0], Jx = P[1], Jy = P[2], Jz = P[3], arm = P[4], ky = P[5], g = P[6];
  const double dd = arm / std::sqrt(2.0);
  const S qw = x[3], qx = x[4], qy = x[5], qz = x[6];
  const S wx = x[10], wy = x[11], wz = x[12];
  const S F = f[0] + f[1] + f[2] + f[3];
  const S tx = dd * (f[0] + f[1] - f[2] - f[3]);
  const S ty = dd * (-f[0] + f[1] + f[2] - f[3]);
  const S tz = ky * (-f[0] + f[1] - f[2] + f[3]);
  xd[0] = x[7];
  xd[1] = x[8];
  xd[2] = x[9];
  xd[3] = 0.5 * (-qx * wx - qy * wy - qz * wz);
  xd[4] = 0.5 * (qw * wx + qy * wz - qz * wy);
  xd[5] = 0.5 * (qw * wy - qx * wz + qz * wx);
  xd[6] = 0.5 * (qw * wz + qx * wy - qy * wx);
  xd[7] = (2.0 * (qx * qz + qw * qy)) * F / mass;
  xd[8] = (2.0 * (qy * qz - qw * qx)) * F / mass;
  xd[9] = (1.0 - 2.0 * (qx * qx + qy * qy)) * F / mass - g;
  xd[10] = (tx - (Jz - Jy) * wy * wz) / Jx;
  xd[11] = (ty - (Jx - Jz) * wz * wx) / Jy;
  xd[12] = (tz - (Jy - Jx) * wx * wy) / Jz;
}

// RK4 step with the control held (turbompc/dynamics/integrators.py:67-76).
template <typename S>
void quad_rk4(const S* x, const S* f, double dt, const double* P, S* xn) {
  S k1[13], k2[13], k3[13], k4[13], tmp[13];
  quad_xdot(x, f, P, k1);
  for (int i = 0; i < 13; ++i) tmp[i] = x[i] + 0.5 * dt * k1[i];
  quad_xdot(tmp, f, P, k2);
  for (int i = 0; i < 13; ++i) tmp[i] = x[i] + 0.5 * dt * k2[i];
  quad_xdot(tmp, f, P, k3);
  for (int i = 0; i < 13; ++i) tmp[i] = x[i] + dt * k3[i];
  quad_xdot(tmp, f, P, k4);
  for (int i = 0; i < 13; ++i)
    xn[i] = x[i] + (1.0 / 6.0) * (k1[i] + 2.0 * k2[i] + 2.0 * k3[i] + k4[i]) * dt;
}

}  // namespace

// ================================================================ C ABI ====
extern "C" {

int ora_admm_solve(int dtype, int schur, const ora_dims* d, const ora_qp* qp,
                   const ora_state* in, ora_state* out, int32_t* iters, int32_t* pcg_iters,
                   const ora_cfg* cfg, int nthreads) {
  if (dtype == 8) return admm_solve_t<double>(schur, d, qp, in, out, iters, pcg_iters, cfg, nthreads);
  if (dtype == 4) return admm_solve_t<float>(schur, d, qp, in, out, iters, pcg_iters, cfg, nthreads);
  return -1;
}

int ora_schur_build(int dtype, const ora_dims* d, const ora_qp* qp, const void* rho,
                    double sigma, double rho_f_factor, void* S, void* Phiinv, int nthreads) {
  if (dtype == 8) return schur_build_t<double>(d, qp, rho, sigma, rho_f_factor, S, Phiinv, nthreads);
  if (dtype == 4) return schur_build_t<float>(d, qp, rho, sigma, rho_f_factor, S, Phiinv, nthreads);
  return -1;
}

int ora_pcg(int dtype, int B, int T, int n, const void* S, const void* Phiinv, const void* rhs,
            const void* x0, void* x, int32_t* iters, double eps, int32_t max_iter, int nthreads) {
  if (dtype == 8) return pcg_t<double>(B, T, n, S, Phiinv, rhs, x0, x, iters, eps, max_iter, nthreads);
  if (dtype == 4) return pcg_t<float>(B, T, n, S, Phiinv, rhs, x0, x, iters, eps, max_iter, nthreads);
  return -1;
}

int ora_blktri_solve(int dtype, int B, int T, int n, const void* S, const void* rhs, void* x,
                     int nthreads) {
  if (dtype == 8) return blktri_t<double>(B, T, n, S, rhs, x, nthreads);
  if (dtype == 4) return blktri_t<float>(B, T, n, S, rhs, x, nthreads);
  return -1;
}

int ora_adjoint_kkt(int dtype, const ora_dims* d, const ora_qp* qp, void* dz, void* mult,
                    int nthreads) {
  if (dtype == 8) return adjoint_t<double>(d, qp, dz, mult, nthreads);
  if (dtype == 4) return adjoint_t<float>(d, qp, dz, mult, nthreads);
  return -1;
}

int ora_quadrotor_rk4_jac(int K, const double* xu, double dt, const double* params, double* f,
                          double* J, int nthreads) {
  using C = std::complex<double>;
  const double h = 1e-30;  // complex-step differentiation (Squire & Trapp 1998)
#pragma omp parallel for schedule(static) num_threads(nthreads)
  for (int k = 0; k < K; ++k) {
    const double* z = xu + (size_t)k * 17;
    double xn[13];
    quad_rk4<double>(z, z + 13, dt, params, xn);
    for (int i = 0; i < 13; ++i) f[(size_t)k * 13 + i] = xn[i];
    for (int j = 0; j < 17; ++j) {
      C zc[17], out[13];
      for (int i = 0; i < 17; ++i) zc[i] = C(z[i], i == j ? h : 0.0);
      quad_rk4<C>(zc, zc + 13, dt, params, out);
      for (int i = 0; i < 13; ++i) J[(size_t)k * 13 * 17 + i * 17 + j] = out[i].imag() / h;
    }
  }
  return 0;
}

}  // extern "C"
