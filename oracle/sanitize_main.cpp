// TEST INFRASTRUCTURE ONLY — drives every entry point of the CPU oracle on a
// small random QP, in fp32 and fp64, so that a build with AddressSanitizer and
// UndefinedBehaviorSanitizer (`make -C oracle asan`) checks the oracle's own
// memory accesses and arithmetic.  Exit status 0 when every call returns 0 and
// every output is finite; the sanitizers abort on their first finding.
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <vector>

#include "oracle.h"

namespace {

struct Lcg {
  uint64_t s = 0x9e3779b97f4a7c15ull;
  double uni() {  // [0, 1)
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return (double)(s >> 11) * (1.0 / 9007199254740992.0);
  }
  double sym() { return 2.0 * uni() - 1.0; }
};

template <typename R>
bool finite(const std::vector<R>& v) {
  for (R x : v)
    if (!std::isfinite((double)x)) return false;
  return true;
}

template <typename R>
int run(int schur, bool slack) {
  const int B = 3, T = 6, N = T - 1, n = 5, nx = 3, n0 = 3, m = 2;
  Lcg g;
  std::vector<R> D(B * T * n * n, 0), E(B * N * n * n, 0), q(B * T * n), A0(B * n0 * n, 0), Am(B * N * nx * n),
      Ap(B * N * nx * n, 0), G(B * T * m * n), l(B * T * m), u(B * T * m), c0(B * n0), c(B * N * nx);
  for (int b = 0; b < B; ++b) {
    for (int t = 0; t < T; ++t)
      for (int i = 0; i < n; ++i) {
        D[((b * T + t) * n + i) * n + i] = (R)(1.0 + g.uni());
        q[(b * T + t) * n + i] = (R)g.sym();
      }
    for (int i = 0; i < n0; ++i) {
      A0[(b * n0 + i) * n + i] = 1;
      c0[b * n0 + i] = (R)g.sym();
    }
    for (int t = 0; t < N; ++t)
      for (int i = 0; i < nx; ++i) {
        for (int k = 0; k < n; ++k) Am[((b * N + t) * nx + i) * n + k] = (R)((k == i ? 1.0 : 0.0) + 0.2 * g.sym());
        Ap[((b * N + t) * nx + i) * n + i] = -1;
        c[(b * N + t) * nx + i] = (R)(0.1 * g.sym());
      }
    for (int t = 0; t < T; ++t)
      for (int r = 0; r < m; ++r) {
        for (int k = 0; k < n; ++k) G[((b * T + t) * m + r) * n + k] = (R)g.sym();
        l[(b * T + t) * m + r] = (R)(-0.5 - g.uni());
        u[(b * T + t) * m + r] = (R)(0.5 + g.uni());
      }
  }
  const ora_dims d{B, T, n, nx, n0, m};
  const ora_qp qp{D.data(), E.data(), q.data(), A0.data(), Am.data(), Ap.data(), G.data(), l.data(), u.data(),
                  c0.data(), c.data(), slack ? 10.0 : 0.0, slack ? 1 : 0};
  std::vector<R> x(B * T * n, 0), z(B * T * m, 0), yg(B * T * m, 0), yf0(B * n0, 0), yf(B * N * nx, 0),
      xi(B * T * m, 0), rho(B, (R)0.1);
  std::vector<R> xo(x.size()), zo(z.size()), ygo(yg.size()), yf0o(yf0.size()), yfo(yf.size()), xio(xi.size()),
      rhoo(rho.size());
  const ora_state in{x.data(), z.data(), yg.data(), yf0.data(), yf.data(), xi.data(), rho.data()};
  ora_state out{xo.data(), zo.data(), ygo.data(), yf0o.data(), yfo.data(), xio.data(), rhoo.data()};
  std::vector<int32_t> iters(B), pcg(B);
  const ora_cfg cfg{40, 5, 10, 30, 1e-6, 1e-6, 1e-6, 1e-6, 1e6, 5.0, 100.0, 1.6, 1e-10};
  const int e = (int)sizeof(R);
  if (ora_admm_solve(e, schur, &d, &qp, &in, &out, iters.data(), pcg.data(), &cfg, 2)) return 1;
  if (!finite(xo) || !finite(yfo) || !finite(ygo) || !finite(rhoo)) return 2;
  std::vector<R> S(B * T * n * 3 * n), P(S.size());
  if (ora_schur_build(e, &d, &qp, rho.data(), 1e-6, 100.0, S.data(), P.data(), 2)) return 3;
  std::vector<R> rhs(B * T * n), xs(B * T * n);
  for (auto& v : rhs) v = (R)g.sym();
  if (ora_pcg(e, B, T, n, S.data(), P.data(), rhs.data(), x.data(), xs.data(), iters.data(), 1e-8, 50, 2)) return 4;
  if (ora_blktri_solve(e, B, T, n, S.data(), rhs.data(), xs.data(), 2)) return 5;
  if (!finite(xs)) return 6;
  std::vector<R> dz(B * T * n), mult(B * (n0 + N * nx + T * m));
  if (ora_adjoint_kkt(e, &d, &qp, dz.data(), mult.data(), 2)) return 7;
  if (!finite(dz) || !finite(mult)) return 8;
  return 0;
}

int quad() {
  const int K = 4;
  std::vector<double> xu(K * 17), f(K * 13), J(K * 13 * 17);
  Lcg g;
  for (int k = 0; k < K; ++k) {
    for (int i = 0; i < 17; ++i) xu[k * 17 + i] = 0.3 * g.sym();
    xu[k * 17 + 3] = 1.0;  // near-unit quaternion
    for (int i = 13; i < 17; ++i) xu[k * 17 + i] = 2.0 + g.uni();
  }
  const double params[7] = {1.0, 0.01, 0.01, 0.02, 0.15, 0.016, 9.81};
  if (ora_quadrotor_rk4_jac(K, xu.data(), 0.02, params, f.data(), J.data(), 2)) return 9;
  return finite(f) && finite(J) ? 0 : 10;
}

}  // namespace

int main() {
  int fails = 0;
  for (int schur = 0; schur < 2; ++schur)
    for (int slack = 0; slack < 2; ++slack) {
      const int a = run<float>(schur, slack != 0), b = run<double>(schur, slack != 0);
      if (a || b) {
        std::printf("schur %d slack %d: fp32 status %d, fp64 status %d\n", schur, slack, a, b);
        ++fails;
      }
    }
  const int qs = quad();
  if (qs) {
    std::printf("quadrotor: status %d\n", qs);
    ++fails;
  }
  std::printf(fails ? "oracle sanitize: %d failures\n" : "oracle sanitize: ok\n", fails);
  return fails ? 1 : 0;
}
