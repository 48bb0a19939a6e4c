// On-device linearization of spherical obstacle-avoidance constraints.
//
// Each obstacle k of problem b adds one inequality row per stage
// (OptimalControlProblemObstacle.step_inequality_constraints,
// turbompc/problems/obstacle_avoidance.py:16-52):
//   g_k(x) = 1 - |p - c_k| / (r_k + 0.001) <= 0,   p = x[0:dim]
// with lower bound -1e9 and upper bound 0.  The SQP linearizes it at the
// iterate xbar_t (get_inequalities_linearized_matrices,
// turbompc/problems/optimal_control_problem.py:580-626):
//   G row   = [dg/dx, dg/du] = [-(p - c)^T / (|p - c| (r + 0.001)), 0]
//   offset  = g(xbar) - dg/dx xbar
//   l = -1e9 - offset,  u = 0 - offset.
// The rows sit after the box rows (row0 .. row0 + K - 1 of the stage's m rows).
//
// For the exact-Hessian backward pass the same rows contribute
// sum_k mu_k d^2 g_k / dx^2 to D_t (get_inequality_lagrangian_hessian,
// optimal_control_problem.py:1443-1480), with
//   d^2 g_k / dp^2 = -(I / |d| - d d^T / |d|^3) / (r_k + 0.001),  d = p - c_k,
// and zeros outside the position block.
//
// Layouts (row-major, batch leading): states (B, T, nx), centers (B, K, dim),
// radii (B, K), G (B, T, m, n), l/u (B, T, m), mus (B, T, m), H (B, T, n, n).
#pragma once
#include "common.hpp"

namespace tmpc {

constexpr double kObstacleMargin = 0.001;
constexpr double kObstacleLower = -1.0e9;

// One thread per G entry (b, t, k, j): the G rows are written with adjacent
// threads on adjacent columns; thread j = 0 also writes l and u.  Each thread
// recomputes the distance (dim <= nx terms), which is cheaper than staging it.
template <typename R>
__global__ void obstacle_linearize_kernel(int B, int T, int nx, int n, int dim, int K, const R* __restrict__ states,
                                          const R* __restrict__ centers, const R* __restrict__ radii, int m,
                                          int row0, R* __restrict__ G, R* __restrict__ l, R* __restrict__ u) {
  const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)B * T * K * n;
  if (e >= total) return;
  const int j = (int)(e % n);
  const long long r = e / n;  // (b, t, k)
  const int k = (int)(r % K);
  const long long bt = r / K;
  const int b = (int)(bt / T);
  const R* x = states + bt * nx;
  const R* c = centers + ((long long)b * K + k) * dim;
  R ss = R(0);
  for (int i = 0; i < dim; ++i) {
    const R d = x[i] - c[i];
    ss += d * d;
  }
  const R nrm = sqrt(ss);
  const R den = radii[(long long)b * K + k] + R(kObstacleMargin);
  const long long row = bt * m + row0 + k;
  G[row * n + j] = j < dim ? -((x[j] - c[j]) / nrm) / den : R(0);
  if (j == 0) {
    R gx = R(0);  // dg/dx . xbar over the position block (zero elsewhere)
    for (int i = 0; i < dim; ++i) gx += (-((x[i] - c[i]) / nrm) / den) * x[i];
    const R off = (R(1) - nrm / den) - gx;
    l[row] = R(kObstacleLower) - off;
    u[row] = R(0) - off;
  }
}

// One thread per H entry (b, t, i, j).
template <typename R>
__global__ void obstacle_hessian_kernel(int B, int T, int nx, int n, int dim, int K, const R* __restrict__ states,
                                        const R* __restrict__ centers, const R* __restrict__ radii, int m, int row0,
                                        const R* __restrict__ mus, R* __restrict__ H) {
  const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)B * T * n * n;
  if (e >= total) return;
  const int j = (int)(e % n);
  const int i = (int)((e / n) % n);
  const long long bt = e / ((long long)n * n);
  const int b = (int)(bt / T);
  R h = R(0);
  if (i < dim && j < dim) {
    const R* x = states + bt * nx;
    const R* mu = mus + bt * m + row0;
    for (int k = 0; k < K; ++k) {
      const R* c = centers + ((long long)b * K + k) * dim;
      R ss = R(0);
      for (int q = 0; q < dim; ++q) {
        const R d = x[q] - c[q];
        ss += d * d;
      }
      const R nrm = sqrt(ss);
      const R den = radii[(long long)b * K + k] + R(kObstacleMargin);
      const R di = x[i] - c[i], dj = x[j] - c[j];
      const R hn = (i == j ? R(1) / nrm : R(0)) - di * dj / (nrm * nrm * nrm);
      h += mu[k] * (-hn / den);
    }
  }
  H[e] = h;
}

}  // namespace tmpc
