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

// One thread per obstacle row (b, t, k), k fastest: the distance once, the
// row's n G entries into LDS, l and u directly; then the block writes its
// rows' G entries with adjacent threads on adjacent entries (a stage's K rows
// are contiguous in G).  Row indices are 32-bit (the host checks
// B T K < 2^31); G addresses are formed in 64 bits.
constexpr int kObstacleBlock = 128;

// Optional second destination of the rows: the streaming solve's stage
// records (the M record of (t, b) at am + (t B + b) amp, its rows of n
// entries, the obstacle rows from g_off; l and u at l_off and u_off of the rv
// record), so that an SQP step needs no copy of them.
template <typename R>
struct ObsRecOut {
  R* am = nullptr;  // null: the QP layout only
  R* rv = nullptr;
  int amp = 0, rvp = 0, g_off = 0, l_off = 0, u_off = 0;
};

// states: rows of ls >= dim elements per (b, t) (the positions first)
template <typename R>
__global__ __launch_bounds__(kObstacleBlock) void obstacle_linearize_kernel(int B, int T, int ls, int n, int dim,
                                                                            int K, const R* __restrict__ states,
                                                                            const R* __restrict__ centers,
                                                                            const R* __restrict__ radii, int m,
                                                                            int row0, R* __restrict__ G,
                                                                            R* __restrict__ l, R* __restrict__ u,
                                                                            ObsRecOut<R> rec) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  // each row's destinations (element offsets of its first entry in G and in
  // the records), then its n entries
  size_t* qrow = reinterpret_cast<size_t*>(smem_raw);  // [kObstacleBlock]
  size_t* rrow = qrow + kObstacleBlock;                 // [kObstacleBlock]
  R* rowv = reinterpret_cast<R*>(rrow + kObstacleBlock);  // [kObstacleBlock][n]
  const unsigned rows = (unsigned)B * (unsigned)T * (unsigned)K;
  const unsigned r0 = blockIdx.x * kObstacleBlock;
  const unsigned r = r0 + threadIdx.x;
  if (r < rows) {
    const unsigned bt = r / (unsigned)K, k = r - bt * (unsigned)K;
    const unsigned b = bt / (unsigned)T;
    const R* x = states + (size_t)bt * ls;
    const R* c = centers + ((size_t)b * K + k) * dim;
    R ss = R(0);
    for (int i = 0; i < dim; ++i) {
      const R d = x[i] - c[i];
      ss += d * d;
    }
    const R nrm = sqrt(ss);
    const R den = radii[(size_t)b * K + k] + R(kObstacleMargin);
    R* g = rowv + threadIdx.x * n;
    R gx = R(0);  // dg/dx . xbar over the position block (zero elsewhere)
    for (int j = 0; j < dim; ++j) {
      const R gj = -((x[j] - c[j]) / nrm) / den;
      g[j] = gj;
      gx += gj * x[j];
    }
    for (int j = dim; j < n; ++j) g[j] = R(0);
    const R off = (R(1) - nrm / den) - gx;
    const size_t row = (size_t)bt * m + row0 + k;
    const R lo = R(kObstacleLower) - off, hi = R(0) - off;
    l[row] = lo;
    u[row] = hi;
    qrow[threadIdx.x] = row * n;
    const size_t ri = (size_t)(bt - b * (unsigned)T) * B + b;  // the record of (t, b)
    if (rec.rv != nullptr) {
      rec.rv[ri * rec.rvp + rec.l_off + k] = lo;
      rec.rv[ri * rec.rvp + rec.u_off + k] = hi;
    }
    if (rec.am != nullptr) rrow[threadIdx.x] = ri * rec.amp + rec.g_off + (size_t)k * n;
  }
  __syncthreads();
  // the block's rows in passes of kObstacleBlock / n rows, a thread per entry
  // (n <= 64: at least two rows per pass)
  const unsigned nb = rows - r0 < (unsigned)kObstacleBlock ? rows - r0 : (unsigned)kObstacleBlock;
  const unsigned per = (unsigned)kObstacleBlock / (unsigned)n;
  const unsigned lr0 = threadIdx.x / (unsigned)n, j = threadIdx.x - lr0 * (unsigned)n;
  if (lr0 < per) {
    for (unsigned lr = lr0; lr < nb; lr += per) {
      const R v = rowv[lr * n + j];
      G[qrow[lr] + j] = v;
      if (rec.am != nullptr) rec.am[rrow[lr] + j] = v;
    }
  }
}

// One thread per stage (b, t): the position block of
// sum_k mu_k d^2 g_k / dx^2, written with the zeros of the rest of the n x n
// block.  Stage indices are 32-bit (the host checks B T < 2^31).
template <typename R>
__global__ __launch_bounds__(256) void obstacle_hessian_kernel(int B, int T, int nx, int n, int dim, int K,
                                                               const R* __restrict__ states,
                                                               const R* __restrict__ centers,
                                                               const R* __restrict__ radii, int m, int row0,
                                                               const R* __restrict__ mus, R* __restrict__ H) {
  const unsigned bt = blockIdx.x * blockDim.x + threadIdx.x;
  if (bt >= (unsigned)B * (unsigned)T) return;
  const unsigned b = bt / (unsigned)T;
  const R* x = states + (size_t)bt * nx;
  const R* mu = mus + (size_t)bt * m + row0;
  R* h = H + (size_t)bt * n * n;
  for (int i = 0; i < n; ++i) {
    for (int j = 0; j < n; ++j) {
      R v = R(0);
      if (i < dim && j < dim) {
        for (int k = 0; k < K; ++k) {
          const R* c = centers + ((size_t)b * K + k) * dim;
          R ss = R(0);
          for (int q = 0; q < dim; ++q) {
            const R d = x[q] - c[q];
            ss += d * d;
          }
          const R nrm = sqrt(ss);
          const R den = radii[(size_t)b * K + k] + R(kObstacleMargin);
          const R di = x[i] - c[i], dj = x[j] - c[j];
          const R hn = (i == j ? R(1) / nrm : R(0)) - di * dj / (nrm * nrm * nrm);
          v += mu[k] * (-hn / den);
        }
      }
      h[i * n + j] = v;
    }
  }
}

}  // namespace tmpc
