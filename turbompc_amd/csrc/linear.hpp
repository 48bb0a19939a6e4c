// x_{t+1} = A x_t + B u_t + b for t < N: the dynamics part of the equality
// residuals of linear problems (LinearDynamics, turbompc/dynamics/linear_dynamics.py,
// through equality_constraints, turbompc/problems/optimal_control_problem.py:841-912),
// which the merit line search evaluates at trial points.  One thread per
// (problem, stage, row); the two products are summed in order and added, then b.
#pragma once
#include "common.hpp"

namespace tmpc {

template <typename R>
__global__ __launch_bounds__(256) void linear_step_kernel(int B, int N, int nx, int nu, const R* __restrict__ states,
                                                          const R* __restrict__ controls, const R* __restrict__ A,
                                                          const R* __restrict__ Bm, const R* __restrict__ bv,
                                                          R* __restrict__ next) {
  const unsigned e = blockIdx.x * blockDim.x + threadIdx.x;  // (b, t, i), i fastest
  if (e >= (unsigned)B * (unsigned)N * (unsigned)nx) return;
  const unsigned bt = e / (unsigned)nx, i = e - bt * (unsigned)nx;
  const unsigned b = bt / (unsigned)N, t = bt - b * (unsigned)N;
  const size_t st = (size_t)b * (N + 1) + t;  // states and controls hold N + 1 stages
  const R* x = states + st * nx;
  const R* u = controls + st * nu;
  const R* a = A + ((size_t)b * nx + i) * nx;
  const R* bm = Bm + ((size_t)b * nx + i) * nu;
  R ax = R(0), bu = R(0);
  for (int j = 0; j < nx; ++j) ax += a[j] * x[j];
  for (int k = 0; k < nu; ++k) bu += bm[k] * u[k];
  next[e] = (ax + bu) + bv[(size_t)b * nx + i];
}

}  // namespace tmpc
