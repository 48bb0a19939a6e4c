// On-device SQP linearization of the rotor-thrust quadrotor (explicit RK4).
//
// For every problem b and stage t < N this produces the dynamics blocks of
// get_dynamics_linearized_matrices for explicit schemes
// (turbompc/problems/optimal_control_problem.py:1217-1272):
//   A_minus_t = [df/dx, df/du](xbar_t, ubar_t)                (13 x 17)
//   c_t       = -f(xbar_t, ubar_t) + A xbar_t + B ubar_t       (13)
// with f the RK4 step of turbompc/dynamics/integrators.py:67-76 (control held
// over the step).  A_plus_t = [-I 0] and E = 0 are constant and not written.
//
// Jacobian columns are forward-mode directional derivatives (dual numbers):
// thread (pair, j) propagates the tangent e_j through the RK4 step, j = 0..16;
// thread j = 17 propagates the tangent zbar itself, whose derivative is exactly
// A xbar + B ubar.  Adjacent threads write adjacent columns of a row.
//
// Model: state [p(3), q(4) = (w,x,y,z), v(3), omega(3)], input four rotor
// thrusts of an x-configuration quadrotor.  params = {mass, Jxx, Jyy, Jzz,
// arm, yaw-moment coefficient, g}.
#pragma once
#include "common.hpp"

namespace tmpc {

template <typename R>
struct Dual {
  R v, d;
  __device__ Dual() = default;
  __device__ Dual(R a, R b = R(0)) : v(a), d(b) {}
};
template <typename R>
__device__ __forceinline__ Dual<R> operator+(Dual<R> a, Dual<R> b) { return {a.v + b.v, a.d + b.d}; }
template <typename R>
__device__ __forceinline__ Dual<R> operator-(Dual<R> a, Dual<R> b) { return {a.v - b.v, a.d - b.d}; }
template <typename R>
__device__ __forceinline__ Dual<R> operator-(Dual<R> a) { return {-a.v, -a.d}; }
template <typename R>
__device__ __forceinline__ Dual<R> operator*(Dual<R> a, Dual<R> b) { return {a.v * b.v, a.d * b.v + a.v * b.d}; }
template <typename R>
__device__ __forceinline__ Dual<R> operator*(R s, Dual<R> a) { return {s * a.v, s * a.d}; }

template <typename R>
struct QuadParams {
  R mass, Jx, Jy, Jz, arm, kyaw, g;
};

template <typename R>
__device__ __forceinline__ void quad_xdot(const Dual<R>* x, const Dual<R>* f, const QuadParams<R>& P,
                                          Dual<R>* xd) {
  const R dd = P.arm * R(0.70710678118654752440);
  const R im = R(1) / P.mass;
  const Dual<R> qw = x[3], qx = x[4], qy = x[5], qz = x[6];
  const Dual<R> wx = x[10], wy = x[11], wz = x[12];
  const Dual<R> F = f[0] + f[1] + f[2] + f[3];
  const Dual<R> tx = dd * (f[0] + f[1] - f[2] - f[3]);
  const Dual<R> ty = dd * ((f[1] + f[2]) - (f[0] + f[3]));
  const Dual<R> tz = P.kyaw * ((f[1] + f[3]) - (f[0] + f[2]));
  xd[0] = x[7];
  xd[1] = x[8];
  xd[2] = x[9];
  xd[3] = R(0.5) * (-(qx * wx) - qy * wy - qz * wz);
  xd[4] = R(0.5) * (qw * wx + qy * wz - qz * wy);
  xd[5] = R(0.5) * (qw * wy - qx * wz + qz * wx);
  xd[6] = R(0.5) * (qw * wz + qx * wy - qy * wx);
  xd[7] = (R(2) * im) * ((qx * qz + qw * qy) * F);
  xd[8] = (R(2) * im) * ((qy * qz - qw * qx) * F);
  xd[9] = im * ((Dual<R>(R(1)) - R(2) * (qx * qx + qy * qy)) * F) - Dual<R>(P.g);
  xd[10] = (R(1) / P.Jx) * (tx - (P.Jz - P.Jy) * (wy * wz));
  xd[11] = (R(1) / P.Jy) * (ty - (P.Jx - P.Jz) * (wz * wx));
  xd[12] = (R(1) / P.Jz) * (tz - (P.Jy - P.Jx) * (wx * wy));
}

template <typename R>
__global__ __launch_bounds__(256) void quad_linearize_kernel(int B, int N, const R* __restrict__ states,
                                                             const R* __restrict__ controls, R dt,
                                                             QuadParams<R> P, R* __restrict__ Am,
                                                             R* __restrict__ c) {
  const long long gidx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long pairs = (long long)B * N;
  if (gidx >= pairs * 18) return;
  const long long pr = gidx / 18;
  const int j = (int)(gidx - pr * 18);
  const int b = (int)(pr / N), t = (int)(pr - (long long)b * N);
  const int T = N + 1;
  const R* xs = states + ((size_t)b * T + t) * 13;
  const R* us = controls + ((size_t)b * T + t) * 4;
  Dual<R> x[13], u[4];
#pragma unroll
  for (int k = 0; k < 13; ++k) x[k] = Dual<R>(xs[k], j == 17 ? xs[k] : (j == k ? R(1) : R(0)));
#pragma unroll
  for (int k = 0; k < 4; ++k) u[k] = Dual<R>(us[k], j == 17 ? us[k] : (j == 13 + k ? R(1) : R(0)));
  Dual<R> k1[13], k2[13], k3[13], k4[13], tmp[13];
  quad_xdot(x, u, P, k1);
#pragma unroll
  for (int k = 0; k < 13; ++k) tmp[k] = x[k] + (R(0.5) * dt) * k1[k];
  quad_xdot(tmp, u, P, k2);
#pragma unroll
  for (int k = 0; k < 13; ++k) tmp[k] = x[k] + (R(0.5) * dt) * k2[k];
  quad_xdot(tmp, u, P, k3);
#pragma unroll
  for (int k = 0; k < 13; ++k) tmp[k] = x[k] + dt * k3[k];
  quad_xdot(tmp, u, P, k4);
  R* A = Am + ((size_t)b * N + t) * 13 * 17;
#pragma unroll
  for (int k = 0; k < 13; ++k) {
    const Dual<R> xn = x[k] + (R(1) / R(6)) * ((k1[k] + R(2) * k2[k] + R(2) * k3[k] + k4[k]) * Dual<R>(dt));
    if (j < 17)
      A[k * 17 + j] = xn.d;
    else
      c[((size_t)b * N + t) * 13 + k] = xn.d - xn.v;
  }
}

}  // namespace tmpc
