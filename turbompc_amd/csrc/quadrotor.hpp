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

// Hyper-dual numbers v + a e1 + b e2 + c e1 e2 (e1^2 = e2^2 = 0): seeding e1
// along z_i and e2 along z_j, the e1 e2 part of f(z) is d^2 f / dz_i dz_j.
template <typename R>
struct HDual {
  R v, a, b, c;
  __device__ HDual() = default;
  __device__ HDual(R x, R da = R(0), R db = R(0), R dab = R(0)) : v(x), a(da), b(db), c(dab) {}
};
template <typename R>
__device__ __forceinline__ HDual<R> operator+(HDual<R> x, HDual<R> y) { return {x.v + y.v, x.a + y.a, x.b + y.b, x.c + y.c}; }
template <typename R>
__device__ __forceinline__ HDual<R> operator-(HDual<R> x, HDual<R> y) { return {x.v - y.v, x.a - y.a, x.b - y.b, x.c - y.c}; }
template <typename R>
__device__ __forceinline__ HDual<R> operator-(HDual<R> x) { return {-x.v, -x.a, -x.b, -x.c}; }
template <typename R>
__device__ __forceinline__ HDual<R> operator*(HDual<R> x, HDual<R> y) {
  return {x.v * y.v, x.a * y.v + x.v * y.a, x.b * y.v + x.v * y.b, x.c * y.v + x.a * y.b + x.b * y.a + x.v * y.c};
}
template <typename R>
__device__ __forceinline__ HDual<R> operator*(R s, HDual<R> x) { return {s * x.v, s * x.a, s * x.b, s * x.c}; }

template <typename R>
struct QuadParams {
  R mass, Jx, Jy, Jz, arm, kyaw, g;
};

// Continuous dynamics, for any of the number types above (D built from R).
template <typename R, typename D>
__device__ __forceinline__ void quad_xdot(const D* x, const D* f, const QuadParams<R>& P, D* xd) {
  const R dd = P.arm * R(0.70710678118654752440);
  const R im = R(1) / P.mass;
  const D qw = x[3], qx = x[4], qy = x[5], qz = x[6];
  const D wx = x[10], wy = x[11], wz = x[12];
  const D F = f[0] + f[1] + f[2] + f[3];
  const D tx = dd * (f[0] + f[1] - f[2] - f[3]);
  const D ty = dd * ((f[1] + f[2]) - (f[0] + f[3]));
  const D tz = P.kyaw * ((f[1] + f[3]) - (f[0] + f[2]));
  xd[0] = x[7];
  xd[1] = x[8];
  xd[2] = x[9];
  xd[3] = R(0.5) * (-(qx * wx) - qy * wy - qz * wz);
  xd[4] = R(0.5) * (qw * wx + qy * wz - qz * wy);
  xd[5] = R(0.5) * (qw * wy - qx * wz + qz * wx);
  xd[6] = R(0.5) * (qw * wz + qx * wy - qy * wx);
  xd[7] = (R(2) * im) * ((qx * qz + qw * qy) * F);
  xd[8] = (R(2) * im) * ((qy * qz - qw * qx) * F);
  xd[9] = im * ((D(R(1)) - R(2) * (qx * qx + qy * qy)) * F) - D(P.g);
  xd[10] = (R(1) / P.Jx) * (tx - (P.Jz - P.Jy) * (wy * wz));
  xd[11] = (R(1) / P.Jy) * (ty - (P.Jx - P.Jz) * (wz * wx));
  xd[12] = (R(1) / P.Jz) * (tz - (P.Jy - P.Jx) * (wx * wy));
}

// Optional second destination of the blocks: the streaming solve's stage
// records (M record of (t, b) at am + (t B + b) amp with rows of 17, c_t at
// offset c_off of the rv record), so that an SQP step needs no copy of them.
template <typename R>
struct QuadRecOut {
  R* am = nullptr;  // null: the QP layout only
  R* rv = nullptr;
  int amp = 0, rvp = 0, c_off = 0;
};

template <typename R>
__global__ __launch_bounds__(256) void quad_linearize_kernel(int B, int N, const R* __restrict__ states, int ls,
                                                             const R* __restrict__ controls, int lu, R dt,
                                                             QuadParams<R> P, R* __restrict__ Am,
                                                             R* __restrict__ c, QuadRecOut<R> rec) {
  const long long gidx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long pairs = (long long)B * N;
  if (gidx >= pairs * 18) return;
  const long long pr = gidx / 18;
  const int j = (int)(gidx - pr * 18);
  const int b = (int)(pr / N), t = (int)(pr - (long long)b * N);
  const int T = N + 1;
  const R* xs = states + ((size_t)b * T + t) * ls;  // rows of ls (>= 13) and lu (>= 4) elements
  const R* us = controls + ((size_t)b * T + t) * lu;
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
  const size_t ri = (size_t)t * B + b;  // the stage record of (t, b)
#pragma unroll
  for (int k = 0; k < 13; ++k) {
    const Dual<R> xn = x[k] + (R(1) / R(6)) * ((k1[k] + R(2) * k2[k] + R(2) * k3[k] + k4[k]) * Dual<R>(dt));
    if (j < 17) {
      A[k * 17 + j] = xn.d;
      if (rec.am != nullptr) rec.am[ri * rec.amp + k * 17 + j] = xn.d;
    } else {
      const R ck = xn.d - xn.v;
      c[((size_t)b * N + t) * 13 + k] = ck;
      if (rec.rv != nullptr) rec.rv[ri * rec.rvp + rec.c_off + k] = ck;
    }
  }
}

// The RK4 step itself (predict_next_state for the explicit scheme, as used by
// equality_constraints, turbompc/problems/optimal_control_problem.py:841-912):
// next[b][t] = x_t + dt/6 (k1 + 2 k2 + 2 k3 + k4), one thread per (b, t < N).
template <typename R>
__global__ __launch_bounds__(256) void quad_step_kernel(int B, int N, const R* __restrict__ states,
                                                        const R* __restrict__ controls, R dt, QuadParams<R> P,
                                                        R* __restrict__ next) {
  const long long pr = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (pr >= (long long)B * N) return;
  const int b = (int)(pr / N), t = (int)(pr - (long long)b * N);
  const int T = N + 1;
  const R* xs = states + ((size_t)b * T + t) * 13;
  const R* us = controls + ((size_t)b * T + t) * 4;
  R x[13], u[4], k1[13], k2[13], k3[13], k4[13], tmp[13];
#pragma unroll
  for (int k = 0; k < 13; ++k) x[k] = xs[k];
#pragma unroll
  for (int k = 0; k < 4; ++k) u[k] = us[k];
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
  R* o = next + (size_t)pr * 13;
#pragma unroll
  for (int k = 0; k < 13; ++k) o[k] = x[k] + (R(1) / R(6)) * ((k1[k] + R(2) * k2[k] + R(2) * k3[k] + k4[k]) * dt);
}

// Lagrangian Hessian of the dynamics rows, get_dynamics_lagrangian_hessian for
// explicit schemes (turbompc/problems/optimal_control_problem.py:1334-1441):
//   H_t = d^2 / dz_t^2 [lambda_t . f(z_t)],  t < N;   H_N = 0,
// with f the RK4 step above.  Thread (pair, p) evaluates the step once in
// hyper-dual numbers for one entry (i, j), i <= j, of the 17 x 17 block and
// writes it to (i, j) and (j, i).
template <typename R>
__global__ __launch_bounds__(256) void quad_lag_hessian_kernel(int B, int N, const R* __restrict__ states,
                                                               const R* __restrict__ controls, R dt,
                                                               QuadParams<R> P, const R* __restrict__ lambdas,
                                                               R* __restrict__ H) {
  constexpr int n = 17, NP = n * (n + 1) / 2;
  const long long gidx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int T = N + 1;
  if (gidx >= (long long)B * T * NP) return;
  const long long pr = gidx / NP;
  int e = (int)(gidx - pr * NP);
  int i = 0;
  while (e >= n - i) {
    e -= n - i;
    ++i;
  }
  const int j = i + e;
  const int b = (int)(pr / T), t = (int)(pr - (long long)b * T);
  R* Hb = H + ((size_t)b * T + t) * n * n;
  if (t == N) {
    Hb[i * n + j] = R(0);
    Hb[j * n + i] = R(0);
    return;
  }
  const R* xs = states + ((size_t)b * T + t) * 13;
  const R* us = controls + ((size_t)b * T + t) * 4;
  HDual<R> x[13], u[4];
#pragma unroll
  for (int k = 0; k < 13; ++k) x[k] = HDual<R>(xs[k], k == i ? R(1) : R(0), k == j ? R(1) : R(0));
#pragma unroll
  for (int k = 0; k < 4; ++k) u[k] = HDual<R>(us[k], 13 + k == i ? R(1) : R(0), 13 + k == j ? R(1) : R(0));
  HDual<R> k1[13], k2[13], k3[13], k4[13], tmp[13];
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
  const R* lam = lambdas + ((size_t)b * N + t) * 13;
  R h = R(0);
#pragma unroll
  for (int k = 0; k < 13; ++k) {
    const HDual<R> xn = x[k] + (R(1) / R(6)) * ((k1[k] + R(2) * k2[k] + R(2) * k3[k] + k4[k]) * HDual<R>(dt));
    h += lam[k] * xn.c;
  }
  Hb[i * n + j] = h;
  Hb[j * n + i] = h;
}

}  // namespace tmpc
