// Adjoint (backward) KKT in stage-block form.
//
// The reference solves, per problem (turbompc/solvers/backward/backward_kkt_jax.py:10-211,
// or through cuDSS on one merged CSR matrix, backward_kkt_cudss_ffi.py:329-401):
//   [ P   C^T  G_act^T ] [dz  ]   [-q]
//   [ C    0     0     ] [y   ] = [ 0]
//   [G_act 0   -eps I_inactive] [mu] [ 0]
// Here the unknowns are regrouped by stage, w_t = [z_t (n) | lambda_t (p) | mu_t (m)]
// with p = max(n0, nx): lambda_0 are the multipliers of the A0 rows, lambda_t
// (t >= 1) those of dynamics row t-1 (which couples z_{t-1} and z_t), mu_t those
// of the G_act rows of stage t.  In this order the KKT matrix is block
// tridiagonal with blocks of size nb = n + p + m:
//   diag  K_tt  = [[D_t, Chat_t^T], [Chat_t, 0]],  Chat_t = [A0 | A_plus_{t-1}; G_act_t]
//   below K_t,t-1 = [[E_{t-1}, 0], [A_minus_{t-1} (lambda rows), 0]]
// so the same block-tridiagonal factorization (factor.hpp, SRC_S) and sweeps
// (blktri_solve_kernel) that solve the ADMM Schur system solve it.  A small
// shift (+s I on z, -s I on the active multipliers, s = reg * max|D|) makes
// every stage block quasi-definite, which Gauss-Jordan without pivoting
// factors stably when the primal rows are eliminated first; iterative
// refinement against the unshifted matrix removes the shift.  Padding rows
// and inactive G_act rows carry -1 on the diagonal and no coupling, so their
// multipliers are exactly zero (the reference's -1e-12 rows).
#pragma once
#include "admm_direct.hpp"
#include "common.hpp"

namespace tmpc {

struct KktDims {
  int B, T, N, n, nx, n0, m, p, nb;
};

template <typename R>
__global__ void kkt_scale_kernel(KktDims k, const R* __restrict__ D, R reg, R* __restrict__ shift) {
  __shared__ R red[256];
  const int b = blockIdx.x, tid = threadIdx.x;
  const size_t L = (size_t)k.T * k.n * k.n;
  R mx = R(0);
  for (size_t e = tid; e < L; e += blockDim.x) mx = rmax(mx, rabs(D[(size_t)b * L + e]));
  red[tid] = mx;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (tid < s) red[tid] = rmax(red[tid], red[tid + s]);
    __syncthreads();
  }
  if (tid == 0) shift[b] = reg * rmax(red[0], R(1));
}

// One block per (problem, stage); threads stride over the nb x 3nb block row.
template <typename R>
__global__ void kkt_assemble_kernel(KktDims k, QPDev<R> qp, const R* __restrict__ shift, R* __restrict__ K,
                                    R* __restrict__ dreg, R* __restrict__ rhs) {
  const int b = blockIdx.x / k.T, t = blockIdx.x - (blockIdx.x / k.T) * k.T;
  const int n = k.n, nx = k.nx, n0 = k.n0, m = k.m, p = k.p, nb = k.nb, N = k.N, T = k.T;
  const int w3 = 3 * nb;
  const R s = shift[b];
  R* Kt = K + ((size_t)b * T + t) * nb * w3;
  const R* Dt = qp.D + ((size_t)b * T + t) * n * n;
  const R* Gt = m ? qp.G + ((size_t)b * T + t) * m * n : nullptr;
  const int nlam = (t == 0) ? n0 : nx;
  const R* Chat = (t == 0) ? qp.A0 + (size_t)b * n0 * n : qp.Ap + ((size_t)b * N + t - 1) * nx * n;
  for (int e = threadIdx.x; e < nb * w3; e += blockDim.x) {
    const int i = e / w3, c = e - (e / w3) * w3;
    const int blk = c / nb, j = c - (c / nb) * nb;  // 0 = below, 1 = diag, 2 = above
    R v = R(0);
    if (blk == 1) {
      if (i < n && j < n) {
        v = Dt[i * n + j];
      } else if (i < n && j < n + p) {
        const int r = j - n;
        v = r < nlam ? Chat[r * n + i] : R(0);
      } else if (i < n) {
        v = Gt[(j - n - p) * n + i];
      } else if (j < n && i < n + p) {
        const int r = i - n;
        v = r < nlam ? Chat[r * n + j] : R(0);
      } else if (j < n) {
        v = Gt[(i - n - p) * n + j];
      }
    } else if (blk == 0 && t > 0) {  // K_{t,t-1}
      if (i < n && j < n)
        v = qp.E[((size_t)b * N + t - 1) * n * n + i * n + j];
      else if (i >= n && i < n + nx && j < n)
        v = qp.Am[((size_t)b * N + t - 1) * nx * n + (i - n) * n + j];
    } else if (blk == 2 && t < N) {  // K_{t,t+1} = K_{t+1,t}^T
      if (i < n && j < n)
        v = qp.E[((size_t)b * N + t) * n * n + j * n + i];
      else if (i < n && j >= n && j < n + nx)
        v = qp.Am[((size_t)b * N + t) * nx * n + (j - n) * n + i];
    }
    Kt[(size_t)i * w3 + c] = v;
  }
  __syncthreads();
  // diagonal shift / padding and the right-hand side
  for (int i = threadIdx.x; i < nb; i += blockDim.x) {
    bool pad;
    if (i < n) {
      pad = false;
    } else if (i < n + p) {
      pad = (i - n) >= nlam;
    } else {
      R nrm = R(0);
      for (int j = 0; j < n; ++j) nrm += rabs(Gt[(i - n - p) * n + j]);
      pad = !(nrm > R(0));
    }
    const R dv = pad ? R(0) : (i < n ? s : -s);
    R* diag = Kt + (size_t)i * w3 + nb + i;
    *diag = pad ? R(-1) : (*diag + dv);
    dreg[((size_t)b * T + t) * nb + i] = dv;
    rhs[((size_t)b * T + t) * nb + i] = i < n ? -qp.q[((size_t)b * T + t) * n + i] : R(0);
  }
}

// r = rhs - K_shifted x + dreg .* x  (= rhs - K_true x); g = nb lanes per problem.
template <typename R>
__global__ __launch_bounds__(kWave) void kkt_residual_kernel(KktDims k, int P, const R* __restrict__ K,
                                                             const R* __restrict__ dreg, const R* __restrict__ rhs,
                                                             const R* __restrict__ x, R* __restrict__ r) {
  __shared__ R win[3][kWave];
  const int nb = k.nb, T = k.T, w3 = 3 * nb;
  const Group G = make_group(nb, P, k.B);
  const int b = G.prob, i = G.lane, base = G.gid * nb;
  const R* X = x + (size_t)b * T * nb;
  if (i < nb) {
    win[0][base + i] = R(0);
    win[1][base + i] = X[i];
    win[2][base + i] = X[nb + i];
  }
  for (int t = 0; t < T; ++t) {
    wsync();
    if (i < nb) {
      const R* row = K + (((size_t)b * T + t) * nb + i) * w3;
      R s = R(0);
      for (int c = 0; c < nb; ++c) s += row[c] * win[0][base + c];
      for (int c = 0; c < nb; ++c) s += row[nb + c] * win[1][base + c];
      for (int c = 0; c < nb; ++c) s += row[2 * nb + c] * win[2][base + c];
      const size_t o = ((size_t)b * T + t) * nb + i;
      if (G.live) r[o] = rhs[o] - s + dreg[o] * win[1][base + i];
    }
    wsync();
    if (i < nb) {
      win[0][base + i] = win[1][base + i];
      win[1][base + i] = win[2][base + i];
      win[2][base + i] = (t + 2 < T) ? X[(size_t)(t + 2) * nb + i] : R(0);
    }
  }
}

template <typename R>
__global__ void axpy_kernel(size_t L, const R* __restrict__ dx, R* __restrict__ x) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < L) x[e] += dx[e];
}

// dz (B,T,n) and mult (B, n0 + N nx + T m) = [y_f0 | y_f_dyn | y_ineq]
template <typename R>
__global__ void kkt_unpack_kernel(KktDims k, const R* __restrict__ x, R* __restrict__ dz, R* __restrict__ mult) {
  const int b = blockIdx.x;
  const int n = k.n, nx = k.nx, n0 = k.n0, m = k.m, p = k.p, nb = k.nb, T = k.T, N = k.N;
  const R* X = x + (size_t)b * T * nb;
  const size_t L = (size_t)n0 + (size_t)N * nx + (size_t)T * m;
  for (size_t e = threadIdx.x; e < (size_t)T * n; e += blockDim.x) {
    const size_t t = e / n, i = e - (e / n) * n;
    dz[(size_t)b * T * n + e] = X[t * nb + i];
  }
  R* M = mult + (size_t)b * L;
  for (size_t e = threadIdx.x; e < L; e += blockDim.x) {
    R v;
    if (e < (size_t)n0) {
      v = X[n + e];
    } else if (e < (size_t)n0 + (size_t)N * nx) {
      const size_t q = e - n0, t = q / nx + 1, r = q - (q / nx) * nx;
      v = X[t * nb + n + r];
    } else {
      const size_t mm = m > 0 ? m : 1;
      const size_t q = e - n0 - (size_t)N * nx, t = q / mm, r = q - (q / mm) * mm;
      v = X[t * nb + n + p + r];
    }
    M[e] = v;
  }
}

}  // namespace tmpc
