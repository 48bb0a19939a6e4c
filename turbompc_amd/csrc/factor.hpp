// Batched block-tridiagonal factorization of the ADMM Schur matrix
//
//   S = P + sigma I + rho_f C^T C + rho G^T G         (SPD, block tridiagonal)
//
// with diagonal blocks theta_t and sub-diagonal blocks phi_{t-1}
// (turbompc/solvers/admm/admm.py:88-101).  This replaces the cuDSS
// ANALYSIS/FACTORIZATION calls of the reference's direct path
// (turbompc/solvers/admm/csrc/admm_cudss.cu:1046-1053,
// turbompc/solvers/linear_systems_solvers/csrc/cudss_blktridi.cu:59-184).
//
// Factor form (block LDL^T with the stage Schur complements kept inverted):
//   Theta_0 = theta_0
//   Theta_t = theta_t - phi_{t-1} Theta_{t-1}^{-1} phi_{t-1}^T
// and the kernel stores Theta_t^{-1} (symmetric, packed lower) per stage.  The
// solves then need only matrix-vector products (admm_direct.hpp):
//   forward   w_t = Theta_t^{-1} (g_t - phi_{t-1} w_{t-1})
//   backward  x_t = w_t - Theta_t^{-1} phi_t^T x_{t+1}.
//
// One wavefront per problem; the n x n stage matrices live in LDS and the 64
// lanes stride over their entries.  Theta_t is inverted in place by
// Gauss-Jordan elimination without pivoting, which is stable for SPD input
// (and, eliminating the primal block first, for the quasi-definite adjoint
// KKT blocks of adjoint.hpp).
//
// The recursion is computed in double precision for every storage type: in
// fp32 the update theta_t - phi Theta^{-1} phi^T cancels terms of size rho_f
// |A|^2 down to the curvature of the control directions, and the factor
// would lose most of its digits.  Only the stored Theta_t^{-1} is rounded to
// the storage type; the kernel runs once per QP solve (and per rho change).
#pragma once
#include "common.hpp"

namespace tmpc {

// SRC_QP: assemble theta/phi from QP blocks.  SRC_S: read them from S blocks
// (T, n, 3n) laid out [phi_{t-1} | theta_t | phi_t^T] per block row.
enum FactorSource { SRC_QP = 0, SRC_S = 1 };

template <typename C>
__device__ void gj_invert_spd(C* A, C* rowk, C* colk, int n) {
  const int tid = threadIdx.x;
  const int nn = n * n;
  for (int k = 0; k < n; ++k) {
    if (tid < n) {
      rowk[tid] = A[k * n + tid];
      colk[tid] = A[tid * n + k];
    }
    wsync();
    const C ip = C(1) / rowk[k];
    for (int e = tid; e < nn; e += kWave) {
      const int i = e / n, j = e - (e / n) * n;
      C v;
      if (i == k && j == k)
        v = ip;
      else if (i == k)
        v = rowk[j] * ip;
      else if (j == k)
        v = -colk[i] * ip;
      else
        v = A[e] - colk[i] * rowk[j] * ip;
      A[e] = v;
    }
    wsync();
  }
}

using Cmp = double;  // compute type of the factorization

template <typename R, int SRC>
__global__ __launch_bounds__(kWave) void factor_kernel(Dims d, QPDev<R> qp,
                                                       const R* __restrict__ S,
                                                       const R* __restrict__ rho,
                                                       R sigma, R rho_f_factor,
                                                       int32_t* __restrict__ ctl,
                                                       R* __restrict__ thinv) {
  const int b = blockIdx.x;
  if (b >= d.B) return;
  if (ctl != nullptr && ctl[b * 4 + 2] == 0) return;  // refactor only when flagged
  const int tid = threadIdx.x;
  const int T = d.T, N = d.N, n = d.n, nx = d.nx, n0 = d.n0, m = d.m;
  const int nn = n * n, pk = th_pitch(n);
  extern __shared__ unsigned char smem_raw[];
  Cmp* sm = reinterpret_cast<Cmp*>(smem_raw);
  Cmp* A = sm;              // Theta_t, inverted in place
  Cmp* Ainv = A + nn;       // Theta_{t-1}^{-1}
  Cmp* ph = Ainv + nn;      // phi_{t-1}
  Cmp* tmp = ph + nn;
  Cmp* rowk = tmp + nn;
  Cmp* colk = rowk + n;
  Cmp* sG = colk + n;       // G_t        (m x n)
  Cmp* sAm = sG + m * n;    // A_minus_t  (nx x n)
  Cmp* sAp = sAm + nx * n;  // A_plus_t   (nx x n)
  Cmp* sApp = sAp + nx * n; // A_plus_{t-1}
  Cmp* sA0 = sApp + nx * n; // A0         (n0 x n)

  Cmp rho_i = 0, rho_f = 0;
  if (SRC == SRC_QP) {
    rho_i = (Cmp)rho[b];
    rho_f = rho_i * (Cmp)rho_f_factor;
    for (int e = tid; e < n0 * n; e += kWave) sA0[e] = (Cmp)qp.A0[(size_t)b * n0 * n + e];
  }
  const Cmp sig = (Cmp)sigma;

  for (int t = 0; t < T; ++t) {
    // ---- stage data and theta_t --------------------------------------------
    if (SRC == SRC_QP) {
      for (int e = tid; e < m * n; e += kWave) sG[e] = (Cmp)qp.G[((size_t)b * T + t) * m * n + e];
      if (t < N)
        for (int e = tid; e < nx * n; e += kWave) {
          sAm[e] = (Cmp)qp.Am[((size_t)b * N + t) * nx * n + e];
          sAp[e] = (Cmp)qp.Ap[((size_t)b * N + t) * nx * n + e];
        }
      wsync();
      for (int e = tid; e < nn; e += kWave) {
        const int i = e / n, j = e - (e / n) * n;
        Cmp v = (Cmp)qp.D[((size_t)b * T + t) * nn + e] + (i == j ? sig : Cmp(0));
        Cmp gg = 0;
        for (int r = 0; r < m; ++r) gg += sG[r * n + i] * sG[r * n + j];
        Cmp cc = 0;
        if (t == 0)
          for (int r = 0; r < n0; ++r) cc += sA0[r * n + i] * sA0[r * n + j];
        if (t < N)
          for (int r = 0; r < nx; ++r) cc += sAm[r * n + i] * sAm[r * n + j];
        if (t > 0)
          for (int r = 0; r < nx; ++r) cc += sApp[r * n + i] * sApp[r * n + j];
        A[e] = v + rho_i * gg + rho_f * cc;
      }
    } else {
      for (int e = tid; e < nn; e += kWave) {
        const int i = e / n, j = e - (e / n) * n;
        A[e] = (Cmp)S[(((size_t)b * T + t) * n + i) * (3 * n) + n + j];
      }
    }
    wsync();
    // ---- Theta_t = theta_t - phi_{t-1} Theta_{t-1}^{-1} phi_{t-1}^T ---------
    if (t > 0) {
      for (int e = tid; e < nn; e += kWave) {
        const int i = e / n, j = e - (e / n) * n;
        Cmp s = 0;
        for (int l = 0; l < n; ++l) s += Ainv[i * n + l] * ph[j * n + l];
        tmp[e] = s;
      }
      wsync();
      for (int e = tid; e < nn; e += kWave) {
        const int i = e / n, j = e - (e / n) * n;
        Cmp s = 0;
        for (int l = 0; l < n; ++l) s += ph[i * n + l] * tmp[l * n + j];
        A[e] -= s;
      }
      wsync();
    }
    // ---- invert and store packed ------------------------------------------
    gj_invert_spd(A, rowk, colk, n);
    wsync();
    // the computed inverse is slightly asymmetric; its symmetric part (not one
    // triangle mirrored, which at cond(Theta) ~ 1e9 breaks the inverse's small
    // residual and makes the ADMM iteration diverge) is what the solves and
    // the next Schur complement use
    R* out = thinv + ((size_t)t * d.B + b) * pk;
    for (int e = tid; e < nn; e += kWave) {
      const int i = e / n, j = e - (e / n) * n;
      const Cmp v = Cmp(0.5) * (A[e] + A[j * n + i]);
      if (j <= i) out[((i * (i + 1)) >> 1) + j] = (R)v;
      Ainv[e] = v;
    }
    wsync();
    for (int e = tid; e < nn; e += kWave) A[e] = Ainv[e];
    // ---- phi_t for the next stage ------------------------------------------
    if (t < N) {
      if (SRC == SRC_QP) {
        for (int e = tid; e < nn; e += kWave) {
          const int i = e / n, j = e - (e / n) * n;
          Cmp s = 0;
          for (int r = 0; r < nx; ++r) s += sAp[r * n + i] * sAm[r * n + j];
          ph[e] = (Cmp)qp.E[((size_t)b * N + t) * nn + e] + rho_f * s;
        }
        for (int e = tid; e < nx * n; e += kWave) sApp[e] = sAp[e];
      } else {
        for (int e = tid; e < nn; e += kWave) {
          const int i = e / n, j = e - (e / n) * n;
          ph[e] = (Cmp)S[(((size_t)b * T + t + 1) * n + i) * (3 * n) + j];
        }
      }
    }
    wsync();
  }
  if (ctl != nullptr && tid == 0) ctl[b * 4 + 2] = 0;
}

inline size_t factor_smem_bytes(const Dims& d) {
  const size_t n = d.n;
  return sizeof(Cmp) * (4 * n * n + 2 * n + (size_t)d.m * n + 3 * (size_t)d.nx * n + (size_t)d.n0 * n);
}

}  // namespace tmpc
