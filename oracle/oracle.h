/*
 * TEST INFRASTRUCTURE ONLY — CPU oracle for the batched ADMM / Schur / adjoint path.
 *
 * This library restates, on the CPU, the reference's pure-JAX solver path
 * (TurboMPC `ADMM_JAX_LOOP_*` backends and the dense backward KKT).  Only the
 * test suite, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may
 * load it, and only as the checker / the timed CPU baseline: the product path
 * (`turbompc_amd`) never links or calls it.
 *
 * Layout: every array is batched with a leading problem axis B and row-major
 * per problem, exactly the layout the reference's FFI calls receive under
 * `vmap(..., vmap_method="broadcast_all")`:
 *   D (B,T,n,n)  E (B,N,n,n)  q (B,T,n)  A0 (B,n0,n)  A_minus/A_plus (B,N,nx,n)
 *   G (B,T,m,n)  l/u (B,T,m)  c0 (B,n0)  c (B,N,nx)
 *   state: x (B,T,n)  z_g/y_g/xi_g (B,T,m)  y_f_0 (B,n0)  y_f_dyn (B,N,nx)  rho (B)
 * with T = N + 1 stages and n = nx + nu.  `dtype` is 4 (float) or 8 (double);
 * all arithmetic is carried out in that type.
 *
 * Parity status of each function is listed in oracle.cpp next to it.
 */
#ifndef TMPC_ORACLE_H
#define TMPC_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ora_dims {
  int32_t B, T, n, nx, n0, m;
} ora_dims;

typedef struct ora_qp {
  const void *D, *E, *q, *A0, *A_minus, *A_plus, *G, *l, *u, *c0, *c;
  double slack_weight;
  int32_t use_slack;
} ora_qp;

typedef struct ora_state {
  void *x, *z_g, *y_g, *y_f0, *y_f, *xi_g, *rho;
} ora_state;

typedef struct ora_cfg {
  int32_t max_iter, check_every, adapt_rho_every, pcg_max_iter;
  double sigma, eps_abs, eps_rel, rho_min, rho_max, adaptive_rho_tolerance,
      rho_f_factor, alpha, pcg_eps;
} ora_cfg;

/* ADMM JAX-loop restatement.  schur: 0 = exact Schur solve (block Cholesky),
 * 1 = PCG with the reference's block preconditioner.  iters[B] receives the
 * ADMM iteration count, pcg_iters[B] (may be NULL) the summed PCG iterations. */
int ora_admm_solve(int dtype, int schur, const ora_dims* d, const ora_qp* qp,
                   const ora_state* in, ora_state* out, int32_t* iters,
                   int32_t* pcg_iters, const ora_cfg* cfg, int nthreads);

/* compute_S_Phiinv for every problem with its own rho[b]. S, Phiinv: (B,T,n,3n). */
int ora_schur_build(int dtype, const ora_dims* d, const ora_qp* qp, const void* rho,
                    double sigma, double rho_f_factor, void* S, void* Phiinv,
                    int nthreads);

/* Schur-only PCG on (S, Phiinv, rhs, x0) -> x, iters. */
int ora_pcg(int dtype, int B, int T, int n, const void* S, const void* Phiinv,
            const void* rhs, const void* x0, void* x, int32_t* iters, double eps,
            int32_t max_iter, int nthreads);

/* Exact solve S x = rhs of a block-tridiagonal SPD system (block Cholesky). */
int ora_blktri_solve(int dtype, int B, int T, int n, const void* S, const void* rhs,
                     void* x, int nthreads);

/* Dense backward KKT: qp->G is the signed active-row matrix G_act, qp->q the
 * adjoint linear term.  dz (B,T,n), mult (B, n0 + N*nx + T*m). */
int ora_adjoint_kkt(int dtype, const ora_dims* d, const ora_qp* qp, void* dz,
                    void* mult, int nthreads);

/* Quadrotor (13 states, 4 rotor thrusts) RK4 step and its Jacobian by
 * complex-step differentiation, for K (state, control) pairs (double only).
 * xu (K,17) -> f (K,13), J (K,13,17). */
int ora_quadrotor_rk4_jac(int K, const double* xu, double dt, const double* params,
                          double* f, double* J, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
