/*
 * libtmpc_hip — MI355X (gfx950) batched MPC solver kernels behind a C ABI.
 *
 * Every entry point is asynchronous on the caller's HIP stream, takes
 * caller-owned device buffers, allocates nothing and keeps no global state:
 * scratch memory is a caller-provided workspace whose size the matching
 * *_workspace_bytes() query returns.  Return values are tmpc_status codes;
 * nothing aborts.
 *
 * Array layout (all device pointers, row-major, leading problem axis B) is the
 * reference's batched FFI layout (turbompc/solvers/admm/admm_cudss_ffi_backend.py:131-169):
 *   D (B,T,n,n)  E (B,N,n,n)  q (B,T,n)  A0 (B,n0,n)  A_minus, A_plus (B,N,nx,n)
 *   G (B,T,m,n)  l, u (B,T,m)  c0 (B,n0)  c (B,N,nx)
 *   state: x (B,T,n)  z_g, y_g, xi_g (B,T,m)  y_f0 (B,n0)  y_f (B,N,nx)  rho (B)
 * with T = N + 1 stages and n = nx + nu.  *_f32 entry points take float
 * buffers, *_f64 double buffers.  Shapes need 1 <= n <= 64, 0 <= m <= 64,
 * 1 <= nx <= n, 1 <= n0 <= n and T >= 2.
 */
#ifndef TMPC_H
#define TMPC_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum tmpc_status {
  TMPC_OK = 0,
  TMPC_EBADSHAPE = 1,  /* dimensions outside the supported range          */
  TMPC_EBADARG = 2,    /* null pointer or invalid configuration value     */
  TMPC_EWORKSPACE = 3, /* workspace smaller than *_workspace_bytes()      */
  TMPC_ELAUNCH = 4,    /* a HIP launch or copy failed                     */
  TMPC_ESCRATCH = 5,   /* the problem needs more scratch than the
                          allocation-free entry point holds               */
  TMPC_ENONFINITE = 6  /* a solution holds NaN or infinity: never returned
                          by the asynchronous entry points, which flag it
                          per problem in iters_out (TMPC_ITERS_NONFINITE);
                          for host layers that turn the flag into an error */
} tmpc_status;

/* Bit 31 of iters_out[b] (tmpc_admm_direct_*, tmpc_sqp_admm_step_*,
 * tmpc_admm_pcg_*, tmpc_admm_direct_noalloc): set when problem b's output
 * state (x, z_g, y_g, xi_g, y_f0, y_f or rho) holds a NaN or an infinity.
 * The iteration count is iters_out[b] & 0x7fffffff. */
#define TMPC_ITERS_NONFINITE 0x80000000u

typedef struct tmpc_dims {
  int32_t B, T, n, nx, n0, m;
} tmpc_dims;

typedef struct tmpc_qp {
  const void *D, *E, *q, *A0, *A_minus, *A_plus, *G, *l, *u, *c0, *c;
  const void* slack_weight; /* (B,) slack penalty per problem, or NULL (0)   */
} tmpc_qp;

typedef struct tmpc_state {
  void *x, *z_g, *y_g, *y_f0, *y_f, *xi_g, *rho;
} tmpc_state;

/* Structure the caller vouches for: A_plus_t == [-I 0] and E_t == 0 for all t
 * (explicit integrators without a control-rate cost).  Lets the solve skip
 * reading A_plus and E. */
#define TMPC_FLAG_STD_DYNAMICS 1u
/* With TMPC_FLAG_STD_DYNAMICS the direct solve streams stage records through
 * a batched kernel when the shape allows it: n <= 17 and nx < n, with the
 * records' block width w the smallest of 6, 9, 16, 17 that is >= n and holds
 * nx + m <= w with m <= 8 (or a wide form: w = 9 with nx + m <= 17 and
 * m <= 12, w = 16 with nx + m <= 32 and m <= 28); for
 * n < w the records carry w - n decoupled dummy variables, which never reach
 * the state.  TMPC_FLAG_GENERIC_KERNEL selects the generic per-stage kernel
 * instead (same iteration; for cross-checks).  Bits 8-9 force the number of
 * problems per wavefront of the streaming kernel (1-3; 0 = chosen from B). */
#define TMPC_FLAG_GENERIC_KERNEL 2u
#define TMPC_FLAG_STREAM_P(p) (((uint32_t)(p) & 3u) << 8)
/* tmpc_admm_pcg_* with TMPC_FLAG_STD_DYNAMICS runs the whole solve in one
 * launch, one problem per workgroup, when the shape allows it: the
 * row-broadcast kernel (n in {6, 9, 16}, 16 T <= 1024, T m <= 1024), else the
 * LDS-resident kernel (n in {6, 9, 16, 17}, T n <= 1024, T m <= 1024), else
 * (or with TMPC_FLAG_GENERIC_KERNEL) the chunked kernel that streams S and
 * Phiinv.  Bits 10-11 force one of them (1 = row-broadcast, 2 = LDS-resident,
 * 3 = chunked; TMPC_EBADSHAPE if it does not cover the shape), for
 * cross-checks. */
#define TMPC_FLAG_PCG_KERNEL(k) (((uint32_t)(k) & 3u) << 10)
/* The direct solve's factorization of the explicit-integrator Schur blocks
 * runs one problem per 16-lane row (four per wavefront); this flag selects
 * the factorization with P problems per wavefront in lane groups and LDS
 * pivot rows instead (same blocks; for cross-checks). */
#define TMPC_FLAG_FACTOR_GROUPS (1u << 12)
/* Every D_t is diagonal (quadratic costs with per-variable weights), vouched
 * for by the caller.  The streaming kernel then keeps diag(D_t) in its stage
 * records and forms the D_t x terms from it, and the first-order check reads
 * only the diagonal: the same products term by term (ignored by the other
 * paths). */
#define TMPC_FLAG_DIAG_COST 4u
/* Warm stage records (streaming path of tmpc_admm_direct_* and
 * tmpc_sqp_admm_step_*): the workspace holds the stage records of the previous
 * call, whose output state is this call's input state, and this QP differs from
 * that call's only in A_minus and c (an SQP iteration relinearizing explicit
 * dynamics: D, E, q, G, l, u, A0, c0 and the slack weight are unchanged).  Only
 * the A_minus and c records are rewritten.  Vouched for by the caller; the
 * other paths ignore it. */
#define TMPC_FLAG_WARM_RECORDS 8u
/* With TMPC_FLAG_WARM_RECORDS: the QP also differs from the previous call's in
 * G, l and u (inequality rows relinearized at the new iterate, as the obstacle
 * rows are), whose records are rewritten too; D, E, q, A0, c0 and the slack
 * weight are still unchanged. */
#define TMPC_FLAG_WARM_INEQ 16u
/* With TMPC_FLAG_WARM_RECORDS: A_minus and c are the previous call's as well
 * (linear dynamics), so the records keep them and only what else changed
 * (G, l, u with TMPC_FLAG_WARM_INEQ) is rewritten. */
#define TMPC_FLAG_WARM_SAME_DYNAMICS (1u << 13)
/* Every G_t is the same for every stage and problem (box rows of a tracking
 * problem), vouched for by the caller.  The streaming kernel for n = 17
 * records then keeps the G rows of its stage blocks in LDS and streams only
 * the A_minus rows of the stage records in its backward sweep, as in its
 * forward sweep (fewer bytes per iteration; the same products, so the same
 * iterates bit for bit).  Ignored by the other paths and shapes. */
#define TMPC_FLAG_CONST_G 32u
/* With TMPC_FLAG_CONST_G on the same n = 17 records (nx n <= 224, at most two
 * problems per wavefront, a workspace of the size
 * tmpc_admm_direct_workspace_bytes reports): the entries of A_minus_t that are
 * the same, bit for bit, in every stage t < N of a problem (found on the
 * device on every call; a rigid body's position and velocity columns, for
 * example) stay in LDS, and both sweeps stream only the others (the same
 * products, so the same iterates bit for bit).  Needs no promise from the
 * caller; ignored by the other paths and shapes. */
#define TMPC_FLAG_INVARIANT_A 64u

typedef struct tmpc_admm_cfg {
  int32_t max_iter, check_every, adapt_rho_every, pcg_max_iter, use_slack;
  uint32_t flags;
  double sigma, eps_abs, eps_rel, rho_min, rho_max, adaptive_rho_tolerance,
      rho_f_factor, alpha, pcg_eps;
} tmpc_admm_cfg;

const char* tmpc_status_string(int status);
int tmpc_version(void);

/* Measurement hook (no counterpart in the reference): while set, every
 * tmpc_admm_direct_* / tmpc_sqp_admm_step_* / tmpc_admm_pcg_* call records
 * `before` on its stream right before its ADMM-iteration phase (the iteration
 * kernels and any refactorizations or Schur rebuilds between chunks) and
 * `after` right after it, so the caller can time that phase alone with
 * hipEventElapsedTime.  NULL, NULL switches it off.  The
 * setting is process-wide and not synchronised: set it from the thread that
 * launches the solves. */
void tmpc_set_timing_events(hipEvent_t before, hipEvent_t after);

/* ---- zero fill by a kernel ---------------------------------------------------
 * No counterpart in the reference: for bindings that must zero a result the
 * reference writes as zero (kernel_ns of the fused ADMM targets,
 * turbompc/solvers/admm/csrc/admm_cudss.cu:1189-1197) without recording a
 * memset node into a captured HIP graph.  p and bytes must be multiples of 4
 * (TMPC_EBADARG otherwise); bytes = 0 does nothing. */
int tmpc_fill_zero(hipStream_t stream, void* p, size_t bytes);

/* ---- ADMM with the exact block-tridiagonal Schur solve ---------------------
 * Replaces the `admm_cudss_cuda[_f64]` FFI target: AdmmCudssCudaImpl
 * (turbompc/solvers/admm/csrc/admm_cudss_ffi.cc:13-140) / launchADMMCudss
 * (turbompc/solvers/admm/csrc/admm_cudss.cu:853-1199), with the semantics of
 * the reference's pure-JAX loop (turbompc/solvers/admm/admm.py:795-1049).
 * `in` is the warm start; `out` receives the final state (in == out allowed).
 * iters_out (B,) uint32 receives the ADMM iteration count per problem, with
 * TMPC_ITERS_NONFINITE set for a problem whose final state is not finite.
 * The workspace size reported covers every form; TMPC_FLAG_INVARIANT_A needs
 * all of it, the rest of the solve runs in less (the stage records and the
 * factor, without the compressed A_minus runs of that form). */
size_t tmpc_admm_direct_workspace_bytes(int elem_bytes, const tmpc_dims* dims);
int tmpc_admm_direct_f32(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                         const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                         const tmpc_admm_cfg* cfg, void* workspace, size_t workspace_bytes);
int tmpc_admm_direct_f64(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                         const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                         const tmpc_admm_cfg* cfg, void* workspace, size_t workspace_bytes);

/* ---- allocation-free variant of tmpc_admm_direct_* -------------------------
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory or pass a workspace: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Same solve as
 * tmpc_admm_direct_f32 (elem_bytes 4) / _f64 (elem_bytes 8), with the
 * workspace taken from a scratch array of TMPC_NOALLOC_SCRATCH_BYTES that the
 * library holds on each GPU it runs on until the process ends; the call
 * itself allocates nothing.  A problem batch whose workspace
 * (tmpc_admm_direct_workspace_bytes) exceeds that size is rejected with
 * TMPC_ESCRATCH.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (different streams or host threads) race, so serialise
 * them.  TMPC_FLAG_WARM_RECORDS is rejected (TMPC_EBADARG), since the shared
 * array cannot vouch for the previous call's records.  `stream` must belong
 * to the current device. */
#define TMPC_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int tmpc_admm_direct_noalloc(hipStream_t stream, int elem_bytes, const tmpc_dims* dims, const tmpc_qp* qp,
                             const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                             const tmpc_admm_cfg* cfg);

/* ---- one SQP step on the device --------------------------------------------
 * The body of the reference's SQP while_loop (turbompc/solvers/turbompc_solver.py:1570-1711)
 * evaluates _compute_first_order_convergence_error (:1158-1225) on the new
 * iterate and its relinearized QP; the next test of cond_fun (conv >
 * tol_convergence per problem under vmap, :1713-1718) is followed by
 * ADMMSolver.solve of that same QP from that same iterate (:1575-1581).
 * This entry point does the three in one call: the check of `in` against
 * `qp` (fused into the first sweep of the ADMM kernel on the explicit-
 * integrator path), the activity test, and the ADMM solve of the problems
 * that pass it.  A problem that fails it runs no iteration: `out` keeps `in`
 * and iters_out is 0, so the caller needs no masked commit.  The workspace is
 * the one of tmpc_admm_direct_*.
 * With conv NULL the activity is given: no check is evaluated (eq_err,
 * ineq_err and g_out must be NULL too), active_out = active_in, and the
 * problems with active_in = 0 run no iteration (for callers whose iterate is
 * not the ADMM state's x, such as the merit line search's blend). */
typedef struct {
  const uint8_t* active_in; /* (B,) 1 = still iterating, or NULL = all */
  uint8_t* active_out;      /* (B,) active_in && conv > tol (may alias active_in) */
  double tol;               /* tol_convergence */
  void* conv;               /* (B,) first-order error of `in`, or NULL: activity given */
  void* eq_err;             /* (B,) equality violation, or NULL */
  void* ineq_err;           /* (B,) inequality violation, or NULL */
  void* g_out;              /* (B,T,m) G x (+ slack) of `in`, or NULL */
} tmpc_sqp_step;
int tmpc_sqp_admm_step_f32(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                           const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                           const tmpc_admm_cfg* cfg, const tmpc_sqp_step* sqp, void* workspace,
                           size_t workspace_bytes);
int tmpc_sqp_admm_step_f64(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                           const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                           const tmpc_admm_cfg* cfg, const tmpc_sqp_step* sqp, void* workspace,
                           size_t workspace_bytes);

/* The same SQP step for the rotor-thrust quadrotor (n = 17, nx = 13), which
 * also builds the QP's dynamics rows: qp->A_minus (B,N,13,17) and qp->c
 * (B,N,13) are OUTPUTS, written first with the RK4 linearization of
 * tmpc_quadrotor_linearize_* at the input iterate (the rows [x_t; u_t] of
 * in->x; dt and the 7 model parameters as there).  With
 * TMPC_FLAG_WARM_RECORDS the same values go straight into the workspace's
 * stage records on the streaming path, so the step copies no dynamics rows
 * from the QP layout.  This fuses the linearization
 * of the next SQP iteration (turbompc/solvers/turbompc_solver.py:1098-1156,
 * optimal_control_problem.py:1217-1272) into the step that consumes it. */
int tmpc_sqp_admm_step_quadrotor_f32(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                                     const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                                     const tmpc_admm_cfg* cfg, const tmpc_sqp_step* sqp, double dt,
                                     const double* params, void* workspace, size_t workspace_bytes);
int tmpc_sqp_admm_step_quadrotor_f64(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                                     const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                                     const tmpc_admm_cfg* cfg, const tmpc_sqp_step* sqp, double dt,
                                     const double* params, void* workspace, size_t workspace_bytes);

/* The same SQP step for a QP with K spherical obstacle rows (rows row0 ..
 * row0 + K - 1 of every stage; centers (B,K,dim), radii (B,K) as in
 * tmpc_obstacle_linearize_*), which also builds those rows: they are OUTPUTS
 * of qp->G, qp->l and qp->u, written first with the linearization of
 * tmpc_obstacle_linearize_* at the input iterate (the first dim entries of
 * the rows of in->x); the other rows of G, l and u are inputs.  With
 * TMPC_FLAG_WARM_RECORDS the same values go straight into the workspace's
 * stage records on the streaming path, and the other rows of G, l and u must
 * then be the previous call's (the records keep them).  This fuses the
 * obstacle linearization of the next SQP iteration
 * (turbompc/solvers/turbompc_solver.py:1098-1156,
 * optimal_control_problem.py:580-626) into the step that consumes it. */
int tmpc_sqp_admm_step_obstacle_f32(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                                    const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                                    const tmpc_admm_cfg* cfg, const tmpc_sqp_step* sqp, int32_t dim, int32_t K,
                                    const float* centers, const float* radii, int32_t row0, void* workspace,
                                    size_t workspace_bytes);
int tmpc_sqp_admm_step_obstacle_f64(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                                    const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                                    const tmpc_admm_cfg* cfg, const tmpc_sqp_step* sqp, int32_t dim, int32_t K,
                                    const double* centers, const double* radii, int32_t row0, void* workspace,
                                    size_t workspace_bytes);

/* ---- ADMM with the PCG Schur solve -----------------------------------------
 * Replaces the `admm_fused_cuda[_f64]` FFI target: AdmmFusedCudaImpl
 * (turbompc/solvers/admm/csrc/admm_ffi.cc:13-148) / LaunchADMMFusedF32/F64
 * (turbompc/solvers/admm/csrc/admm_fused.cuh:25-120), with the semantics of the
 * reference's JAX loop over PCGPrimalOptimalControl
 * (turbompc/solvers/linear_systems_solvers/pcg_primal.py:70-175): S and the
 * block preconditioner Phiinv are built on the device (compute_S_Phiinv), PCG
 * is warm-started at the previous x, cfg->pcg_eps / cfg->pcg_max_iter control
 * it.  pcg_iters_out (B, max_iter) uint32 may be NULL; otherwise it receives
 * the PCG iteration count of every ADMM iteration (zero past the last). */
size_t tmpc_admm_pcg_workspace_bytes(int elem_bytes, const tmpc_dims* dims);
int tmpc_admm_pcg_f32(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                      const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                      uint32_t* pcg_iters_out, const tmpc_admm_cfg* cfg, void* workspace,
                      size_t workspace_bytes);
int tmpc_admm_pcg_f64(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                      const tmpc_state* in, tmpc_state* out, uint32_t* iters_out,
                      uint32_t* pcg_iters_out, const tmpc_admm_cfg* cfg, void* workspace,
                      size_t workspace_bytes);

/* ---- Schur matrix and block preconditioner ---------------------------------
 * Replaces compute_S_Phiinv (turbompc/solvers/admm/admm.py:71-154), which the
 * reference evaluates in XLA before every fused solve: rho (B,) per problem,
 * rho_f = rho * rho_f_factor.  S, Phiinv (B,T,n,3n). */
int tmpc_schur_build_f32(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                         const float* rho, double sigma, double rho_f_factor, float* S,
                         float* Phiinv);
int tmpc_schur_build_f64(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp,
                         const double* rho, double sigma, double rho_f_factor, double* S,
                         double* Phiinv);

/* ---- Schur-level PCG ---------------------------------------------------------
 * Replaces `pcg_blktridi_cuda[_f64]` (LaunchPcgBlkTridiF32/F64,
 * turbompc/solvers/linear_systems_solvers/csrc/pcg_blktridi.cuh:7-33):
 * S, Phiinv (B,T,n,3n), rhs, x0 (B,T,n) -> x (B,T,n) (x != x0), iters (B,). */
size_t tmpc_schur_pcg_workspace_bytes(int elem_bytes, int32_t B, int32_t T, int32_t n);
int tmpc_schur_pcg_f32(hipStream_t stream, int32_t B, int32_t T, int32_t n, const float* S,
                       const float* Phiinv, const float* rhs, const float* x0, float* x,
                       uint32_t* iters, double eps, int32_t max_iter, void* workspace,
                       size_t workspace_bytes);
int tmpc_schur_pcg_f64(hipStream_t stream, int32_t B, int32_t T, int32_t n, const double* S,
                       const double* Phiinv, const double* rhs, const double* x0, double* x,
                       uint32_t* iters, double eps, int32_t max_iter, void* workspace,
                       size_t workspace_bytes);

/* ---- Schur-level direct solve ----------------------------------------------
 * Replaces `cudss_blktridi_cuda[_f64]` (CudssBlkTridiSolveF32/F64,
 * turbompc/solvers/linear_systems_solvers/csrc/cudss_blktridi.cuh:5-21):
 * S (B,T,n,3n) block rows [prev | diag | next] of an SPD block-tridiagonal
 * matrix, rhs (B,T,n) -> x (B,T,n).  The factor (workspace) can be reused by
 * further tmpc_blktri_solve_* calls with the same S. */
size_t tmpc_blktri_workspace_bytes(int elem_bytes, int32_t B, int32_t T, int32_t n);
int tmpc_blktri_factor_f32(hipStream_t stream, int32_t B, int32_t T, int32_t n, const float* S,
                           void* workspace, size_t workspace_bytes);
int tmpc_blktri_factor_f64(hipStream_t stream, int32_t B, int32_t T, int32_t n, const double* S,
                           void* workspace, size_t workspace_bytes);
int tmpc_blktri_solve_f32(hipStream_t stream, int32_t B, int32_t T, int32_t n, const float* S,
                          const float* rhs, float* x, const void* workspace, size_t workspace_bytes);
int tmpc_blktri_solve_f64(hipStream_t stream, int32_t B, int32_t T, int32_t n, const double* S,
                          const double* rhs, double* x, const void* workspace,
                          size_t workspace_bytes);

/* ---- Adjoint (backward) KKT solve ------------------------------------------
 * Replaces `cudss_sparse_kkt_f32/f64` (solve_sparse_kkt_f32/f64,
 * turbompc/solvers/backward/csrc/cudss_sparse_kkt.cuh:21-41) as used by
 * solve_backward_kkt_cudss_ffi (turbompc/solvers/backward/backward_kkt_cudss_ffi.py:232-277):
 * solves [[P, C^T, G_act^T], [C, 0, 0], [G_act, 0, 0]] [dz; y_eq; y_ineq] = [-q; 0; 0]
 * in block form, no CSR.  qp->G holds G_act (inactive rows zero), qp->q the
 * adjoint linear term; l, u, c0, c are ignored (the constraints are
 * homogeneous).  dz (B,T,n); mult (B, n0 + N*nx + T*m) laid out
 * [y_f0 | y_f_dyn | y_ineq] (turbompc/solvers/turbompc_solver.py:727-763).
 * Method: the KKT regrouped by stage is block tridiagonal with blocks of size
 * nb = n + max(n0, nx) + m (nb <= 64); it is factorized by a block LDL^T
 * recursion after a quasi-definite shift reg * max|D| (reg <= 0: 1e-12), and
 * refine_steps rounds of iterative refinement against the unshifted matrix
 * remove the shift (< 0: 2 in fp64, 3 in fp32).  Inactive rows get zero
 * multipliers, as in the reference.  For n <= 16 and nb <= 32 the
 * factorization, solves and residuals hold a stage block's rows in lanes and
 * read the QP blocks directly; other shapes assemble the stage blocks in the
 * workspace and run the ADMM Schur matrix's generic kernels; flags:
 * TMPC_FLAG_GENERIC_KERNEL selects the latter (for cross-checks). */
size_t tmpc_adjoint_kkt_workspace_bytes(int elem_bytes, const tmpc_dims* dims);
int tmpc_adjoint_kkt_f32(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp, float* dz,
                         float* mult, double reg, int32_t refine_steps, uint32_t flags, void* workspace,
                         size_t workspace_bytes);
int tmpc_adjoint_kkt_f64(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp, double* dz,
                         double* mult, double reg, int32_t refine_steps, uint32_t flags, void* workspace,
                         size_t workspace_bytes);

/* ---- SQP linearization: rotor-thrust quadrotor, RK4 ------------------------
 * Replaces, for this model, the host JAX linearization
 * get_dynamics_linearized_matrices (turbompc/problems/optimal_control_problem.py:1176-1332,
 * explicit branch :1217-1272): states (B,N+1,13), controls (B,N+1,4) ->
 * A_minus (B,N,13,17) = [df/dx, df/du], c (B,N,13) = -f + A x + B u.
 * params (host, 7 doubles): mass, Jxx, Jyy, Jzz, arm, yaw coefficient, g. */
int tmpc_quadrotor_linearize_f32(hipStream_t stream, int32_t B, int32_t N, const float* states,
                                 const float* controls, double dt, const double* params,
                                 float* A_minus, float* c);
int tmpc_quadrotor_linearize_f64(hipStream_t stream, int32_t B, int32_t N, const double* states,
                                 const double* controls, double dt, const double* params,
                                 double* A_minus, double* c);
/* The same with row strides (elements between consecutive (b, t) rows; >= 13
 * for states, >= 4 for controls, row (b, t) at b (N+1) + t): for an iterate
 * held packed, as the QP's z_t = [x_t; u_t] rows of an ADMM state (states at
 * z, stride n; controls at z + 13, stride n), read in place. */
int tmpc_quadrotor_linearize_strided_f32(hipStream_t stream, int32_t B, int32_t N, const float* states,
                                         int64_t states_row_stride, const float* controls,
                                         int64_t controls_row_stride, double dt, const double* params,
                                         float* A_minus, float* c);
int tmpc_quadrotor_linearize_strided_f64(hipStream_t stream, int32_t B, int32_t N, const double* states,
                                         int64_t states_row_stride, const double* controls,
                                         int64_t controls_row_stride, double dt, const double* params,
                                         double* A_minus, double* c);

/* The RK4 step of the same dynamics: next (B,N,13) = predict_next_state(x_t, u_t)
 * for t < N, the dynamics part of equality_constraints
 * (turbompc/problems/optimal_control_problem.py:841-912), which the merit line
 * search evaluates at trial points (turbompc/solvers/linesearch.py:14-52). */
int tmpc_quadrotor_dynamics_f32(hipStream_t stream, int32_t B, int32_t N, const float* states,
                                const float* controls, double dt, const double* params, float* next);
int tmpc_quadrotor_dynamics_f64(hipStream_t stream, int32_t B, int32_t N, const double* states,
                                const double* controls, double dt, const double* params, double* next);

/* Linear dynamics: next (B,N,nx) = A x_t + Bm u_t + b for t < N, the dynamics
 * part of equality_constraints (turbompc/problems/optimal_control_problem.py:841-912)
 * for LinearDynamics (turbompc/dynamics/linear_dynamics.py:28-70), which the
 * merit line search evaluates at trial points (turbompc/solvers/linesearch.py:14-52).
 * states (B,N+1,nx), controls (B,N+1,nu), A (B,nx,nx), Bm (B,nx,nu), b (B,nx). */
int tmpc_linear_dynamics_f32(hipStream_t stream, int32_t B, int32_t N, int32_t nx, int32_t nu, const float* states,
                             const float* controls, const float* A, const float* Bm, const float* b, float* next);
int tmpc_linear_dynamics_f64(hipStream_t stream, int32_t B, int32_t N, int32_t nx, int32_t nu, const double* states,
                             const double* controls, const double* A, const double* Bm, const double* b,
                             double* next);

/* Lagrangian Hessian of the same dynamics rows for the exact-Hessian backward
 * pass: replaces get_dynamics_lagrangian_hessian for explicit schemes
 * (turbompc/problems/optimal_control_problem.py:1334-1441), called from
 * _augment_D_with_dynamics_hessian (turbompc/solvers/turbompc_solver.py:1323-1349).
 * lambdas (B,N,13) are the dynamics multipliers y_f_dyn; H (B,N+1,17,17) gets
 * H_t = d^2/dz_t^2 [lambda_t . f(z_t)] for t < N and zeros at t = N. */
int tmpc_quadrotor_lagrangian_hessian_f32(hipStream_t stream, int32_t B, int32_t N, const float* states,
                                          const float* controls, double dt, const double* params,
                                          const float* lambdas, float* H);
int tmpc_quadrotor_lagrangian_hessian_f64(hipStream_t stream, int32_t B, int32_t N, const double* states,
                                          const double* controls, double dt, const double* params,
                                          const double* lambdas, double* H);

/* ---- spherical obstacle constraints ----------------------------------------
 * Linearized obstacle rows g_k = 1 - |p - c_k| / (r_k + 0.001) <= 0, p = the
 * first dim state coordinates: replaces the vmapped jacfwd of
 * get_inequalities_linearized_matrices (turbompc/problems/optimal_control_problem.py:580-626)
 * over OptimalControlProblemObstacle.step_inequality_constraints
 * (turbompc/problems/obstacle_avoidance.py:16-52).  states (B,N+1,nx),
 * centers (B,K,dim), radii (B,K).  Writes rows row0..row0+K-1 of G (B,N+1,m,n),
 * l and u (B,N+1,m): the gradient row, l = -1e9 - offset, u = -offset with
 * offset = g(xbar) - dg/dx xbar.  Other rows are left untouched. */
int tmpc_obstacle_linearize_f32(hipStream_t stream, int32_t B, int32_t N, int32_t nx, int32_t nu, int32_t dim,
                                int32_t K, const float* states, const float* centers, const float* radii, int32_t m,
                                int32_t row0, float* G, float* l, float* u);
int tmpc_obstacle_linearize_f64(hipStream_t stream, int32_t B, int32_t N, int32_t nx, int32_t nu, int32_t dim,
                                int32_t K, const double* states, const double* centers, const double* radii,
                                int32_t m, int32_t row0, double* G, double* l, double* u);

/* Inequality Lagrangian Hessian of the obstacle rows for the exact-Hessian
 * backward pass: replaces get_inequality_lagrangian_hessian
 * (turbompc/problems/optimal_control_problem.py:1443-1480), called from
 * _augment_D_with_inequality_hessian (turbompc/solvers/turbompc_solver.py:1357-1385).
 * mus (B,N+1,m) are the multipliers of all m rows (active mask times y_g; the
 * box rows are linear and contribute nothing).  H (B,N+1,n,n) is overwritten
 * with sum_k mus[row0+k] d^2 g_k / dz^2. */
int tmpc_obstacle_lagrangian_hessian_f32(hipStream_t stream, int32_t B, int32_t N, int32_t nx, int32_t nu, int32_t dim,
                                         int32_t K, const float* states, const float* centers, const float* radii,
                                         int32_t m, int32_t row0, const float* mus, float* H);
int tmpc_obstacle_lagrangian_hessian_f64(hipStream_t stream, int32_t B, int32_t N, int32_t nx, int32_t nu, int32_t dim,
                                         int32_t K, const double* states, const double* centers,
                                         const double* radii, int32_t m, int32_t row0, const double* mus,
                                         double* H);

/* ---- SQP first-order convergence check ------------------------------------
 * Replaces _compute_first_order_convergence_error
 * (turbompc/solvers/turbompc_solver.py:1158-1225), evaluated in XLA by the
 * reference: x (B,T,n) = packed (states, controls), duals y_f0 (B,n0),
 * y_f (B,N,nx), y_g (B,T,m); slack (B,T,m) or NULL when slack variables are off.
 * conv (B,) = max(stationarity, equality, inequality-violation, slack
 * stationarity) inf-norms; eq_err, ineq_err (B,) and g_out (B,T,m) = G x (+ slack)
 * may be NULL.  flags: TMPC_FLAG_STD_DYNAMICS asserts A_plus_t = [-I 0] and
 * E_t = 0, which are then not read; TMPC_FLAG_DIAG_COST asserts diagonal D_t
 * (only the diagonal is read). */
int tmpc_sqp_first_order_f32(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp, const float* x,
                             const float* y_f0, const float* y_f, const float* y_g, const float* slack,
                             double slack_weight, uint32_t flags, float* conv, float* eq_err, float* ineq_err, float* g_out);
int tmpc_sqp_first_order_f64(hipStream_t stream, const tmpc_dims* dims, const tmpc_qp* qp, const double* x,
                             const double* y_f0, const double* y_f, const double* y_g, const double* slack,
                             double slack_weight, uint32_t flags, double* conv, double* eq_err, double* ineq_err, double* g_out);

/* ---- KKT state: active inequality sets -------------------------------------
 * Replaces the XLA-evaluated active-set classification of the solution's KKT
 * state: identify_active_inequalities (turbompc/solvers/turbompc_solver.py:269-292)
 * and its disambiguation by the dual's sign in _build_kkt_state (:1387-1439).
 * Over `count` inequality rows (any layout, the same for every array):
 * a row is active where min(g - l, u - g) <= eps_abs + eps_rel |bound| (the
 * bound of the nearer side, upper where u - g < g - l), lower / upper by that
 * side; with y (the rows' duals, or NULL) a row with y < -dual_tol is lower,
 * y > dual_tol upper, and the proximity decides only in between.  Outputs
 * lower, upper (count bytes, 0 / 1).  eps_abs, eps_rel and dual_tol are
 * rounded to the element type first; the classification then equals the
 * elementwise torch evaluation of the same formula. */
int tmpc_kkt_active_sets_f32(hipStream_t stream, int64_t count, const float* g, const float* l, const float* u,
                             const float* y, double eps_abs, double eps_rel, double dual_tol, uint8_t* lower,
                             uint8_t* upper);
int tmpc_kkt_active_sets_f64(hipStream_t stream, int64_t count, const double* g, const double* l,
                             const double* u, const double* y, double eps_abs, double eps_rel, double dual_tol,
                             uint8_t* lower, uint8_t* upper);

/* ---- SQP line search: merit terms -------------------------------------------
 * Replaces the XLA evaluation of the l1 merit function's terms in
 * backtracking_linesearch / evaluate_constraints_with_bounds
 * (turbompc/solvers/linesearch.py:14-178) for the tracking OCP whose
 * inequality rows are its box rows (cost, :982-1066 and :1504-1515;
 * equality_constraints, :841-912; step_inequality_constraints, :413-471 of
 * turbompc/problems/optimal_control_problem.py).  P = copies * B0 problems
 * (problem p reads the batch's per-problem arrays at row p % B0): states
 * (P, T, nx), controls (P, T, nu) and next (P, T-1, nx) = the model's step
 * f(x_t, u_t) are device arrays, as are x0 (B0, nx), u0 (B0, nu) or NULL,
 * the tracking weights w and reference zref (B0, T, nx+nu), slacks
 * (P, T, mbox) or NULL, the direction (dstates, dcontrols[, dslacks]) or
 * NULL, and the outputs cost, dcost (or NULL), eq, iq (P).  The per-row
 * constants are host arrays: box_idx (mbox <= 32 variable indices < nx+nu),
 * box_lo, box_hi, and with scaled != 0 box_scale (mbox), state_scale (nx) and
 * control_scale (nu) (nx, nu <= 64).  Outputs per problem:
 *   cost = sum w (z - zref)^2 (+ gamma/2 |s|^2), dcost its derivative along
 *   the direction, eq = |x_0 - x0|_1 + sum_t |f_t - x_{t+1}|_1 (+ |u_0 - u0|_1),
 *   rows divided by the variable scales when scaled, iq = the l1 violation of
 *   the box rows (scaled by box_scale when scaled, + slack) against
 *   [box_lo, box_hi] (scaled alike), then with nobs > 0 of the obstacle rows
 *   of OptimalControlProblemObstacle (obstacle_avoidance.py:16-52):
 *   g_k = 1 - |p_t - c_k| / (r_k + 0.001) with p_t the first dim (<= nx)
 *   state coordinates, bounds (-1e9, 0), all scaled by obs_scale when scaled;
 *   centers (B0, nobs, dim) and radii (B0, nobs) are device arrays (nobs <=
 *   32), and slacks then cover mbox + nobs rows.  NaN propagates into every
 *   term.  With lin_A set the dynamics are linear and next may be NULL:
 *   f_t = A x_t + Bm u_t + b is formed in the kernel as tmpc_linear_dynamics_*
 *   forms it, from lin_A (B0, nx, nx), lin_B (B0, nx, nu) and lin_b (B0, nx),
 *   device arrays. */
typedef struct {
  int32_t P, B0, T, nx, nu, mbox;
  const void* states;
  const void* controls;
  const void* next;
  const void* x0;
  const void* u0;
  const void* w;
  const void* zref;
  int32_t scaled;
  const double* state_scale;   /* host (nx) */
  const double* control_scale; /* host (nu) */
  const int32_t* box_idx;      /* host (mbox) */
  const double* box_lo;        /* host (mbox) */
  const double* box_hi;        /* host (mbox) */
  const double* box_scale;     /* host (mbox) */
  const void* slacks;
  double gamma;
  const void* dstates;
  const void* dcontrols;
  const void* dslacks;
  void* cost;
  void* dcost;
  void* eq;
  void* iq;
  int32_t nobs, dim;
  const void* centers;
  const void* radii;
  double obs_scale;
  const void* lin_A; /* NULL: f_t from next */
  const void* lin_B;
  const void* lin_b;
} tmpc_merit_terms;
int tmpc_ocp_merit_terms_f32(hipStream_t stream, const tmpc_merit_terms* args);
int tmpc_ocp_merit_terms_f64(hipStream_t stream, const tmpc_merit_terms* args);

/* The step choice of backtracking_linesearch (turbompc/solvers/linesearch.py:54-178)
 * from merit terms (the outputs of tmpc_ocp_merit_terms_* for the base point,
 * cost, dcost, eq, iq (B), and for the A <= 8 candidates, cost_a, eq_a, iq_a
 * (A B, candidate j of problem b at j B + b)), the candidate steps alphas
 * (host, A) and the parameters eta, mu_min, mu_max and the constraint floor:
 * mu = clip(nan_to_num(dcost / (0.5 max(eq + iq, floor))), mu_min, mu_max);
 * alpha_out[b] = the largest alpha_j whose merit decrease
 * cand_j - (merit + eta alpha_j (dcost - mu (eq + iq))) is finite and <= 0,
 * else the finite candidate of least merit (the first of equal ones), else
 * alpha_0; mu_out (B, or NULL) receives mu.  Every value is rounded as the
 * elementwise form rounds it (one rounding per operation; eta alpha_j is the
 * double product rounded), so the choice equals that form's. */
int tmpc_linesearch_choose_f32(hipStream_t stream, int32_t B, int32_t A, const float* cost, const float* dcost,
                               const float* eq, const float* iq, const float* cost_a, const float* eq_a,
                               const float* iq_a, const double* alphas, double eta, double mu_min, double mu_max,
                               double floor_, float* alpha_out, float* mu_out);
int tmpc_linesearch_choose_f64(hipStream_t stream, int32_t B, int32_t A, const double* cost, const double* dcost,
                               const double* eq, const double* iq, const double* cost_a, const double* eq_a,
                               const double* iq_a, const double* alphas, double eta, double mu_min,
                               double mu_max, double floor_, double* alpha_out, double* mu_out);

#ifdef __cplusplus
}
#endif
#endif /* TMPC_H */
