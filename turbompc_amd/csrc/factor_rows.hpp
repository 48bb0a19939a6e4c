// Block factorization of the explicit-integrator Schur matrix (the cuDSS
// replacement of the direct path, admm_stream.hpp factor_std_kernel computes
// the same blocks), one problem per 16-lane row of a wavefront: four problems
// per wavefront, so B = 4096 is 1024 wavefronts, one per SIMD.
//
//   Theta_0 = theta_0,  Theta_t = theta_t - rho_f^2 [A_{t-1} Theta_{t-1}^{-1} A_{t-1}^T, 0; 0, 0]
//   theta_t = D_t + sigma I + rho_f (A_t^T A_t + A0^T A0 [t = 0] + diag(I_nx, 0) [t > 0]) + rho G_t^T G_t
//
// (compute_S_Phiinv's diagonal blocks, admm.py:93-100, with the block
// elimination of the tridiagonal Schur matrix), and stores the symmetric part
// of Theta_t^{-1}, packed, in fp64 arithmetic rounded on store.
//
// Lane i of a problem's row holds row i of the block; for n = 17 the row
// holds rows 0..15 and row 16 is implied by symmetry: its off-diagonal
// entries are the lanes' column-16 entries and its diagonal is a per-problem
// scalar.  Everything that moves between lanes moves by DPP row broadcasts
// (row_newbcast), folded into v_fmac_f64_dpp:
//   * the gram of the stage's rows [A_t; G_t]: lane i holds column i of the
//     rows, so row r of the block is the row's column values broadcast;
//   * the Schur term through Y = Theta_{t-1}^{-1} A_{t-1}^T: Y's column s is
//     a row product of lane i's Theta^{-1} row with A's row s (the lanes'
//     column values), then S = A_{t-1} Y from lane i's own A row;
//   * the inversion by the symmetric sweep (Goodnight): pivot k's row is lane
//     k's, broadcast; the sweep leaves minus the inverse.  A pivot row is not
//     scaled at its step (its lane keeps 1/d and scales at the end), so every
//     lane runs the same instructions.
// The lanes' two copies of each off-diagonal entry are averaged through LDS
// at the end of the stage (the symmetric part, as factor_std_kernel keeps).
#pragma once
#include "admm_stream.hpp"

namespace tmpc {

constexpr int kFacRow = 16;  // lanes per problem

// fp64 DPP blocks of the row factorization (row_newbcast, a 16-lane row).
// Each block starts with the wait states a DPP read needs after a VALU write
// of its source and ends with those a following DPP read of its results needs.

// c[k] += s * (src of lane k), k < K

template <int N>
__device__ __forceinline__ void axpy_bcast6(double (&c)[N], double src, double s) {
  static_assert(N >= 6, "");
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %6, %7 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %6, %7 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %2, %6, %7 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %3, %6, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %4, %6, %7 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %5, %6, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(c[4]), "+v"(c[5])
      : "v"(src), "v"(s));
}

template <int N>
__device__ __forceinline__ void axpy_bcast9(double (&c)[N], double src, double s) {
  static_assert(N >= 9, "");
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %9, %10 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %9, %10 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %2, %9, %10 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %3, %9, %10 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %4, %9, %10 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %5, %9, %10 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %6, %9, %10 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %7, %9, %10 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %8, %9, %10 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(c[4]), "+v"(c[5]), "+v"(c[6]), "+v"(c[7]), "+v"(c[8])
      : "v"(src), "v"(s));
}

template <int N>
__device__ __forceinline__ void axpy_bcast16(double (&c)[N], double src, double s) {
  static_assert(N >= 16, "");
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %16, %17 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %16, %17 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %2, %16, %17 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %3, %16, %17 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %4, %16, %17 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %5, %16, %17 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %6, %16, %17 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %7, %16, %17 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %8, %16, %17 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %9, %16, %17 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %10, %16, %17 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %11, %16, %17 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %12, %16, %17 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %13, %16, %17 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %14, %16, %17 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %15, %16, %17 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(c[4]), "+v"(c[5]), "+v"(c[6]), "+v"(c[7]), "+v"(c[8]), "+v"(c[9]), "+v"(c[10]), "+v"(c[11]), "+v"(c[12]), "+v"(c[13]), "+v"(c[14]), "+v"(c[15])
      : "v"(src), "v"(s));
}

// a[j] += g * (a[j] of lane KP), j < K: the Gauss-Jordan sweep of pivot KP

template <int KP, int N>
__device__ __forceinline__ void sweep_bcast6(double (&a)[N], double g) {
  static_assert(N >= 6 && KP < 16, "");
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %0, %6 row_newbcast:%c7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %1, %6 row_newbcast:%c7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %2, %2, %6 row_newbcast:%c7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %3, %3, %6 row_newbcast:%c7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %4, %4, %6 row_newbcast:%c7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %5, %5, %6 row_newbcast:%c7 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5])
      : "v"(g), "i"(KP));
}

template <int KP, int N>
__device__ __forceinline__ void sweep_bcast9(double (&a)[N], double g) {
  static_assert(N >= 9 && KP < 16, "");
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %0, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %1, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %2, %2, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %3, %3, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %4, %4, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %5, %5, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %6, %6, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %7, %7, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %8, %8, %9 row_newbcast:%c10 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]), "+v"(a[8])
      : "v"(g), "i"(KP));
}

template <int KP, int N>
__device__ __forceinline__ void sweep_bcast16(double (&a)[N], double g) {
  static_assert(N >= 16 && KP < 16, "");
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %0, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %1, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %2, %2, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %3, %3, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %4, %4, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %5, %5, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %6, %6, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %7, %7, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %8, %8, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %9, %9, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %10, %10, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %11, %11, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %12, %12, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %13, %13, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %14, %14, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %15, %15, %16 row_newbcast:%c17 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]), "+v"(a[8]), "+v"(a[9]), "+v"(a[10]), "+v"(a[11]), "+v"(a[12]), "+v"(a[13]), "+v"(a[14]), "+v"(a[15])
      : "v"(g), "i"(KP));
}

template <int KP, int N>
__device__ __forceinline__ void sweep_bcast17(double (&a)[N], double g) {
  static_assert(N >= 17 && KP < 16, "");
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %0, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %1, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %2, %2, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %3, %3, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %4, %4, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %5, %5, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %6, %6, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %7, %7, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %8, %8, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %9, %9, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %10, %10, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %11, %11, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %12, %12, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %13, %13, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %14, %14, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %15, %15, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %16, %16, %17 row_newbcast:%c18 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]), "+v"(a[8]), "+v"(a[9]), "+v"(a[10]), "+v"(a[11]), "+v"(a[12]), "+v"(a[13]), "+v"(a[14]), "+v"(a[15]), "+v"(a[16])
      : "v"(g), "i"(KP));
}

template <int NC, int N>
__device__ __forceinline__ void fac_axpy(double (&c)[N], double src, double s) {
  if constexpr (NC == 6)
    axpy_bcast6(c, src, s);
  else if constexpr (NC == 9)
    axpy_bcast9(c, src, s);
  else
    axpy_bcast16(c, src, s);  // n = 16, and the lane rows of n = 17
}

template <int NC, int KP, int N>
__device__ __forceinline__ void fac_sweep(double (&a)[N], double g) {
  if constexpr (NC == 6)
    sweep_bcast6<KP>(a, g);
  else if constexpr (NC == 9)
    sweep_bcast9<KP>(a, g);
  else if constexpr (NC == 16)
    sweep_bcast16<KP>(a, g);
  else
    sweep_bcast17<KP>(a, g);  // the lane rows and column 16
}

// sum_k w[k] (s of lane k) over the lane rows
template <int NC, int N>
__device__ __forceinline__ double fac_dot(const double (&w)[N], double s) {
  constexpr int NL = NC < kFacRow ? NC : kFacRow;
  double v[NL];
#pragma unroll
  for (int k = 0; k < NL; ++k) v[k] = w[k];
  return row_dot_dpp(v, s);
}

// 1/d by the hardware reciprocal estimate refined with two Newton-Raphson
// steps r <- r + r (1 - d r) (each roughly squares the relative error; d is
// a pivot of an SPD block, far from the denormal and overflow ranges)
__device__ __forceinline__ double recip(double d) {
  double r = __builtin_amdgcn_rcp(d);
  double e = __builtin_fma(-d, r, 1.0);
  r = __builtin_fma(r, e, r);
  e = __builtin_fma(-d, r, 1.0);
  return __builtin_fma(r, e, r);
}

template <int KP, int NL, typename F>
__device__ __forceinline__ void static_for_pivots(F&& f) {
  if constexpr (KP < NL) {
    f(std::integral_constant<int, KP>{});
    static_for_pivots<KP + 1, NL>(f);
  }
}

// NC in {6, 9, 16, 17}; NR bounds the stacked rows nx + m of a stage record;
// DIAG: the D_t records hold the diagonal (RecGeom); FULL: nx + m == NR, so
// every stacked row of a record is live (no per-row tests).
//
// Register budget (one wavefront per SIMD, 4 problems): the records stay in
// the storage type R until a product reads them (fp64 conversions at the
// use), the next stage's records are prefetched in R, and each lane writes
// its own row of the packed inverse from registers (no index arithmetic, no
// LDS re-read).  The arithmetic, and its order, is that of the symmetric
// sweep described above.
template <typename R, int NC, int NR, bool DIAG, bool FULL>
__global__ __launch_bounds__(kWave, 1) void factor_row_kernel(Dims d, const R* __restrict__ am,
                                                              const R* __restrict__ dm, const R* __restrict__ A0,
                                                              const R* __restrict__ rho, R sigma, R rho_f_factor,
                                                              int32_t* __restrict__ ctl, R* __restrict__ thinv) {
  using C = double;
  constexpr int W = kFacRow;
  constexpr int NL = NC < W ? NC : W;  // rows held by lanes
  constexpr bool IMP = NC > W;         // row 16 implied by symmetry
  constexpr int n = NC, PITCH = th_pitch(NC);
  const int T = d.T, N = d.N, nx = d.nx, n0 = d.n0, m = d.m, B = d.B;
  const int nr = FULL ? NR : nx + m;
  const RecGeom rg = rec_geom(d, DIAG);
  const int tid = threadIdx.x, q = tid / W, i = tid - q * W;
  const int braw = blockIdx.x * (kWave / W) + q;
  const bool real = braw < B;
  const int b = real ? braw : B - 1;
  const bool lrow = NL == W || i < NL;  // the lane holds a row
  const int ic = lrow ? i : 0;          // clamped row index for loads
  const int arow = min(ic, nr - 1);     // the M row read as the lane's A row (used for i < nx only)
  if (ctl != nullptr && __ballot(real && ctl[b * 4 + 2] != 0) == 0) return;  // nothing flagged here
  __shared__ C sym[kWave / W][W][W + 1];  // the lane rows of each problem
  const C rho_i = (C)rho[b], rho_f = rho_i * (C)rho_f_factor, sig = (C)sigma;

  // ---- stage records of the next stage, prefetched into registers (type R) ----
  R pMc[NR], pM16[NR], pAr[NC], pD[DIAG ? 1 : NC], pD16 = R(0);
  auto load = [&](int t) __attribute__((always_inline)) {
    const R* M = am + ((size_t)t * B + b) * rg.amp;
    const R* Dr = dm + ((size_t)t * B + b) * rg.dmp;
    // idle lanes read column 0 (their rows are zeroed where theta_t is built);
    // lanes i >= nx read a G row as their A row, which only their own unused
    // Schur values see
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (FULL || r < nr) {
        pMc[r] = M[r * n + ic];
        if (IMP) pM16[r] = M[r * n + (n - 1)];
      } else {
        pMc[r] = R(0);
        if (IMP) pM16[r] = R(0);
      }
    }
#pragma unroll
    for (int k = 0; k < NC; ++k) pAr[k] = M[arow * n + k];
    if constexpr (DIAG) {
      pD[0] = lrow ? Dr[ic] : R(0);
      if (IMP) pD16 = Dr[n - 1];
    } else {
#pragma unroll
      for (int k = 0; k < NC; ++k) pD[k] = lrow ? Dr[pidx(ic, k)] : R(0);
      if (IMP) pD16 = Dr[pidx(n - 1, n - 1)];
    }
  };
  load(0);

  C a[NC];    // row i of Theta_t, then of Theta_t^{-1}; a[16]: column 16 (n = 17)
  C a16 = 0;  // Theta[16][16] (n = 17)
  R Mc[NR], M16[NR];  // the stage's rows [A_t; G_t]: column i, column 16
  C Ar[NC];           // row i of A_t
#pragma unroll
  for (int k = 0; k < NC; ++k) a[k] = C(0);
#pragma unroll
  for (int r = 0; r < NR; ++r) Mc[r] = M16[r] = R(0);
#pragma unroll
  for (int k = 0; k < NC; ++k) Ar[k] = C(0);
  // this lane's row of the packed lower triangle starts at i (i + 1) / 2; the
  // wavefront's problems are wb0 .. wb0 + wnp - 1
  const int prow = (i * (i + 1)) >> 1;
  const int wb0 = blockIdx.x * (kWave / W), wnp = min(kWave / W, B - wb0);

  for (int t = 0; t < T; ++t) {
    // Schur term rho_f^2 (A_{t-1} Theta_{t-1}^{-1} A_{t-1}^T)[i][s], s < nx, from
    // the previous stage's inverse (a, a16) and records (Mc, M16, Ar)
    C sv[NC];
#pragma unroll
    for (int s = 0; s < NC; ++s) sv[s] = C(0);
    if (t > 0 && !IMP) {
#pragma unroll
      for (int s = 0; s < NC; ++s) {
        if (s < nx) {
          const C y = fac_dot<NC>(a, (C)Mc[s]);  // Y[i][s] = (Theta^{-1} A^T)[i][s]
          sv[s] = fac_dot<NC>(Ar, y);            // sum_j A[i][j] Y[j][s]
        }
      }
    }
    if (t > 0 && IMP) {
      // n = 17: U = A Theta^{-1} from lane i's A row (row 16 of Theta^{-1} is
      // the lanes' column 16), then S[i][s] = sum_k U[i][k] A[s][k]
      C u[NC];
#pragma unroll
      for (int k = 0; k < NC - 1; ++k) {
        u[k] = fac_dot<NC>(Ar, a[k]);
        u[k] += Ar[NC - 1] * row_bcast_at(a[NC - 1], k);  // A[i][16] Theta^{-1}[16][k]
      }
      u[NC - 1] = fac_dot<NC>(Ar, a[NC - 1]) + Ar[NC - 1] * a16;
#pragma unroll
      for (int s = 0; s < NC; ++s)
        if (s < nx) sv[s] = fac_dot<NC>(u, (C)Mc[s]) + u[NC - 1] * (C)M16[s];
    }

    // this stage's records
    C Dd[DIAG ? 1 : NC], D16 = C(0);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      Mc[r] = pMc[r];
      if (IMP) M16[r] = pM16[r];
    }
#pragma unroll
    for (int k = 0; k < NC; ++k) Ar[k] = (C)pAr[k];
#pragma unroll
    for (int k = 0; k < (DIAG ? 1 : NC); ++k) Dd[k] = (C)pD[k];
    if (IMP) D16 = (C)pD16;
    if (t + 1 < T) load(t + 1);

    // theta_t row i (and Theta[16][16]); the diagonal terms D_ii (diagonal
    // records), sigma and rho_f A_plus^T A_plus = rho_f diag(I_nx, 0) in one
    int ii = i;  // the comparisons with the lane's row index are made here
    __asm__ volatile("" : "+v"(ii));
    const C dgl = (DIAG ? Dd[0] : C(0)) + sig + ((t > 0 && ii < nx) ? rho_f : C(0));
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const C off = DIAG ? C(0) : Dd[DIAG ? 0 : k];
      a[k] = lrow ? (k == ii ? off + dgl : off) : C(0);
    }
    if (IMP) a16 = D16 + sig;
    const int r0 = t < N ? 0 : nx;  // the last stage has no dynamics rows
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (r >= r0 && (FULL || r < nr)) {
        const C w = r < nx ? rho_f : rho_i;
        const C mc = (C)Mc[r];
        const C s = w * mc;
        fac_axpy<NC>(a, mc, s);
        if (IMP) {
          const C m16 = (C)M16[r];
          a[NC - 1] += s * m16;
          a16 += (w * m16) * m16;
        }
      }
    }
    if (t == 0) {
      const R* A0b = A0 + (size_t)b * n0 * n;
      for (int r = 0; r < n0; ++r) {
        const C c = lrow ? (C)A0b[r * n + ic] : C(0);
        const C c16 = IMP ? (C)A0b[r * n + (n - 1)] : C(0);
        const C s = rho_f * c;
        fac_axpy<NC>(a, c, s);
        if (IMP) {
          a[NC - 1] += s * c16;
          a16 += (rho_f * c16) * c16;
        }
      }
    }
    if (t > 0) {
      const C fs = ii < nx ? rho_f * rho_f : C(0);  // the Schur term touches rows and columns < nx
#pragma unroll
      for (int k = 0; k < NC; ++k)
        if (k < nx) a[k] -= fs * sv[k];
    }

    // symmetric sweep: minus the inverse, lane rows scaled by their pivots
    C myip = C(1);
    static_for_pivots<0, NL>([&](auto kc) __attribute__((always_inline)) {
      constexpr int KP = decltype(kc)::value;
      const C dk = row_bcast<KP>(a[KP]);
      const C ip = recip(dk);
      const bool me = ii == KP;
      const C f = a[KP];
      const C g = me ? C(0) : -f * ip;
      const C fk = me ? C(-1) : f * ip;
      myip = me ? ip : myip;
      C p16 = C(0);
      if (IMP) p16 = row_bcast<KP>(a[NC - 1]);
      fac_sweep<NC, KP>(a, g);
      a[KP] = fk;
      if (IMP) a16 -= (p16 * ip) * p16;
    });
    if (IMP) {
      // pivot 16: its row is the lanes' column 16 (true values: scaled back)
      const C ip = recip(a16);
      const C f = a[NC - 1];
      const C tr = f * myip;
      fac_axpy<NC>(a, tr, -f * ip);
      a[NC - 1] = f * ip;
      a16 = -ip;
    }
#pragma unroll
    for (int k = 0; k < NC; ++k) a[k] *= -myip;
    if (IMP) a16 = -a16;

    // symmetric part of the lane block: row i averaged with column i
#pragma unroll
    for (int k = 0; k < NL; ++k) sym[q][i][k] = a[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NL; ++k) a[k] = lrow ? C(0.5) * (a[k] + sym[q][k][i]) : C(0);
    // the packed lower triangle: lane i writes its row's entries k <= i (and,
    // n = 17, entry i of row 16, which is its column-16 value, and lane 0 the
    // last diagonal entry).  The stores go through a buffer resource whose
    // range is the problem's block: a store that is off takes an offset past
    // the range and is dropped (no exec-mask branches).
    {
      // one resource per wavefront (uniform): the blocks of its problems
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          thinv + ((size_t)t * B + wb0) * PITCH, (short)0, (int)(wnp * PITCH * sizeof(R)), kBufferFlags);
      const bool on = real && lrow;
      const unsigned base = (unsigned)(q * PITCH);
#pragma unroll
      for (int k = 0; k < NL; ++k) buf_store((R)a[k], rs, on && k <= ii, base + (unsigned)(prow + k));
      if (IMP) {
        buf_store((R)a[NC - 1], rs, on, base + (unsigned)(packed_size(NC - 1) + ii));
        buf_store((R)a16, rs, on && ii == 0, base + (unsigned)(packed_size(NC) - 1));
      }
    }
    __syncthreads();
  }
  if (ctl != nullptr && real && i == 0) ctl[b * 4 + 2] = 0;
}

}  // namespace tmpc
