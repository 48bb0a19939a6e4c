// ADMM on the PCG Schur solve with the whole problem on one compute unit
// (explicit-integrator QPs: A_plus_t = [-I 0], E_t = 0).
//
// Same iteration as admm_pcg_chunk_kernel (pcg.hpp), which follows the
// reference's JAX loop over PCGPrimalOptimalControl
// (turbompc/solvers/admm/admm.py:795-1049, pcg_primal.py:70-175), organised
// for the MI355X's 160 KB LDS instead of streaming S and Phiinv from HBM on
// every PCG iteration:
//
//   * one problem per 1024-thread workgroup; thread (t, i) owns element i of
//     stage t of every n-vector, G row (t, r) of the m-vectors (thread t m + r)
//     and dynamics row (t - 1, i) (i < nx) of the equality multipliers;
//   * theta_t (the S diagonal block) and theta_t^{-1} are built in fp64 on the
//     device (as compute_S_Phiinv, admm.py:71-154) and rebuilt in place when
//     rho changes; the thread keeps row i of theta_t^{-1} in registers, the
//     theta_t rows sit in LDS when they fit (fp32) and in the workspace
//     otherwise (fp64, read through the caches), A_minus sits in LDS;
//   * S and Phiinv are applied in product form from those blocks:
//       S p   = theta_t p_t + phi_{t-1} p_{t-1} + phi_t^T p_{t+1},
//               phi_t = -rho_f [A_minus_t; 0]
//       Phiinv r = theta_t^{-1}(-r_t + phi_{t-1} v_{t-1} + phi_t^T v_{t+1}),
//               v = theta^{-1} r
//     which are the products of the reference's S rows [phi_{t-1} | theta_t
//     | phi_t^T] and Phiinv rows [theta_t^{-1} phi_{t-1} theta_{t-1}^{-1} |
//     -theta_t^{-1} | theta_t^{-1} phi_t^T theta_{t+1}^{-1}] (admm.py:107-153);
//   * the PCG vectors p, r, v, u live in LDS (row pitch n | 1, so the rows of
//     one wavefront fall in different banks); x, gamma, the search direction's
//     own element and the ADMM state live in registers;
//   * dot products reduce within the wavefront by butterfly shuffles and
//     across the 16 wavefronts through LDS, in a fixed order (deterministic).
// QP data that an ADMM iteration reads once (D, G, A0, q) come from global
// memory; per solve the kernel reads the problem's blocks and writes its
// state once, and no PCG iteration touches HBM.
#pragma once
#include "pcg.hpp"

namespace tmpc {

constexpr int kPcgThreads = 1024;
constexpr size_t kPcgMaxLds = 160 * 1024;

__host__ __device__ inline int pcg_pitch(int n) { return n | 1; }

struct PcgLdsLayout {
  int vp, vr, vv, vu, sc, sz, red, am, th;  // element offsets (in R) from the LDS base
  size_t bytes;
};

// LDS of admm_pcg_lds_kernel; `thl` = theta_t rows in LDS (else in the workspace).
template <typename R>
__host__ __device__ inline PcgLdsLayout pcg_lds_layout(const Dims& d, bool thl) {
  PcgLdsLayout L;
  const int P = pcg_pitch(d.n), Tv = d.T * P;
  int off = 0;
  auto take = [&](int cnt) {
    const int o = off;
    off += (cnt + 3) & ~3;
    return o;
  };
  L.vp = take(Tv);
  L.vr = take(Tv);
  L.vv = take(Tv);
  L.vu = take(Tv);
  L.sc = take(d.N * d.nx + d.n0);
  L.sz = take(d.T * d.m > 0 ? d.T * d.m : 1);
  // two block-sum slots, the residual maxima (11 x 16 + 11) and results (6)
  L.red = take(2 * 32 + 12 * 16 + 8);
  L.am = take(d.N * d.nx * P);
  L.th = thl ? take(d.T * d.n * P) : 0;
  L.bytes = (size_t)off * sizeof(R);
  return L;
}

// 0: the kernel does not cover the shape; 1: theta_t rows in the workspace;
// 2: theta_t rows in LDS.  Every role must fit in one workgroup (and the fp64
// pivot rows of the setup in the v/u region, which n0 <= n, nx < n ensure).
template <typename R>
inline int pcg_lds_mode(const Dims& d) {
  if (!(d.T * d.n <= kPcgThreads && d.T * d.m <= kPcgThreads && d.n0 <= d.n && d.nx < d.n &&
        (d.n == 6 || d.n == 9 || d.n == 16 || d.n == 17)))
    return 0;
  if (pcg_lds_layout<R>(d, true).bytes <= kPcgMaxLds) return 2;
  if (pcg_lds_layout<R>(d, false).bytes <= kPcgMaxLds) return 1;
  return 0;
}

template <typename R, int NC, bool THL>
__global__ __launch_bounds__(kPcgThreads) void admm_pcg_lds_kernel(AdmmPcgArgs<R> pa) {
  const AdmmArgs<R>& a = pa.a;
  const Dims d = a.d;
  constexpr int n = NC;
  constexpr int NW = kPcgThreads / kWave;
  static_assert(NW == 16, "block sums read one wavefront sum per lane of a 16-lane row");
  const int T = d.T, N = d.N, nx = d.nx, n0 = d.n0, m = d.m;
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const int P = pcg_pitch(n);
  extern __shared__ __align__(16) unsigned char smem_raw[];
  R* sm = reinterpret_cast<R*>(smem_raw);
  const PcgLdsLayout L = pcg_lds_layout<R>(d, THL);
  R* vp = sm + L.vp;
  R* vr = sm + L.vr;
  R* vv = sm + L.vv;
  R* vu = sm + L.vu;
  R* sc = sm + L.sc;
  R* sz = sm + L.sz;
  R* red = sm + L.red;
  R* aml = sm + L.am;
  double* piv = reinterpret_cast<double*>(vv);  // setup only: [T][n] fp64 pivot rows (v and u regions)

  // ---- roles ------------------------------------------------------------------
  const bool el = tid < T * n;
  const int t = el ? tid / n : 0, i = el ? tid - (tid / n) * n : 0;
  const int ev = t * P + i;  // this element in an LDS vector
  const bool gr = m > 0 && tid < T * m;
  const int tg = gr ? tid / m : 0, rg = gr ? tid - (tid / m) * m : 0;
  const bool dr = el && t >= 1 && i < nx;   // dynamics row (t - 1, i)
  const bool a0r = el && t == 0 && i < n0;  // row i of A0
  const size_t boff = (size_t)b;
  // This problem's blocks (uniform bases) and the thread's 32-bit offsets into
  // them, so that global accesses take a scalar base and one offset register.
  const R* const Dq = a.qp.D + boff * T * n * n;
  const R* const Gq = a.qp.G + boff * T * m * n;
  const R* const A0q = a.qp.A0 + boff * n0 * n;
  const R* const qq = a.qp.q + boff * T * n;
  const R* const cq = a.qp.c + boff * N * nx;
  const R* const c0q = a.qp.c0 + boff * n0;
  const R* const lq = a.qp.l + boff * T * m;
  const R* const uq = a.qp.u + boff * T * m;
  const unsigned ue = el ? (unsigned)tid : 0u;                      // element (t, i)
  const unsigned ug = gr ? (unsigned)tid : 0u;                      // G row (tg, rg)
  const unsigned uf = dr ? (unsigned)((t - 1) * nx + i) : 0u;       // dynamics row (t - 1, i)
  const unsigned uf0 = a0r ? (unsigned)i : 0u;                      // A0 row i
  // theta_t row i: LDS or this problem's [T][n][n] slice of the workspace's S region
  R* const thq = THL ? sm + L.th : const_cast<R*>(pa.S) + boff * T * n * n;
  const unsigned uth = THL ? ue * P : ue * n;

  // ---- A_minus to LDS ([N nx][P] rows) ----------------------------------------------
  #pragma unroll 1
  for (int e = tid; e < N * nx * n; e += kPcgThreads) {
    const int r = e / n, k = e - (e / n) * n;
    aml[r * P + k] = a.qp.Am[boff * N * nx * n + (unsigned)e];
  }

  // ---- state in registers (QP vectors are re-read where used, once per ADMM iteration) ----
  R x = el ? a.st.x[boff * T * n + ue] : R(0);
  R z = R(0), yg = R(0), xi = R(0);
  if (gr) {
    z = a.st.z[boff * T * m + ug];
    yg = a.st.y_g[boff * T * m + ug];
    xi = a.st.xi[boff * T * m + ug];
  }
  R yf = dr ? a.st.y_f[boff * N * nx + uf] : R(0);
  R yf0 = a0r ? a.st.y_f0[boff * n0 + uf0] : R(0);
  const bool slack = a.use_slack && m > 0;
  const R gs = (slack && a.qp.slack_w) ? a.qp.slack_w[b] : R(0);
  R rho = a.st.rho[b];
  const R alpha = a.alpha, oma = R(1) - a.alpha;

  // ---- theta_t and theta_t^{-1} (fp64, rounded on store) --------------------------
  R ti[NC];
  auto setup = [&](R rho_v) __attribute__((always_inline)) {
    const double rho_i = (double)rho_v, rho_f = rho_i * (double)a.rho_f_factor;
    // The row index passes through an empty asm so that the comparisons with
    // it below are made here, not hoisted out of the ADMM loop as NC masks
    // held for the whole solve.
    int ii = i;
    __asm__ volatile("" : "+v"(ii));
    double ar[NC];
    if (el) {
      // D_t + sigma I + rho G_t^T G_t + rho_f (A0^T A0 [t = 0] + A_minus_t^T A_minus_t [t < N]
      // + A_plus_{t-1}^T A_plus_{t-1} [t > 0]), A_plus = [-I 0]
#pragma unroll
      for (int k = 0; k < NC; ++k) ar[k] = (double)Dq[ue * n + k] + (k == ii ? (double)a.sigma : 0.0);
      if (m) {
        const unsigned gt = (unsigned)(t * m * n);
        #pragma unroll 1
        for (int r = 0; r < m; ++r) {
          const double gi = rho_i * (double)Gq[gt + r * n + i];
#pragma unroll
          for (int k = 0; k < NC; ++k) ar[k] += gi * (double)Gq[gt + r * n + k];
        }
      }
      if (t == 0) {
        #pragma unroll 1
        for (int r = 0; r < n0; ++r) {
          const double ai = rho_f * (double)A0q[r * n + i];
#pragma unroll
          for (int k = 0; k < NC; ++k) ar[k] += ai * (double)A0q[r * n + k];
        }
      }
      if (t < N) {
        const R* At = aml + t * nx * P;
        #pragma unroll 1
        for (int r = 0; r < nx; ++r) {
          const double ai = rho_f * (double)At[r * P + i];
#pragma unroll
          for (int k = 0; k < NC; ++k) ar[k] += ai * (double)At[r * P + k];
        }
      }
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        if (t > 0 && ii < nx && k == ii) ar[k] += rho_f;
        thq[uth + k] = (R)ar[k];
      }
    }
    // Gauss-Jordan in place without pivoting (theta_t is SPD): row i of theta_t^{-1}
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      __syncthreads();
      if (el && ii == k)
#pragma unroll
        for (int j = 0; j < NC; ++j) piv[t * n + j] = ar[j];
      __syncthreads();
      if (el) {
        const double ip = 1.0 / piv[t * n + k];
        const double f = ar[k];
        const bool me = ii == k;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          const double pj = piv[t * n + j];
          ar[j] = me ? ((j == k) ? ip : ar[j] * ip) : ((j == k) ? -f * ip : ar[j] - f * (pj * ip));
        }
      }
    }
    __syncthreads();  // pivot rows read; theta rows complete
#pragma unroll
    for (int k = 0; k < NC; ++k) ti[k] = el ? (R)ar[k] : R(0);
  };

  // ---- products ------------------------------------------------------------------
  // phi_{t-1} s_{t-1} + phi_t^T s_{t+1} for this element
  auto offdiag = [&](const R* s, R rho_f) __attribute__((always_inline)) -> R {
    R acc = R(0);
    if (el && t > 0 && i < nx) {
      const R* ar_ = aml + ((t - 1) * nx + i) * P;
      const R* sp = s + (t - 1) * P;
      R a_ = R(0);
#pragma unroll
      for (int k = 0; k < NC; ++k) a_ += ar_[k] * sp[k];
      acc -= rho_f * a_;
    }
    if (el && t < N) {
      const R* ac = aml + t * nx * P + i;
      const R* sn = s + (t + 1) * P;
      R a_ = R(0);
#pragma unroll
      for (int j = 0; j < NC - 1; ++j)
        if (j < nx) a_ += ac[j * P] * sn[j];
      acc -= rho_f * a_;
    }
    return acc;
  };
  auto theta_dot = [&](const R* s) __attribute__((always_inline)) -> R {
    const R* st_ = s + t * P;
    R acc = R(0);
#pragma unroll
    for (int k = 0; k < NC; ++k) acc += thq[uth + k] * st_[k];
    return acc;
  };
  auto thinv_dot = [&](const R* s) __attribute__((always_inline)) -> R {
    const R* st_ = s + t * P;
    R acc = R(0);
#pragma unroll
    for (int k = 0; k < NC; ++k) acc += ti[k] * st_[k];
    return acc;
  };
  int rslot = 0;
  auto block_sum = [&](R v) __attribute__((always_inline)) -> R {
    v = wave_sum(v);
    R* rr = red + rslot * 32;
    rslot ^= 1;
    if (lane == 0) rr[wid] = v;
    __syncthreads();
    return row_sum(rr[lane & (NW - 1)]);  // the 16 wavefront sums, one per lane of each row
  };
  // rt = Phiinv r for r in vr (complete in LDS); returns this element's rt
  auto apply_phiinv = [&](R rho_f) __attribute__((always_inline)) -> R {
    const R v = el ? thinv_dot(vr) : R(0);
    if (el) vv[ev] = v;
    __syncthreads();
    const R rr = el ? vr[ev] : R(0);
    const R u = offdiag(vv, rho_f) - rr;
    if (el) vu[ev] = u;
    __syncthreads();
    return el ? thinv_dot(vu) : R(0);
  };

  // ---- per-problem control state (as admm_pcg_chunk_kernel, one chunk) ------------
  int it = 0;
  bool done = false;
  bool tl = true;  // residuals above tolerance (the initial residuals are infinite)
  bool rebuild = true;  // theta of the current rho not built yet
  __syncthreads();      // A_minus in LDS
  const int last = a.max_iter > 1 ? a.max_iter : 1;
  for (int iter = 0; iter < last; ++iter) {
    if (!done) {
      const bool sc_ = mod_zero(iter, a.check_every);
      bool active = (iter < a.max_iter) && (!sc_ || tl);
      active = active || iter < 1;
      if (!active) done = true;
    }
    if (done) break;
    if (rebuild) {
      setup(rho);  // S and Phiinv of the new rho (admm.py:515-528)
      rebuild = false;
    }
    const R rho_f = rho * a.rho_f_factor;

    // gamma = sigma x - q + C^T (rho_f c - y_f) + G^T (rho z - y_g) (admm.py:157-174)
    if (dr) sc[(t - 1) * nx + i] = rho_f * cq[uf] - yf;
    if (a0r) sc[N * nx + i] = rho_f * c0q[uf0] - yf0;
    if (gr) sz[tid] = rho * z - yg;
    __syncthreads();
    R gam = R(0);
    if (el) {
      gam = a.sigma * x - qq[ue];
      if (t < N) {
        const R* ac = aml + t * nx * P + i;
        R s = R(0);
        #pragma unroll 1
        for (int j = 0; j < nx; ++j) s += ac[j * P] * sc[t * nx + j];
        gam += s;
      }
      if (t > 0) gam += (i < nx) ? -sc[(t - 1) * nx + i] : R(0);
      if (m) {
        const unsigned gt = (unsigned)(t * m * n + i);
        R s = R(0);
        #pragma unroll 1
        for (int r = 0; r < m; ++r) s += Gq[gt + r * n] * sz[t * m + r];
        gam += s;
      }
      if (t == 0) {
        R s = R(0);
        #pragma unroll 1
        for (int r = 0; r < n0; ++r) s += A0q[r * n + i] * sc[N * nx + r];
        gam += s;
      }
    }

    // PCG on S xt = gamma from xt = x (pcg_primal.py:70-175)
    R xt = x;
    if (el) vp[ev] = x;
    __syncthreads();
    R rv = R(0);
    if (el) rv = gam - (theta_dot(vp) + offdiag(vp, rho_f));
    if (el) vr[ev] = rv;
    __syncthreads();
    R rt = apply_phiinv(rho_f);
    R eta = block_sum(rv * rt);
    R pv = rt;
    if (el) vp[ev] = pv;
    const R eta0 = rabs(eta);
    int pit = 0;
    bool running = !(eta0 <= R(1e-12));
    while (running) {
      const bool conv = rabs(eta) < R(1e-12) + pa.pcg_eps * eta0;
      const bool cont = (!conv && pit <= pa.pcg_max_iter - 1) || pit < 1;
      if (!cont) break;
      __syncthreads();  // p complete in LDS
      const R qq = el ? theta_dot(vp) + offdiag(vp, rho_f) : R(0);
      const R vq = block_sum(pv * qq);
      const R al = eta / vq;
      xt += al * pv;
      rv -= al * qq;
      if (el) vr[ev] = rv;
      __syncthreads();
      rt = apply_phiinv(rho_f);
      const R etap = block_sum(rv * rt);
      const R be = etap / eta;
      pv = rt + be * pv;
      if (el) vp[ev] = pv;
      eta = etap;
      ++pit;
    }
    if (pa.pcg_iters && tid == 0 && iter < a.max_iter) pa.pcg_iters[boff * a.max_iter + iter] = (uint32_t)pit;

    // C/G products on xt, relaxation, projection, duals (admm.py:884-931)
    __syncthreads();
    if (el) vp[ev] = xt;
    __syncthreads();
    if (dr) {
      const R* ar_ = aml + ((t - 1) * nx + i) * P;
      const R* sp = vp + (t - 1) * P;
      R s = R(0);
#pragma unroll
      for (int k = 0; k < NC; ++k) s += ar_[k] * sp[k];
      const R cx = s - vp[ev];  // A_minus_{t-1} xt_{t-1} + A_plus_{t-1} xt_t
      const R cv = cq[uf];
      yf = yf + rho_f * (alpha * cx + oma * cv - cv);
    }
    if (a0r) {
      R s = R(0);
#pragma unroll
      for (int k = 0; k < NC; ++k) s += A0q[uf0 * n + k] * vp[k];
      const R c0v = c0q[uf0];
      yf0 = yf0 + rho_f * (alpha * s + oma * c0v - c0v);
    }
    if (gr) {
      const R* sp = vp + tg * P;
      R gx = R(0);
#pragma unroll
      for (int k = 0; k < NC; ++k) gx += Gq[ug * n + k] * sp[k];
      const R zt = alpha * gx + oma * z + yg / rho;
      const R proj = rmin(rmax(zt, lq[ug]), uq[ug]);
      R zn, xin;
      if (slack) {
        const R frac = gs / (gs + rho);
        zn = (R(1) - frac) * zt + frac * proj;
        xin = (rho / (gs + rho)) * (proj - zt);
      } else {
        zn = proj;
        xin = R(0);
      }
      yg = yg + rho * (alpha * gx + oma * z - zn);
      z = zn;
      xi = xin;
    }
    x = alpha * xt + oma * x;
    it = iter + 1;

    // residuals and adaptive rho on the new iterate (admm.py:266-344, :491-528)
    if (mod_zero(iter, a.check_every)) {
      __syncthreads();
      if (el) vp[ev] = x;
      if (dr) sc[(t - 1) * nx + i] = yf;
      if (a0r) sc[N * nx + i] = yf0;
      if (gr) sz[tid] = yg;
      __syncthreads();
      // rp, nCx, nc, nGx, nz, rd, nPx, nAty, nq, nxi, nyg (infinity norms)
      R v[11] = {R(0), R(0), R(0), R(0), R(0), R(0), R(0), R(0), R(0), R(0), R(0)};
      if (el) {
        const R* sp = vp + t * P;
        R px = R(0);
        #pragma unroll 1
        for (int k = 0; k < n; ++k) px += Dq[ue * n + k] * sp[k];
        R aty = R(0);
        if (t == 0) {
          R s = R(0);
          #pragma unroll 1
          for (int r = 0; r < n0; ++r) s += A0q[r * n + i] * sc[N * nx + r];
          aty += s;
        }
        if (t < N) {
          const R* ac = aml + t * nx * P + i;
          R s = R(0);
          #pragma unroll 1
          for (int j = 0; j < nx; ++j) s += ac[j * P] * sc[t * nx + j];
          aty += s;
        }
        if (t > 0) aty += (i < nx) ? -sc[(t - 1) * nx + i] : R(0);
        if (m) {
          const unsigned gt = (unsigned)(t * m * n + i);
          R s = R(0);
          #pragma unroll 1
          for (int r = 0; r < m; ++r) s += Gq[gt + r * n] * sz[t * m + r];
          aty += s;
        }
        const R qv = qq[ue];
        v[5] = rabs(px + qv + aty);
        v[6] = rabs(px);
        v[7] = rabs(aty);
        v[8] = rabs(qv);
      }
      if (dr) {
        const R* ar_ = aml + ((t - 1) * nx + i) * P;
        const R* sp = vp + (t - 1) * P;
        R s = R(0);
        #pragma unroll 1
        for (int k = 0; k < n; ++k) s += ar_[k] * sp[k];
        const R cx = s - vp[ev];
        const R cv = cq[uf];
        v[0] = rabs(cx - cv);
        v[1] = rabs(cx);
        v[2] = rabs(cv);
      }
      if (a0r) {
        R s = R(0);
        #pragma unroll 1
        for (int k = 0; k < n; ++k) s += A0q[uf0 * n + k] * vp[k];
        const R c0v = c0q[uf0];
        v[0] = rmax(v[0], rabs(s - c0v));
        v[1] = rmax(v[1], rabs(s));
        v[2] = rmax(v[2], rabs(c0v));
      }
      if (gr) {
        const R* sp = vp + tg * P;
        R gx = R(0);
        #pragma unroll 1
        for (int k = 0; k < n; ++k) gx += Gq[ug * n + k] * sp[k];
        v[0] = rmax(v[0], rabs(gx - z));
        v[3] = rabs(gx);
        v[4] = rabs(z);
        if (slack) {
          v[5] = rmax(v[5], rabs(gs * xi + yg));
          v[9] = rabs(xi);
          v[10] = rabs(yg);
        }
      }
      // workgroup maxima: wavefront maxima, then thread k < 11 folds value k
      R* rm = red + 64;
#pragma unroll
      for (int k = 0; k < 11; ++k) {
        const R w = wave_max(v[k]);
        if (lane == 0) rm[k * NW + wid] = w;
      }
      __syncthreads();
      if (tid < 11) {
        R mx = R(0);
        for (int w = 0; w < NW; ++w) mx = rmax(mx, rm[tid * NW + w]);
        rm[11 * NW + tid] = mx;
      }
      __syncthreads();
      const R* r_ = rm + 11 * NW;
      const R np = rmax(rmax(r_[1], r_[3]), rmax(r_[2], r_[4]));
      R nd = rmax(rmax(r_[6], r_[7]), r_[8]);
      if (slack) nd = rmax(nd, rmax(gs * r_[9], r_[10]));
      const R pn = r_[0] / (R(1e-10) + np), dn = r_[5] / (R(1e-10) + nd);
      const R cand = rmin(rmax(rho * r_sqrt(pn / dn), a.rho_min), a.rho_max);
      const R ratio = rmax(cand / rho, rho / cand);
      tl = (r_[0] > a.eps_abs + a.eps_rel * np) || (r_[5] > a.eps_abs + a.eps_rel * nd);
      const bool conv = !tl;
      bool keep = iter < 2 || !mod_zero(iter, a.adapt_every);
      keep = keep || conv;
      keep = keep || ratio < a.rho_tol;
      if (!keep) {
        rho = cand;
        rebuild = true;
      }
    }
    __syncthreads();  // the shared vectors are rewritten by the next iteration
  }

  // ---- state back to the caller ---------------------------------------------------
  if (el) a.st.x[boff * T * n + ue] = x;
  if (gr) {
    a.st.z[boff * T * m + ug] = z;
    a.st.y_g[boff * T * m + ug] = yg;
    a.st.xi[boff * T * m + ug] = xi;
  }
  if (dr) a.st.y_f[boff * N * nx + uf] = yf;
  if (a0r) a.st.y_f0[boff * n0 + uf0] = yf0;
  if (tid == 0) {
    a.st.rho[b] = rho;
    a.iters_out[b] = (uint32_t)it;
  }
}

// ---------------------------------------------------------------------------
// Row-broadcast variant (n <= 16, T <= 64): stage t of a problem occupies one
// 16-lane row of a wavefront (thread 16 t + i, lanes i >= n idle), so every
// product with a block of the stage's own vector -- theta_t p_t, theta_t^{-1}
// r_t and the Gauss-Jordan pivot rows of the setup -- takes its operands by
// DPP row broadcasts (row_newbcast) instead of LDS reads.  Only the
// neighbouring stages' elements cross rows: each lane reads s_{t-1}[i] and
// s_{t+1}[i] from LDS and broadcasts those within its row.  A PCG iteration
// has four workgroup barriers (p complete, p.q, v complete, r.z) and each lane
// makes two LDS reads per product with S or Phiinv.  Same iteration and
// stopping rules as admm_pcg_lds_kernel, and the same product form.

constexpr int kPcgRow = 16;  // lanes per stage

struct PcgDppLayout {
  int pb, vb, sc, sz, red, am, az;  // element offsets (in R)
  size_t bytes;
};

template <typename R>
__host__ __device__ inline PcgDppLayout pcg_dpp_layout(const Dims& d, bool amr) {
  PcgDppLayout L;
  const int P = pcg_pitch(d.n);
  int off = 0;
  auto take = [&](int cnt) {
    const int o = off;
    off += (cnt + 3) & ~3;
    return o;
  };
  L.pb = take(d.T * kPcgRow);
  L.vb = take(d.T * kPcgRow);
  L.sc = take(d.N * d.nx + d.n0);
  L.sz = take(d.T * d.m > 0 ? d.T * d.m : 1);
  L.red = take(2 * 32 + 12 * 16 + 8);
  L.am = amr ? 0 : take(d.N * d.nx * P);
  L.az = amr ? 0 : take(kPcgRow * P);  // zero rows for lanes without an A_minus row or column
  L.bytes = (size_t)off * sizeof(R);
  return L;
}

inline bool pcg_dpp_fits(const Dims& d) {
  return (d.n == 6 || d.n == 9 || d.n == 16) && d.T * kPcgRow <= kPcgThreads && d.T * d.m <= kPcgThreads &&
         d.n0 <= d.n && d.nx < d.n;
}

template <typename R, int NC, bool AMR>
__global__ __launch_bounds__(kPcgThreads) void admm_pcg_dpp_kernel(AdmmPcgArgs<R> pa) {
  const AdmmArgs<R>& a = pa.a;
  const Dims d = a.d;
  constexpr int n = NC, W = kPcgRow;
  constexpr int NW = kPcgThreads / kWave;
  static_assert(NW == 16, "block sums read one wavefront sum per lane of a 16-lane row");
  const int T = d.T, N = d.N, nx = d.nx, n0 = d.n0, m = d.m;
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const int P = pcg_pitch(n);
  extern __shared__ __align__(16) unsigned char smem_raw[];
  R* sm = reinterpret_cast<R*>(smem_raw);
  const PcgDppLayout L = pcg_dpp_layout<R>(d, AMR);
  R* pb = sm + L.pb;  // the vector a product with S reads, lane 16 t + i
  R* vb = sm + L.vb;  // v = theta^{-1} r, the same layout
  R* sc = sm + L.sc;
  R* sz = sm + L.sz;
  R* red = sm + L.red;
  R* aml = sm + L.am;
  R* az = sm + L.az;

  // ---- roles ------------------------------------------------------------------
  const int t = tid / W, i = tid - (tid / W) * W;  // row of this lane (a stage if t < T)
  const bool st = t < T;
  const bool el = st && i < n;
  const bool gr = m > 0 && tid < T * m;
  const int tg = gr ? tid / m : 0;
  const bool dr = el && t >= 1 && i < nx;   // dynamics row (t - 1, i)
  const bool a0r = el && t == 0 && i < n0;  // row i of A0
  const bool wl = wid * (kWave / W) < T;    // the wavefront holds a stage (uniform)
  const size_t boff = (size_t)b;
  const R* const Dq = a.qp.D + boff * T * n * n;
  const R* const Gq = a.qp.G + boff * T * m * n;
  const R* const A0q = a.qp.A0 + boff * n0 * n;
  const R* const Aq = a.qp.Am + boff * N * nx * n;
  const R* const qq = a.qp.q + boff * T * n;
  const R* const cq = a.qp.c + boff * N * nx;
  const R* const c0q = a.qp.c0 + boff * n0;
  const R* const lq = a.qp.l + boff * T * m;
  const R* const uq = a.qp.u + boff * T * m;
  const unsigned ue = el ? (unsigned)(t * n + i) : 0u;                 // element (t, i)
  const unsigned ug = gr ? (unsigned)tid : 0u;                         // G row (tg, rg)
  const unsigned uf = dr ? (unsigned)((t - 1) * nx + i) : 0u;          // dynamics row (t - 1, i)
  const unsigned uf0 = a0r ? (unsigned)i : 0u;                         // A0 row i

  // ---- A_minus: row i of A_minus_{t-1} (dr lanes) and column i of A_minus_t ----------
  R amr[NC], amc[NC];
  if (AMR) {
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      amr[k] = dr ? Aq[uf * n + k] : R(0);
      amc[k] = (el && t < N && k < nx) ? Aq[(unsigned)((t * nx + k) * n + i)] : R(0);
    }
  } else {
    for (int e = tid; e < N * nx * n; e += kPcgThreads) {
      const int r = e / n, k = e - (e / n) * n;
      aml[r * P + k] = Aq[(unsigned)e];
    }
    for (int e = tid; e < W * P; e += kPcgThreads) az[e] = R(0);
  }
  // LDS rows of the A_minus blocks (zero rows for lanes that own none)
  const R* const arow = dr ? aml + ((t - 1) * nx + i) * P : az;
  const R* const acol = (el && t < N) ? aml + t * nx * P + i : az + (i < P ? i : 0);

  // ---- state in registers -------------------------------------------------------
  R x = el ? a.st.x[boff * T * n + ue] : R(0);
  R z = R(0), yg = R(0), xi = R(0);
  if (gr) {
    z = a.st.z[boff * T * m + ug];
    yg = a.st.y_g[boff * T * m + ug];
    xi = a.st.xi[boff * T * m + ug];
  }
  R yf = dr ? a.st.y_f[boff * N * nx + uf] : R(0);
  R yf0 = a0r ? a.st.y_f0[boff * n0 + uf0] : R(0);
  const bool slack = a.use_slack && m > 0;
  const R gs = (slack && a.qp.slack_w) ? a.qp.slack_w[b] : R(0);
  R rho = a.st.rho[b];
  const R alpha = a.alpha, oma = R(1) - a.alpha;
  __syncthreads();  // A_minus in LDS

  // ---- theta_t and theta_t^{-1} (fp64, rounded on store) --------------------------
  R th[NC], ti[NC];
  auto setup = [&](R rho_v) __attribute__((always_inline)) {
    const double rho_i = (double)rho_v, rho_f = rho_i * (double)a.rho_f_factor;
    int ii = i;  // kept in a register: the comparisons below are made here
    __asm__ volatile("" : "+v"(ii));
    double ar[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) ar[k] = 0.0;
    if (el) {
      // D_t + sigma I + rho G_t^T G_t + rho_f (A0^T A0 [t = 0] + A_minus_t^T A_minus_t [t < N]
      // + A_plus_{t-1}^T A_plus_{t-1} [t > 0]), A_plus = [-I 0]
#pragma unroll
      for (int k = 0; k < NC; ++k) ar[k] = (double)Dq[ue * n + k] + (k == ii ? (double)a.sigma : 0.0);
      if (m) {
        const unsigned gt = (unsigned)(t * m * n);
#pragma unroll 1
        for (int r = 0; r < m; ++r) {
          const double gi = rho_i * (double)Gq[gt + r * n + ii];
#pragma unroll
          for (int k = 0; k < NC; ++k) ar[k] += gi * (double)Gq[gt + r * n + k];
        }
      }
      if (t == 0) {
#pragma unroll 1
        for (int r = 0; r < n0; ++r) {
          const double ai = rho_f * (double)A0q[r * n + ii];
#pragma unroll
          for (int k = 0; k < NC; ++k) ar[k] += ai * (double)A0q[r * n + k];
        }
      }
      if (t < N) {
        const unsigned at = (unsigned)(t * nx * n);
#pragma unroll 1
        for (int r = 0; r < nx; ++r) {
          const double ai = rho_f * (double)Aq[at + r * n + ii];
#pragma unroll
          for (int k = 0; k < NC; ++k) ar[k] += ai * (double)Aq[at + r * n + k];
        }
      }
#pragma unroll
      for (int k = 0; k < NC; ++k)
        if (t > 0 && ii < nx && k == ii) ar[k] += rho_f;
    }
#pragma unroll
    for (int k = 0; k < NC; ++k) th[k] = el ? (R)ar[k] : R(0);
    // Gauss-Jordan in place without pivoting (theta_t is SPD): row i of
    // theta_t^{-1}; pivot row k is lane k of the row
    if (wl)
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      double pk[NC];
#pragma unroll
      for (int j = 0; j < NC; ++j) pk[j] = row_bcast_at(ar[j], k);
      const double ip = 1.0 / pk[k];
      const double f = ar[k];
      const bool me = ii == k;
#pragma unroll
      for (int j = 0; j < NC; ++j)
        ar[j] = me ? ((j == k) ? ip : ar[j] * ip) : ((j == k) ? -f * ip : ar[j] - f * (pk[j] * ip));
    }
#pragma unroll
    for (int k = 0; k < NC; ++k) ti[k] = el ? (R)ar[k] : R(0);
  };

  // ---- products (every lane of the workgroup runs them) -----------------------------
  // phi_{t-1} s_{t-1} + phi_t^T s_{t+1}, s in buf (complete)
  auto offdiag = [&](const R* buf, R rho_f) __attribute__((always_inline)) -> R {
    const R sp = (st && t >= 1) ? buf[tid - W] : R(0);  // s_{t-1}[i]
    const R sn = (t < N) ? buf[tid + W] : R(0);          // s_{t+1}[i]
    R rw, cl;
    if (AMR) {
      rw = row_dot_dpp(amr, sp);
      cl = row_dot_dpp(amc, sn);
    } else {
      // one block's operands in registers at a time
      R w_[NC];
#pragma unroll
      for (int k = 0; k < NC; ++k) w_[k] = arow[k];
      rw = row_dot_dpp(w_, sp);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < NC; ++k) w_[k] = k < nx ? acol[k * P] : R(0);
      cl = row_dot_dpp(w_, sn);
    }
    R acc = R(0);
    acc -= rho_f * rw;
    acc -= rho_f * cl;
    return acc;
  };
  int rslot = 0;
  auto block_sum = [&](R v) __attribute__((always_inline)) -> R {
    v = wave_sum(v);
    R* rr = red + rslot * 32;
    rslot ^= 1;
    if (lane == 0) rr[wid] = v;
    __syncthreads();
    return row_sum(rr[lane & (NW - 1)]);  // the 16 wavefront sums, one per lane of each row
  };
  // rt = Phiinv r for this lane's r; returns rt (zero off the elements)
  auto apply_phiinv = [&](R r, R rho_f) __attribute__((always_inline)) -> R {
    R v = R(0);
    if (wl) v = row_dot_dpp(ti, r);
    if (st) vb[tid] = v;
    __syncthreads();
    R zt = R(0);
    if (wl) {
      const R u = offdiag(vb, rho_f) - r;
      zt = row_dot_dpp(ti, u);
    }
    return el ? zt : R(0);
  };
  // S s for this lane, s in buf (complete) and in the lane's own value
  auto apply_s = [&](R sv, const R* buf, R rho_f) __attribute__((always_inline)) -> R {
    R q = R(0);
    if (wl) q = row_dot_dpp(th, sv) + offdiag(buf, rho_f);
    return el ? q : R(0);
  };

  // ---- per-problem control state (as admm_pcg_chunk_kernel, one chunk) ------------
  int it = 0;
  bool done = false;
  bool tl = true;       // residuals above tolerance (the initial residuals are infinite)
  bool rebuild = true;  // theta of the current rho not built yet
  const int last = a.max_iter > 1 ? a.max_iter : 1;
  for (int iter = 0; iter < last; ++iter) {
    if (!done) {
      const bool sc_ = mod_zero(iter, a.check_every);
      bool active = (iter < a.max_iter) && (!sc_ || tl);
      active = active || iter < 1;
      if (!active) done = true;
    }
    if (done) break;
    if (rebuild) {
      setup(rho);  // S and Phiinv of the new rho (admm.py:515-528)
      rebuild = false;
    }
    const R rho_f = rho * a.rho_f_factor;

    // gamma = sigma x - q + C^T (rho_f c - y_f) + G^T (rho z - y_g) (admm.py:157-174)
    if (dr) sc[(t - 1) * nx + i] = rho_f * cq[uf] - yf;
    if (a0r) sc[N * nx + i] = rho_f * c0q[uf0] - yf0;
    if (gr) sz[tid] = rho * z - yg;
    __syncthreads();
    R gam = R(0);
    if (el) {
      gam = a.sigma * x - qq[ue];
      if (t < N) {
        R s_ = R(0);
#pragma unroll 1
        for (int j = 0; j < nx; ++j) s_ += Aq[(unsigned)((t * nx + j) * n + i)] * sc[t * nx + j];
        gam += s_;
      }
      if (t > 0) gam += (i < nx) ? -sc[(t - 1) * nx + i] : R(0);
      if (m) {
        const unsigned gt = (unsigned)(t * m * n + i);
        R s_ = R(0);
#pragma unroll 1
        for (int r = 0; r < m; ++r) s_ += Gq[gt + r * n] * sz[t * m + r];
        gam += s_;
      }
      if (t == 0) {
        R s_ = R(0);
#pragma unroll 1
        for (int r = 0; r < n0; ++r) s_ += A0q[r * n + i] * sc[N * nx + r];
        gam += s_;
      }
    }

    // PCG on S xt = gamma from xt = x (pcg_primal.py:70-175)
    R xt = x;
    if (st) pb[tid] = x;
    __syncthreads();
    const R sx = apply_s(x, pb, rho_f);
    R rv = el ? gam - sx : R(0);
    R rt = apply_phiinv(rv, rho_f);
    R eta = block_sum(rv * rt);
    R pv = rt;
    if (st) pb[tid] = pv;
    const R eta0 = rabs(eta);
    int pit = 0;
    bool running = !(eta0 <= R(1e-12));
    while (running) {
      const bool conv = rabs(eta) < R(1e-12) + pa.pcg_eps * eta0;
      const bool cont = (!conv && pit <= pa.pcg_max_iter - 1) || pit < 1;
      if (!cont) break;
      __syncthreads();  // p complete in LDS
      const R qv = apply_s(pv, pb, rho_f);
      const R vq = block_sum(pv * qv);
      const R al = eta / vq;
      xt += al * pv;
      rv -= al * qv;
      rt = apply_phiinv(rv, rho_f);
      const R etap = block_sum(rv * rt);
      const R be = etap / eta;
      pv = rt + be * pv;
      if (st) pb[tid] = pv;
      eta = etap;
      ++pit;
    }
    if (pa.pcg_iters && tid == 0 && iter < a.max_iter) pa.pcg_iters[boff * a.max_iter + iter] = (uint32_t)pit;

    // C/G products on xt, relaxation, projection, duals (admm.py:884-931)
    __syncthreads();
    if (st) pb[tid] = xt;
    __syncthreads();
    if (dr) {
      const R* sp = pb + (t - 1) * W;
      R s_ = R(0);
#pragma unroll
      for (int k = 0; k < NC; ++k) s_ += (AMR ? amr[k] : arow[k]) * sp[k];
      const R cx = s_ - xt;  // A_minus_{t-1} xt_{t-1} + A_plus_{t-1} xt_t
      const R cv = cq[uf];
      yf = yf + rho_f * (alpha * cx + oma * cv - cv);
    }
    if (a0r) {
      R s_ = R(0);
#pragma unroll
      for (int k = 0; k < NC; ++k) s_ += A0q[uf0 * n + k] * pb[k];
      const R c0v = c0q[uf0];
      yf0 = yf0 + rho_f * (alpha * s_ + oma * c0v - c0v);
    }
    if (gr) {
      const R* sp = pb + tg * W;
      R gx = R(0);
#pragma unroll
      for (int k = 0; k < NC; ++k) gx += Gq[ug * n + k] * sp[k];
      const R zt = alpha * gx + oma * z + yg / rho;
      const R proj = rmin(rmax(zt, lq[ug]), uq[ug]);
      R zn, xin;
      if (slack) {
        const R frac = gs / (gs + rho);
        zn = (R(1) - frac) * zt + frac * proj;
        xin = (rho / (gs + rho)) * (proj - zt);
      } else {
        zn = proj;
        xin = R(0);
      }
      yg = yg + rho * (alpha * gx + oma * z - zn);
      z = zn;
      xi = xin;
    }
    x = alpha * xt + oma * x;
    it = iter + 1;

    // residuals and adaptive rho on the new iterate (admm.py:266-344, :491-528)
    if (mod_zero(iter, a.check_every)) {
      __syncthreads();
      if (st) pb[tid] = x;
      if (dr) sc[(t - 1) * nx + i] = yf;
      if (a0r) sc[N * nx + i] = yf0;
      if (gr) sz[tid] = yg;
      __syncthreads();
      // rp, nCx, nc, nGx, nz, rd, nPx, nAty, nq, nxi, nyg (infinity norms)
      R v[11] = {R(0), R(0), R(0), R(0), R(0), R(0), R(0), R(0), R(0), R(0), R(0)};
      if (el) {
        const R* sp = pb + t * W;
        R px = R(0);
#pragma unroll 1
        for (int k = 0; k < n; ++k) px += Dq[ue * n + k] * sp[k];
        R aty = R(0);
        if (t == 0) {
          R s_ = R(0);
#pragma unroll 1
          for (int r = 0; r < n0; ++r) s_ += A0q[r * n + i] * sc[N * nx + r];
          aty += s_;
        }
        if (t < N) {
          R s_ = R(0);
#pragma unroll 1
          for (int j = 0; j < nx; ++j) s_ += Aq[(unsigned)((t * nx + j) * n + i)] * sc[t * nx + j];
          aty += s_;
        }
        if (t > 0) aty += (i < nx) ? -sc[(t - 1) * nx + i] : R(0);
        if (m) {
          const unsigned gt = (unsigned)(t * m * n + i);
          R s_ = R(0);
#pragma unroll 1
          for (int r = 0; r < m; ++r) s_ += Gq[gt + r * n] * sz[t * m + r];
          aty += s_;
        }
        const R qv = qq[ue];
        v[5] = rabs(px + qv + aty);
        v[6] = rabs(px);
        v[7] = rabs(aty);
        v[8] = rabs(qv);
      }
      if (dr) {
        const R* sp = pb + (t - 1) * W;
        R s_ = R(0);
#pragma unroll 1
        for (int k = 0; k < n; ++k) s_ += Aq[uf * n + k] * sp[k];
        const R cx = s_ - pb[tid];
        const R cv = cq[uf];
        v[0] = rabs(cx - cv);
        v[1] = rabs(cx);
        v[2] = rabs(cv);
      }
      if (a0r) {
        R s_ = R(0);
#pragma unroll 1
        for (int k = 0; k < n; ++k) s_ += A0q[uf0 * n + k] * pb[k];
        const R c0v = c0q[uf0];
        v[0] = rmax(v[0], rabs(s_ - c0v));
        v[1] = rmax(v[1], rabs(s_));
        v[2] = rmax(v[2], rabs(c0v));
      }
      if (gr) {
        const R* sp = pb + tg * W;
        R gx = R(0);
#pragma unroll 1
        for (int k = 0; k < n; ++k) gx += Gq[ug * n + k] * sp[k];
        v[0] = rmax(v[0], rabs(gx - z));
        v[3] = rabs(gx);
        v[4] = rabs(z);
        if (slack) {
          v[5] = rmax(v[5], rabs(gs * xi + yg));
          v[9] = rabs(xi);
          v[10] = rabs(yg);
        }
      }
      // workgroup maxima: wavefront maxima, then thread k < 11 folds value k
      R* rm = red + 64;
#pragma unroll
      for (int k = 0; k < 11; ++k) {
        const R w = wave_max(v[k]);
        if (lane == 0) rm[k * NW + wid] = w;
      }
      __syncthreads();
      if (tid < 11) {
        R mx = R(0);
        for (int w = 0; w < NW; ++w) mx = rmax(mx, rm[tid * NW + w]);
        rm[11 * NW + tid] = mx;
      }
      __syncthreads();
      const R* r_ = rm + 11 * NW;
      const R np = rmax(rmax(r_[1], r_[3]), rmax(r_[2], r_[4]));
      R nd = rmax(rmax(r_[6], r_[7]), r_[8]);
      if (slack) nd = rmax(nd, rmax(gs * r_[9], r_[10]));
      const R pn = r_[0] / (R(1e-10) + np), dn = r_[5] / (R(1e-10) + nd);
      const R cand = rmin(rmax(rho * r_sqrt(pn / dn), a.rho_min), a.rho_max);
      const R ratio = rmax(cand / rho, rho / cand);
      tl = (r_[0] > a.eps_abs + a.eps_rel * np) || (r_[5] > a.eps_abs + a.eps_rel * nd);
      const bool conv = !tl;
      bool keep = iter < 2 || !mod_zero(iter, a.adapt_every);
      keep = keep || conv;
      keep = keep || ratio < a.rho_tol;
      if (!keep) {
        rho = cand;
        rebuild = true;
      }
    }
    __syncthreads();  // the shared vectors are rewritten by the next iteration
  }

  // ---- state back to the caller ---------------------------------------------------
  if (el) a.st.x[boff * T * n + ue] = x;
  if (gr) {
    a.st.z[boff * T * m + ug] = z;
    a.st.y_g[boff * T * m + ug] = yg;
    a.st.xi[boff * T * m + ug] = xi;
  }
  if (dr) a.st.y_f[boff * N * nx + uf] = yf;
  if (a0r) a.st.y_f0[boff * n0 + uf0] = yf0;
  if (tid == 0) {
    a.st.rho[b] = rho;
    a.iters_out[b] = (uint32_t)it;
  }
}

}  // namespace tmpc
