// Streaming fused ADMM for the explicit-integrator structure
// (A_plus_t = [-I 0] and E_t = 0: every dynamics linearized by an explicit
// integrator, turbompc/solvers/turbompc_solver.py:1098-1156).
//
// Same iteration as admm_chunk_kernel (admm_direct.hpp), which keeps the
// reference's ADMMSolver._solve_jax_loop semantics (admm.py:795-1049); this
// path differs in how data reaches the lanes.
//
// Stage records.  Before the first iteration, stage_pack_kernel copies the QP
// and the warm start into stage-major workspace arrays, so that for a stage t
// the P problems of one wavefront (b0 .. b0+P-1) sit in one contiguous run:
//   th [T][B][pitch]  Theta_t^{-1} (packed, written by factor_std_kernel)
//   am [T][B][amp]    M_t = [A_minus_t; G_t], (nx + m) x n (A_minus_N = 0)
//   rv [T][B][rvp]    x q (stage t) | y = [y_f; y_g] | cz = [c; z] | xi l u
//   dm [T][B][dmp]    D_t (packed, or its diagonal when the caller vouches that
//                     every D_t is diagonal; iterations that evaluate the residuals)
// The constraint rows of a stage are stacked: row r < nx is dynamics row t,
// row nx + j is inequality j, so lane r of a problem's group owns both the
// row of M_t and the matching entries of y and cz, and one dot product with
// M_t serves both kinds of constraint.
// and stage_unpack_kernel writes the state back after the last iteration.
//
// Sweeps.  Every sweep over the stages runs in batches of DPF stages: the
// runs of batch k are copied from registers into LDS slots, the 128-bit loads
// of batch k+1 are issued, and batch k is computed from LDS.  One memory
// latency is paid per batch, not one per dependent access.
//
// The w_t / gamma_t trajectory ([T][n] per problem) stays in LDS for the whole
// chunk: the forward sweep overwrites gamma_t with w_t, the backward sweep
// overwrites w_{t+1} with the next iteration's gamma_{t+1}.  y_f0 and c0 stay
// in registers; A0 stays in LDS.
//
// HBM traffic per iteration and problem: Theta^{-1} and M twice (forward and
// backward sweep), the rv record once (D_t too when the residuals are due),
// the written state once.
#pragma once
#include <type_traits>

#include "admm_direct.hpp"
#include "stream_dpp.hpp"

namespace tmpc {

// 16-byte vectors as clang ext vectors (plain values that stay in registers;
// HIP's float4 class wraps a union, which keeps arrays of it in scratch).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));

template <typename R>
struct Vec16;
template <>
struct Vec16<float> {
  using T = f32x4;
  static constexpr int W = 4;
};
template <>
struct Vec16<double> {
  using T = f64x2;
  static constexpr int W = 2;
};

__host__ __device__ inline constexpr int up4(int x) { return (x + 3) & ~3; }

// Stage-record geometry (elements of R).
struct RecGeom {
  int amp;                      // M_t = [A_minus_t; G_t] block pitch
  int rvp;                      // rv record pitch
  int dmp;                      // D_t record pitch
  bool diag;                    // D_t records hold the diagonal only
  int x, q, y, cz, xi, l, u;    // offsets inside an rv record
  int yf, yg, c, z;             // y = [y_f; y_g], cz = [c; z]
};

// Without the flag: the larger (packed) D_t record, for workspace sizing.
__host__ __device__ inline RecGeom rec_geom(const Dims& d, bool diag = false) {
  RecGeom r;
  const int n = d.n, m = d.m, nx = d.nx;
  r.amp = up4((nx + m) * n);
  r.diag = diag;
  r.dmp = diag ? up4(n) : th_pitch(n);
  r.x = 0;
  r.q = n;
  r.y = 2 * n;
  r.cz = r.y + nx + m;
  r.xi = r.cz + nx + m;
  r.l = r.xi + m;
  r.u = r.l + m;
  r.rvp = up4(r.u + m);
  r.yf = r.y;
  r.yg = r.y + nx;
  r.c = r.cz;
  r.z = r.cz + nx;
  return r;
}

// Compile-time caps of the streaming kernel (host checks, else the generic
// kernel runs): nx <= n - 1 and either m <= kMaxStreamM, nx + m <= n (the
// stacked constraint rows of a stage fit the problem's n lanes), or a wide
// form with NL > NC row lanes per problem: n = 9 (the obstacle workload's 6
// states and 3 controls) with m <= kWideMaxM, nx + m <= kWideRows, up to three
// problems per wavefront; n = 16 (box constraints on every variable, as in the
// linear workload) with m <= kWide16MaxM, nx + m <= kWide16Rows, a half-wave
// per problem.
constexpr int kMaxStreamM = 8;
constexpr int kWideRows = 17;
constexpr int kWideMaxM = 12;
constexpr int kWide16Rows = 32;
constexpr int kWide16MaxM = 28;

// NL: lanes of a problem's group that own a stacked constraint row (NL >= NC);
// MM: most inequality rows per stage.
template <typename R, int NC, int P, int NL = NC, int MM = kMaxStreamM>
struct StreamShape {
  static constexpr int W = Vec16<R>::W;
  static constexpr int PITCH = th_pitch(NC);
  static constexpr int AMP_MAX = up4(NL * NC);
  static constexpr int RVP_MAX = up4(2 * NC + 2 * NL + 3 * MM);
  static constexpr int CH_TH = (P * PITCH / W + kWave - 1) / kWave;  // 16-byte chunks per lane
  static constexpr int CH_AM = (P * AMP_MAX / W + kWave - 1) / kWave;
  static constexpr int CH_RV = (P * RVP_MAX / W + kWave - 1) / kWave;
};

constexpr int kNV = 8;  // per-lane broadcast vectors in LDS

// One broadcast vector holds P group slots of up4(64 / P) entries, so that
// every group's slot starts on a 16-byte boundary (16-byte vector reads).
__host__ __device__ inline constexpr int vec_stride(int P) { return P * up4(kWave / P); }

// LDS layout in elements of R (host and device agree).  The DPF Theta^{-1}
// slots come first at a compile-time stride (P x pitch), so one set of
// per-lane row addresses serves every slot through the immediate offset of
// the LDS instructions.
struct StreamLayout {
  int wg;   // [P][T][n]          w_t / gamma_t trajectory
  int th;   // [DPF][P][pitch]    Theta_t^{-1}
  int rv;   // [DPF][P][rvp]
  int dm;   // [DPF][P][dmp]      D_t (iterations that evaluate the residuals)
  int am;   // [max(DPF, 2)][P][amp] (then n x n zeros)
  int a0;   // [P][n0 n]
  int vec;  // [kNV][vec_stride(P)]
  int spill;  // 16-byte dump for the stores of lanes past a run
  int total;
};

__host__ __device__ inline StreamLayout stream_layout(const Dims& d, int P, int DPF, bool diag) {
  const RecGeom g = rec_geom(d, diag);
  StreamLayout L;
  L.wg = 0;
  L.th = up4(P * d.T * d.n);
  L.rv = L.th + DPF * P * th_pitch(d.n);
  L.dm = L.rv + DPF * P * g.rvp;
  L.am = L.dm + DPF * P * g.dmp;
  // at least two M slots: the backward sweep holds the blocks of stages t and t-1
  int end = L.am + (DPF > 2 ? DPF : 2) * P * g.amp;
  if (end < L.th + 12 * kWave) end = L.th + 12 * kWave;  // the residual reduction reuses the slots
  // n x n zeros: column products read all NL rows of a block, so the rows past
  // the last stacked block land here (rows past other blocks land on the
  // next block's data); every such row meets a zero vector entry.  NL rows
  // overshoot a block of nx + m rows by (NL - nx - m) n < n n entries (NL = n,
  // or the wide form's kWideRows with nx + m > n)
  L.a0 = up4(end + d.n * d.n);
  L.vec = up4(L.a0 + P * d.n0 * d.n);
  L.spill = L.vec + kNV * vec_stride(P);
  L.total = L.spill + 4;
  return L;
}

template <typename R>
struct StreamArgs {
  Dims d;
  const R* th;  // [T][B][pitch]
  const R* dm;  // [T][B][dmp]
  const R* am;  // [N][B][amp]
  R* rv;        // [T][B][rvp]
  const R *A0, *c0, *slack_w;
  R *y_f0, *rho;
  int32_t* ctl;  // [B][4]: it, done, refactor flag
  R* res;        // [B][8]
  uint32_t* iters_out;
  R sigma, alpha, rho_f_factor, eps_abs, eps_rel, rho_min, rho_max, rho_tol;
  int max_iter, check_every, adapt_every, use_slack;
  int diag;  // D_t records hold the diagonal (RecGeom)
  int it_lo, it_hi, first_chunk;
  // SQP step (optional, first chunk): first-order check of the input iterate
  // and the activity test act_out = act_in && conv > chk_tol; a problem that
  // fails it runs no iteration.  With chk_conv NULL and act_in set, the
  // activity is given: no check, the problems with act_in = 0 run no
  // iteration.
  R *chk_conv, *chk_eq, *chk_iq, *chk_g;
  const uint8_t* act_in;
  uint8_t* act_out;
  R chk_tol;
  // stage-invariant A_minus entries (AINV form): amask [kAinvWords], bit e set
  // when entry e of the row-major nx x n block varies over the stages
  // (ainv_mask_kernel); ac [N][B][nv] the nv varying entries of each
  // problem's A_minus_t in row-major order, written by the first chunk
  const uint32_t* amask;
  R* ac;
};

// ---- stage-invariant A_minus entries ---------------------------------------------

// Linearized dynamics often have entries that no linearization point changes
// (a rigid body's Jacobian with respect to position and velocity: [I; 0] and
// [dt I; I]); for the quadrotor 97 of the 221 entries of A_minus_t.  The AINV
// form of the streaming kernel keeps those entries resident in LDS and
// streams the others.  The mask is found on the device, bit for bit, on every
// call: entry e is invariant when A_minus_t[e] == A_minus_0[e] as bit patterns
// for every t < N of every problem, so the LDS slots hold exactly the values
// the whole records would.
constexpr int kAinvMaxEntries = 224;  // nx n of the AINV form (7 mask words)
constexpr int kAinvWords = kAinvMaxEntries / 32;
constexpr int kAinvWaves = 4;  // problems per workgroup of ainv_partial_kernel

// Partial masks, one workgroup per kAinvWaves problems: wavefront w compares
// problem b's stage records t = 1..N-1 with its stage 0, 16 bytes per lane
// (bit patterns), and the workgroup's OR of the varying bits lands in
// part[blockIdx.x][8], so that no global atomics are needed.
template <typename R>
__global__ __launch_bounds__(kWave * kAinvWaves) void ainv_partial_kernel(Dims d, const R* __restrict__ am,
                                                                         uint32_t* __restrict__ part) {
  using V = typename Vec16<R>::T;
  constexpr int W = Vec16<R>::W, CQ = (kAinvMaxEntries / W + kWave - 1) / kWave, LPW = 32 / W;
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  __shared__ uint32_t acc[8];
  const int lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  if (threadIdx.x < 8) acc[threadIdx.x] = 0;
  __syncthreads();
  const int b = blockIdx.x * kAinvWaves + wv, ne = d.nx * d.n, B = d.B, N = d.N;
  const int amp = rec_geom(d).amp;
  uint32_t bits[CQ] = {};
  if (b < B) {
    i32x4 a0[CQ];
#pragma unroll
    for (int c = 0; c < CQ; ++c) {
      const int q = c * kWave + lane;
      a0[c] = q * W < ne ? __builtin_bit_cast(i32x4, *reinterpret_cast<const V*>(am + (size_t)b * amp + q * W))
                         : i32x4{};
    }
#pragma unroll 4
    for (int t = 1; t < N; ++t) {
#pragma unroll
      for (int c = 0; c < CQ; ++c) {
        const int q = c * kWave + lane;
        if (q * W < ne) {
          const i32x4 v =
              __builtin_bit_cast(i32x4, *reinterpret_cast<const V*>(am + ((size_t)t * B + b) * amp + q * W));
#pragma unroll
          for (int k = 0; k < W; ++k) {  // entry k of the chunk: 32-bit word(s) k * 4 / W ..
            bool ne_k;
            if constexpr (W == 4)
              ne_k = v[k] != a0[c][k];
            else
              ne_k = v[2 * k] != a0[c][2 * k] || v[2 * k + 1] != a0[c][2 * k + 1];
            bits[c] |= (uint32_t)ne_k << k;
          }
        }
      }
    }
  }
  // chunk q holds entries q W .. q W + W - 1: mask word q / LPW, bits W (q % LPW) ..
#pragma unroll
  for (int c = 0; c < CQ; ++c) {
    const int q = c * kWave + lane;
    uint32_t x = bits[c] << (W * (q % LPW));
#pragma unroll
    for (int sh = 1; sh < LPW; sh <<= 1) x |= (uint32_t)__shfl_xor((int)x, sh);
    if (q % LPW == 0 && q / LPW < 8 && x) atomicOr(&acc[q / LPW], x);  // LDS
  }
  __syncthreads();
  if (threadIdx.x < 8) part[blockIdx.x * 8 + threadIdx.x] = acc[threadIdx.x];
}

// The OR of the nparts partial masks into the mask words (one workgroup).
__global__ __launch_bounds__(256) void ainv_reduce_kernel(const uint32_t* __restrict__ part, int nparts,
                                                          uint32_t* __restrict__ mask) {
  __shared__ uint32_t acc[8];
  if (threadIdx.x < 8) acc[threadIdx.x] = 0;
  __syncthreads();
  const int w = threadIdx.x & 7;
  uint32_t x = 0;
  for (int p = threadIdx.x >> 3; p < nparts; p += 32) x |= part[p * 8 + w];
  if (x) atomicOr(&acc[w], x);  // LDS
  __syncthreads();
  if (threadIdx.x < kAinvWords) mask[threadIdx.x] = acc[threadIdx.x];
}

// Position of the k-th set bit of x (k < popcount(x)).
__device__ __forceinline__ int kth_set_bit(uint32_t x, int k) {
  for (int j = 0; j < k; ++j) x &= x - 1;
  return __builtin_ctz(x);
}

// ---- pack / unpack -----------------------------------------------------------

// One wavefront per (problem, stage), kPackWaves problems of a stage per
// workgroup (adjacent records; one-wavefront workgroups: 215 against 192 us
// at config 3).  Gathering all of a lane's values before its stores, over one
// index space for the three records, was slower (319 us): every unrolled
// value then runs the code of all three records.  The QP and state arrays
// have rows of d.nq entries, the records d.n >= d.nq: variables nq..n-1 are
// dummies with D = 1 on their diagonal and zero everywhere else (x, q, and
// their columns of A_minus, G and A0), so theta keeps them decoupled at
// 1 + sigma and the iteration keeps them at zero without touching any other
// value.  With A0p, the wavefront of (b, 0) also writes the problem's A0 with
// rows of n entries.
constexpr int kPackWaves = 4;

template <typename R>
__global__ __launch_bounds__(kWave * kPackWaves) void stage_pack_kernel(Dims d, QPDev<R> qp, StateDev<R> st,
                                                                        R* __restrict__ am, R* __restrict__ rv,
                                                                        R* __restrict__ dm, int diag,
                                                                        R* __restrict__ A0p) {
  const int b = blockIdx.x * kPackWaves + (int)(threadIdx.x / kWave), t = blockIdx.y;
  const int tid = (int)(threadIdx.x % kWave);
  const int B = d.B, T = d.T, N = d.N, n = d.n, nx = d.nx, m = d.m, nq = d.nq;
  if (b >= B) return;  // the last workgroup's spare wavefronts (no barrier follows)
  const RecGeom g = rec_geom(d, diag != 0);
  const size_t bt = (size_t)b * T + t;
  {
    R* o = am + ((size_t)t * B + b) * g.amp;
    const R* sa = qp.Am + ((size_t)b * N + t) * nx * nq;
    const R* sg = qp.G + bt * m * nq;
    for (int e = tid; e < g.amp; e += kWave) {
      const int r = e / n, k = e - r * n;
      R v = R(0);
      if (k < nq) {
        if (r < nx) {
          if (t < N) v = sa[r * nq + k];
        } else if (r < nx + m) {
          v = sg[(r - nx) * nq + k];
        }
      }
      o[e] = v;
    }
  }
  if (A0p != nullptr && t == 0) {
    const R* sa0 = qp.A0 + (size_t)b * d.n0 * nq;
    for (int e = tid; e < d.n0 * n; e += kWave) {
      const int r = e / n, k = e - r * n;
      A0p[(size_t)b * d.n0 * n + e] = k < nq ? sa0[r * nq + k] : R(0);
    }
  }
  R* o = rv + ((size_t)t * B + b) * g.rvp;
  for (int e = tid; e < g.rvp; e += kWave) {
    R v = R(0);
    if (e >= g.x && e < g.x + n) {
      if (e - g.x < nq) v = st.x[bt * nq + e - g.x];
    } else if (e >= g.q && e < g.q + n) {
      if (e - g.q < nq) v = qp.q[bt * nq + e - g.q];
    } else if (m > 0 && e >= g.z && e < g.z + m) {
      v = st.z[bt * m + e - g.z];
    } else if (m > 0 && e >= g.yg && e < g.yg + m) {
      v = st.y_g[bt * m + e - g.yg];
    } else if (m > 0 && e >= g.xi && e < g.xi + m) {
      v = st.xi[bt * m + e - g.xi];
    } else if (m > 0 && e >= g.l && e < g.l + m) {
      v = qp.l[bt * m + e - g.l];
    } else if (m > 0 && e >= g.u && e < g.u + m) {
      v = qp.u[bt * m + e - g.u];
    } else if (t < N && e >= g.yf && e < g.yf + nx) {
      v = st.y_f[((size_t)b * N + t) * nx + e - g.yf];
    } else if (t < N && e >= g.c && e < g.c + nx) {
      v = qp.c[((size_t)b * N + t) * nx + e - g.c];
    }
    o[e] = v;
  }
  // D_t: the diagonal, or packed lower (D is symmetric); 1 on a dummy's diagonal
  R* od = dm + ((size_t)t * B + b) * g.dmp;
  const R* Dt = qp.D + bt * nq * nq;
  for (int e = tid; e < g.dmp; e += kWave) {
    R v = R(0);
    if (diag) {
      if (e < nq)
        v = Dt[e * nq + e];
      else if (e < n)
        v = R(1);
    } else if (e < packed_size(n)) {
      int i = (int)((sqrtf(8.0f * e + 1.0f) - 1.0f) * 0.5f);
      while ((i + 1) * (i + 2) / 2 <= e) ++i;
      while (i * (i + 1) / 2 > e) --i;
      const int k = e - i * (i + 1) / 2;
      if (i < nq)
        v = Dt[i * nq + k];
      else if (k == i)
        v = R(1);
    }
    od[e] = v;
  }
}

// Warm records: the stage records already hold the previous solve's output
// state and this QP's blocks that do not change between SQP iterations (D, q,
// G, l, u); only the relinearized dynamics rows (A_minus_t into M_t, c_t into
// cz) are written.  A block handles stage t of kRepackProblems consecutive
// problems (adjacent records), one thread per value and problem, so that each
// thread keeps several independent copies in flight.
constexpr int kRepackProblems = 8;

//
// With INEQ the G rows of the M records and the l, u entries of the rv
// records are rewritten as well, at every stage t < T (the grid's y extent;
// N without INEQ).
template <typename R, bool INEQ>
__global__ __launch_bounds__(256) void stage_repack_dynamics_kernel(Dims d, const R* __restrict__ Am,
                                                                    const R* __restrict__ c,
                                                                    const R* __restrict__ G,
                                                                    const R* __restrict__ l,
                                                                    const R* __restrict__ u, R* __restrict__ am,
                                                                    R* __restrict__ rv, int diag, int dyn_rows) {
  const int t = blockIdx.y, b0 = blockIdx.x * kRepackProblems;
  const RecGeom g = rec_geom(d, diag != 0);
  const int n = d.n, nx = d.nx, m = d.m, nq = d.nq;
  // per stage: [A_minus (nx nq) | c (nx)] for t < N (dyn_rows: they changed),
  // then [G (m nq) | l (m) | u (m)]; a record row has n >= nq entries (the
  // dummies' columns stay zero)
  const bool dyn = dyn_rows != 0 && (!INEQ || t < d.N);
  const int na = dyn ? nx * nq : 0, nd = dyn ? na + nx : 0;
  const int ng = INEQ ? m * nq : 0, per = nd + (INEQ ? ng + 2 * m : 0);
  auto rec_col = [&](int e) { return (e / nq) * n + e % nq; };  // row-major nq -> n
  for (int k = threadIdx.x; k < per; k += blockDim.x) {
    R v[kRepackProblems];
#pragma unroll
    for (int j = 0; j < kRepackProblems; ++j) {
      const int b = min(b0 + j, d.B - 1);
      const size_t bn = (size_t)b * d.N + t, bt = (size_t)b * d.T + t;
      if (k < na)
        v[j] = Am[bn * na + k];
      else if (k < nd)
        v[j] = c[bn * nx + (k - na)];
      else if (k < nd + ng)
        v[j] = G[bt * ng + (k - nd)];
      else if (k < nd + ng + m)
        v[j] = l[bt * m + (k - nd - ng)];
      else
        v[j] = u[bt * m + (k - nd - ng - m)];
    }
#pragma unroll
    for (int j = 0; j < kRepackProblems; ++j) {
      if (b0 + j >= d.B) break;
      const size_t rec = (size_t)t * d.B + b0 + j;
      if (k < na)
        am[rec * g.amp + rec_col(k)] = v[j];
      else if (k < nd)
        rv[rec * g.rvp + g.c + (k - na)] = v[j];
      else if (k < nd + ng)
        am[rec * g.amp + nx * n + rec_col(k - nd)] = v[j];  // G rows follow the A_minus rows
      else if (k < nd + ng + m)
        rv[rec * g.rvp + g.l + (k - nd - ng)] = v[j];
      else
        rv[rec * g.rvp + g.u + (k - nd - ng - m)] = v[j];
    }
  }
}

// The state back from the rv records, and each problem's non-finite flag
// (bit 31 of iters[b], TMPC_ITERS_NONFINITE; on this path in place of
// nonfinite_flag_kernel).  A block handles stage t of kUnpackProblems
// consecutive problems; work item (j, k) is state value k (x, z, y_g, xi, then
// y_f for t < N) of problem b0 + j, k fastest, so that the reads of one record
// and the writes of one row are contiguous runs.  Blocks of stage 0 also scan
// y_f0 and rho, which the iteration kernel writes directly.  A problem's flag
// is set by atomicOr from each block that meets one of its non-finite values
// (the result does not depend on their order).
constexpr int kUnpackProblems = 32;

template <typename R>
__global__ __launch_bounds__(256) void stage_unpack_kernel(Dims d, const R* __restrict__ rv, StateDev<R> st,
                                                           uint32_t* __restrict__ iters) {
  __shared__ uint32_t bad[kUnpackProblems];
  const int t = blockIdx.y, b0 = blockIdx.x * kUnpackProblems;
  const int B = d.B, T = d.T, N = d.N, n = d.nq, nx = d.nx, m = d.m;  // n: the state's row length
  const RecGeom g = rec_geom(d);
  const int per = n + 3 * m + (t < N ? nx : 0);
  const int nb = min(kUnpackProblems, B - b0);
  if (threadIdx.x < kUnpackProblems) bad[threadIdx.x] = 0u;
  __syncthreads();
  const unsigned total = (unsigned)(nb * per);
  for (unsigned idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int j = (int)(idx / (unsigned)per), k = (int)idx - j * per;
    // source offset in the record, destination array and its per-problem pitch
    int src, e, pitch;
    R* dst;
    if (k < n) {
      src = g.x + k; dst = st.x; e = k; pitch = n;
    } else if (k < n + m) {
      src = g.z + (k - n); dst = st.z; e = k - n; pitch = m;
    } else if (k < n + 2 * m) {
      src = g.yg + (k - n - m); dst = st.y_g; e = k - n - m; pitch = m;
    } else if (k < n + 3 * m) {
      src = g.xi + (k - n - 2 * m); dst = st.xi; e = k - n - 2 * m; pitch = m;
    } else {
      src = g.yf + (k - n - 3 * m); dst = st.y_f; e = k - n - 3 * m; pitch = nx;
    }
    const bool dyn = k >= n + 3 * m;  // y_f: (B, N, nx); the others (B, T, .)
    const int b = b0 + j;
    const R v = rv[((size_t)t * B + b) * g.rvp + src];
    const size_t row = dyn ? (size_t)b * N + t : (size_t)b * T + t;
    dst[row * pitch + e] = v;
    if (!__builtin_isfinite(v)) bad[j] = 1u;
  }
  if (t == 0) {
    const int n0 = d.n0, pe = n0 + 1;
    for (unsigned idx = threadIdx.x; idx < (unsigned)(nb * pe); idx += blockDim.x) {
      const int j = (int)(idx / (unsigned)pe), k = (int)idx - j * pe;
      const int b = b0 + j;
      const R* p = k < n0 ? (st.y_f0 ? st.y_f0 + (size_t)b * n0 + k : nullptr) : (st.rho ? st.rho + b : nullptr);
      if (p && !__builtin_isfinite(*p)) bad[j] = 1u;
    }
  }
  __syncthreads();
  if (iters && threadIdx.x < nb && bad[threadIdx.x]) atomicOr(iters + b0 + threadIdx.x, 0x80000000u);
}

// ---- wavefront helpers ---------------------------------------------------------

// A run of nch 16-byte chunks, chunk c * 64 + lane in register r[c].  No
// branches: the loads go through a buffer resource whose range is the run
// (lanes past it read zeros), and lanes past the run store to `spill`, a
// 16-byte LDS dump, so every chunk costs the same instructions in every lane
// instead of an exec-mask branch.  `src` is wavefront-uniform.
constexpr int kBufferFlags = 0x00020000;  // dword 3 of a raw buffer resource (gfx9 family)

template <typename V, int CH>
__device__ __forceinline__ void load_run(V (&r)[CH], const V* __restrict__ src, int nch) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<V*>(src), (short)0, nch * 16, kBufferFlags);
  const unsigned tid = threadIdx.x;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int off = (int)((c * kWave + tid) * 16u);
    r[c] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
  }
}

// Stores element `elem` of a buffer when `on`; otherwise the offset lies past
// any range and the hardware drops the store (no exec-mask branch).
__device__ __forceinline__ void buf_store(float v, __amdgpu_buffer_rsrc_t rs, bool on, unsigned elem) {
  const int off = on ? (int)(elem * 4u) : (int)0x80000000u;
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), rs, off, 0, 0);
}
__device__ __forceinline__ void buf_store(double v, __amdgpu_buffer_rsrc_t rs, bool on, unsigned elem) {
  typedef int i32x2 __attribute__((ext_vector_type(2)));
  const int off = on ? (int)(elem * 8u) : (int)0x80000000u;
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, v), rs, off, 0, 0);
}

template <typename V, int CH>
__device__ __forceinline__ void store_run(const V (&r)[CH], V* dst, int nch, V* spill) {
  const unsigned tid = threadIdx.x;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const unsigned e = c * kWave + tid;
    *(e < (unsigned)nch ? dst + e : spill) = r[c];
  }
}

template <typename V, int CH>
__device__ __forceinline__ void store_run(const V (&r)[CH], V* dst, int nch) {
  const unsigned tid = threadIdx.x;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const unsigned e = c * kWave + tid;
    if (e < (unsigned)nch) dst[e] = r[c];
  }
}

// Row i of a (rows x NC) row-major block times v; column i times v (rows entries).
// The dot products first issue all their LDS reads, then (after a scheduling
// barrier) the FMAs: left alone, the compiler interleaves one read pair with
// one FMA pair and waits for every pair.
// The vector operand of the dot products is the same for all lanes of a
// group; it is read with 16-byte loads (4 floats or 2 doubles per LDS
// instruction) when it is 16-byte aligned (VA).
template <typename R, int N, bool VA>
__device__ __forceinline__ void lds_vec(const R* v, R (&out)[N]) {
  if constexpr (VA) {
    using V = typename Vec16<R>::T;
    constexpr int W = Vec16<R>::W;
    const V* v4 = reinterpret_cast<const V*>(v);
#pragma unroll
    for (int q = 0; q < N / W; ++q) {
      const V c = v4[q];
#pragma unroll
      for (int w = 0; w < W; ++w) out[q * W + w] = c[w];
    }
#pragma unroll
    for (int k = (N / W) * W; k < N; ++k) out[k] = v[k];
  } else {
#pragma unroll
    for (int k = 0; k < N; ++k) out[k] = v[k];
  }
}

template <typename R, int NC, bool VA = true>
__device__ __forceinline__ R lrow(const R* A, int i, const R* v) {
  R ak[NC], vk[NC];
  const R* a = A + i * NC;
#pragma unroll
  for (int k = 0; k < NC; ++k) ak[k] = a[k];
  lds_vec<R, NC, VA>(v, vk);
  __builtin_amdgcn_sched_barrier(0);
  R acc = R(0);
#pragma unroll
  for (int k = 0; k < NC; ++k) acc += ak[k] * vk[k];
  return acc;
}
// All NR rows are read: the caller keeps v[r] = 0 for r >= rows and every
// row read finite (LDS is zeroed at kernel start; rows past a block land on
// finite data), so the rows past `rows` add exact zeros.
template <typename R, int NC, int NR = NC>
__device__ __forceinline__ R lcol(const R* A, int rows, int i, const R* v) {
  (void)rows;
  R ak[NR], vk[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) ak[r] = A[r * NC + i];
  lds_vec<R, NR, true>(v, vk);
  __builtin_amdgcn_sched_barrier(0);
  R acc = R(0);
#pragma unroll
  for (int r = 0; r < NR; ++r) acc += ak[r] * vk[r];
  return acc;
}
// Row i of a packed symmetric (lower) block times v.
template <typename R, int NC>
__device__ __forceinline__ R lsym(const R* Th, int i, const R* v) {
  R ak[NC], vk[NC];
  const int ri = (i * (i + 1)) >> 1;
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int idx = k <= i ? ri + k : ((k * (k + 1)) >> 1) + i;
    ak[k] = Th[idx];
  }
  lds_vec<R, NC, true>(v, vk);
  __builtin_amdgcn_sched_barrier(0);
  R acc = R(0);
#pragma unroll
  for (int k = 0; k < NC; ++k) acc += ak[k] * vk[k];
  return acc;
}

// A group vector operand of the products below: with D (one or two problems
// per wavefront, groups on 16-lane row boundaries) the lanes' values seen
// through DPP row broadcasts (stream_dpp.hpp), otherwise the LDS slot the
// lanes wrote it to (read after the next LDS ordering point).
template <typename R, bool D>
struct GVec;
template <typename R>
struct GVec<R, true> {
  RowPair<R> v;
};
template <typename R>
struct GVec<R, false> {
  const R* s;
};

// Lane i's element v of a vector of at most NL elements.  D: all lanes of
// the wavefront must be active (a 17-lane group's element 16 crosses rows).
template <bool D, int NL, typename R>
__device__ __forceinline__ GVec<R, D> gvec(R v, R* slot, int i) {
  if constexpr (D) {
    if constexpr (NL > 16)
      return {row_pair(v)};
    else
      return {RowPair<R>{v, v}};
  } else {
    slot[i] = v;
    return {slot};
  }
}

// lrow / lcol / lsym with a group vector operand.  D: the block entries are
// read from LDS as before, the vector comes by DPP, and every lane of the
// wavefront must be active.
template <typename R, int NC, bool D>
__device__ __forceinline__ R mrow(const R* A, int i, const GVec<R, D>& v) {
  if constexpr (D) {
    R ak[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) ak[k] = A[i * NC + k];
    return dot_pair(ak, v.v);
  } else {
    return lrow<R, NC>(A, i, v.s);
  }
}
template <typename R, int NC, int NR, bool D>
__device__ __forceinline__ R mcol(const R* A, int i, const GVec<R, D>& v) {
  if constexpr (D) {
    R ak[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) ak[r] = A[r * NC + i];
    return dot_pair(ak, v.v);
  } else {
    return lcol<R, NC, NR>(A, 0, i, v.s);
  }
}
template <typename R, int NC, bool D>
__device__ __forceinline__ R msym(const R* Th, int i, const GVec<R, D>& v) {
  if constexpr (D) {
    R ak[NC];
    const int ri = (i * (i + 1)) >> 1;
#pragma unroll
    for (int k = 0; k < NC; ++k) ak[k] = Th[k <= i ? ri + k : ((k * (k + 1)) >> 1) + i];
    return dot_pair(ak, v.v);
  } else {
    return lsym<R, NC>(Th, i, v.s);
  }
}

// Visits t = 0..T-1 (fwd) or T-1..0 in batches of D: stage batch k from
// registers into LDS slots, issue the loads of batch k+1, compute batch k.
template <int D, typename Regs, typename Ld, typename St, typename Cp>
__device__ __forceinline__ void run_sweep(int T, bool fwd, Ld&& load, St&& stage, Cp&& compute) {
  Regs nxt[D];
#pragma unroll
  for (int j = 0; j < D; ++j)
    if (j < T) load(nxt[j], fwd ? j : T - 1 - j);
  for (int k0 = 0; k0 < T; k0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j)
      if (k0 + j < T) stage(nxt[j], j);
    lds_order();
#pragma unroll
    for (int j = 0; j < D; ++j)
      if (k0 + D + j < T) load(nxt[j], fwd ? k0 + D + j : T - 1 - (k0 + D + j));
#pragma unroll
    for (int j = 0; j < D; ++j)
      if (k0 + j < T) compute(j, fwd ? k0 + j : T - 1 - (k0 + j));
  }
}

// Two wavefronts per SIMD (at most 256 VGPRs) for fp32, so that B = 4096 at
// P = 2 is resident in one pass over 1024 SIMDs; one for fp64.
template <typename R>
struct StreamOcc {
  static constexpr int waves = sizeof(R) == 4 ? 2 : 1;
};

// GRES: G_t is the same for every stage and problem (box rows; vouched for by
// the caller, TMPC_FLAG_CONST_G).  The G rows of every M slot are written into
// LDS once, from the wavefront's first record, and the backward sweep streams
// only the A_minus rows of each stage record, as the forward sweep does.
//
// AINV (with GRES): the stage-invariant entries of A_minus (a.amask) are
// written into every M slot from each problem's stage-0 record, and both
// sweeps stream only the varying entries (a.ac), element by element: the
// first chunk's gamma sweep, which stages the whole records anyway, writes
// a.ac.  Outside those fills only varying positions of the slots' A_minus
// rows are written, so the products read the same values as with whole
// records; at stage N (A_minus_N = 0) the slots hold another stage's finite
// entries, which meet zero vector entries only.
template <typename R, int NC, int P, int DPF, int NL = NC, int MM = kMaxStreamM, bool GRES = false,
          bool AINV = false>
__global__ __launch_bounds__(kWave, StreamOcc<R>::waves) void admm_stream_kernel(StreamArgs<R> a) {
  static_assert(NL >= NC && NL <= kWave / P, "row lanes must fit a problem's group");
  static_assert(!AINV || GRES, "the AINV form streams A_minus rows only (G rows resident)");
  using V = typename Vec16<R>::T;
  using K = StreamShape<R, NC, P, NL, MM>;
  constexpr int n = NC, PITCH = K::PITCH, W = K::W;
  constexpr int CH_TH = K::CH_TH, CH_AM = K::CH_AM, CH_RV = K::CH_RV;
  // AINV: rows of 64 16-byte chunks of a wavefront's compressed run
  // (P nx n entries, nx <= n - 1, nx n <= kAinvMaxEntries)
  constexpr int AINV_MAX = (NC - 1) * NC < kAinvMaxEntries ? (NC - 1) * NC : kAinvMaxEntries;
  constexpr int CHD = (P * AINV_MAX / W + kWave - 1) / kWave;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  R* lds = reinterpret_cast<R*>(smem_raw);
  const Dims d = a.d;
  const int T = d.T, N = d.N, nx = d.nx, n0 = d.n0, m = d.m, B = d.B;
  const bool diagD = a.diag != 0;
  const RecGeom rg = rec_geom(d, diagD);
  const int amp = rg.amp, rvp = rg.rvp, dmp = rg.dmp;
  const StreamLayout L = stream_layout(d, P, DPF, diagD);
  // lanes 0..NL-1 of a group are live: the first n hold the n-vectors, the
  // first nx + m the stacked constraint rows
  const Group G = make_group_strided(NL, P, B);
  const int b = G.prob, i = G.lane, p = G.gid, base = p * (kWave / P), tid = threadIdx.x;
  // group vectors by DPP row broadcasts (groups at lane offsets 0 and 32)
  // or through LDS slots (three groups at offsets 0, 21, 42)
  constexpr bool DV = P <= 2;
  const int b0 = blockIdx.x * P;
  const int nprob = min(P, B - b0);
  const int nch_th = nprob * PITCH / W, nch_am = nprob * amp / W, nch_rv = nprob * rvp / W;
  const int nch_dm = nprob * dmp / W;
  const unsigned pl = (unsigned)min(p, nprob - 1);
  const R alpha = a.alpha, one_m_alpha = R(1) - a.alpha, sigma = a.sigma;

  R* wgp = lds + L.wg + p * T * n;
  V* spl = reinterpret_cast<V*>(lds + L.spill);
  constexpr int VW = vec_stride(P);
  R* vec = lds + L.vec + p * up4(kWave / P);
  R* sr = vec + 0 * VW;
  R* su = vec + 1 * VW;
  R* ss = vec + 2 * VW;
  R* sx = vec + 3 * VW;
  R* sc = vec + 4 * VW;
  R* sc0 = vec + 5 * VW;
  R* sy = vec + 6 * VW;   // new stacked duals [y_f; y_g] (residuals)
  R* sy0 = vec + 7 * VW;  // new y_f0 (residuals)
  R* sxn = sr;  // the relaxed iterate for the residuals (sr is free in the backward sweep)
  const int nr = nx + m;            // stacked constraint rows of a stage
  // lane index clamped into the blocks, for lanes that compute values they
  // discard (so that their LDS reads stay inside the blocks and the pad)
  const int icn = min(i, NC - 1), icr = min(i, NL - 1);
  const bool dyn = i < nx, ineq = i >= nx && i < nr;
  const int ji = ineq ? i - nx : 0;  // inequality index of an inequality row
  const R* a0p = lds + L.a0 + p * n0 * n;
  auto thS = [&](int j) { return lds + L.th + j * (P * PITCH); };
  auto amS = [&](int j) { return lds + L.am + j * (P * amp); };
  auto rvS = [&](int j) { return lds + L.rv + j * (P * rvp); };
  auto dmS = [&](int j) { return lds + L.dm + j * (P * dmp); };
  // stage runs: base of this wavefront's problems plus t times the stage
  // stride, in 32-bit element offsets (the host keeps T B pitch below 2^31)
  const R* th0 = a.th + (size_t)b0 * PITCH;
  const R* dm0 = a.dm + (size_t)b0 * dmp;
  const R* am0 = a.am + (size_t)b0 * amp;
  R* rv0 = a.rv + (size_t)b0 * rvp;
  const unsigned sth = (unsigned)B * PITCH, sdm = (unsigned)B * dmp, sam = (unsigned)B * amp, srv = (unsigned)B * rvp;
  auto th_run = [&](int t) { return reinterpret_cast<const V*>(th0 + (unsigned)t * sth); };
  auto dm_run = [&](int t) { return reinterpret_cast<const V*>(dm0 + (unsigned)t * sdm); };
  auto am_run = [&](int t) { return reinterpret_cast<const V*>(am0 + (unsigned)t * sam); };
  auto rv_run = [&](int t) { return reinterpret_cast<const V*>(rv0 + (unsigned)t * srv); };
  const unsigned rv_lane = pl * rvp;  // this lane's problem inside a stage run
  // byte offsets of this lane's 16-byte chunks of the A_minus rows of the M
  // runs (the forward sweep reads no G rows): chunk e of the wavefront maps to
  // problem e / ca, chunk e % ca of its block; -1 marks lanes past the last
  // chunk (their loads go out of range and read zeros)
  int fa_off[CH_AM];
  {
    const int ca = (nx * n + W - 1) / W;
#pragma unroll
    for (int c = 0; c < CH_AM; ++c) {
      const int e = c * kWave + tid, pe = e / ca;
      fa_off[c] = pe < nprob ? (pe * amp + (e - pe * ca) * W) * (int)sizeof(R) : -1;
    }
  }
  // AINV: the varying entries of a wavefront's problems, problem by problem,
  // each in row-major order (entry k of a problem has the row-major index of
  // the k-th set bit of the mask; with no varying entry, entry 0, which is
  // invariant, so streaming it rewrites the value its slot position already
  // holds): nent = nprob nv entries.  They are stored in rows of 64 16-byte
  // chunks (64 W entries): chunk c * 64 + tid holds entries
  // (c W + k) 64 + tid, k < W, so that the k-th LDS store of a row covers 64
  // consecutive entries (few bank conflicts).  Entries past nent repeat entry
  // nent - 1 (the same value to the same place).  A wavefront's rows of a
  // stage are nrow = ceil(P nv / 64 W) long; rows past them are skipped
  // (wavefront-uniform).  The slot offsets of a lane's W entries per row are
  // packed 16 bits each (< 2 amp < 2^16).
  constexpr int APW = W / 2;  // registers of packed offsets per row
  uint32_t adp[AINV ? CHD * APW : 1] = {};
  int nv = 1;
  if constexpr (AINV) {
    uint32_t mw[kAinvWords];
    int cnt_all = 0;
#pragma unroll
    for (int w = 0; w < kAinvWords; ++w) {
      mw[w] = a.amask[w];
      cnt_all += __popc(mw[w]);
    }
    nv = max(cnt_all, 1);
    const int nent = nprob * nv;
#pragma unroll
    for (int c = 0; c < CHD; ++c)
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const int el = min((c * W + k) * kWave + tid, nent - 1), pe = el / nv;
        int kk = el - pe * nv, pos = 0;
        bool found = false;
#pragma unroll
        for (int w = 0; w < kAinvWords; ++w) {
          const int cnt = __popc(mw[w]);
          if (!found && kk < cnt) {
            pos = 32 * w + kth_set_bit(mw[w], kk);
            found = true;
          }
          if (!found) kk -= cnt;
        }
        adp[c * APW + k / 2] |= (uint32_t)(pe * amp + pos) << (16 * (k & 1));
      }
  }
  auto ad = [&](int c, int k) __attribute__((always_inline)) {
    return (int)((adp[c * APW + k / 2] >> (16 * (k & 1))) & 0xFFFFu);
  };
  const int nrow = (P * nv + kWave * W - 1) / (kWave * W);
  // one resource over the compressed runs [N][grid][nrow][64 chunks]: this
  // wavefront's rows of stage t at byte offset t grid nrow 1024 (the host
  // keeps the array below 2^31 bytes)
  const __amdgpu_buffer_rsrc_t acr = __builtin_amdgcn_make_buffer_rsrc(
      AINV ? const_cast<R*>(a.ac + (size_t)blockIdx.x * nrow * kWave * W) : const_cast<R*>(a.am), (short)0,
      0x7FFFFFFF, kBufferFlags);
  const unsigned sacb = gridDim.x * (unsigned)nrow * kWave * 16u;
  // the varying entries of stage t < N into registers, and from registers
  // into an M slot
  auto ac_load = [&](V (&r)[AINV ? CHD : 1], int t) __attribute__((always_inline)) {
    if constexpr (AINV) {
#pragma unroll
      for (int c = 0; c < CHD; ++c) {
        if (c > 0 && nrow <= c) break;
        r[c] = __builtin_bit_cast(
            V, __builtin_amdgcn_raw_buffer_load_b128(acr, (int)((c * kWave + tid) * 16u), (int)((unsigned)t * sacb), 0));
      }
    }
  };
  auto ac_store = [&](const V (&r)[AINV ? CHD : 1], R* slot) __attribute__((always_inline)) {
    if constexpr (AINV) {
#pragma unroll
      for (int c = 0; c < CHD; ++c) {
        if (c > 0 && nrow <= c) break;
#pragma unroll
        for (int k = 0; k < W; ++k) slot[ad(c, k)] = r[c][k];
      }
    }
  };
  // M runs of the backward sweep: the whole records, or (GRES) their A_minus
  // rows only, through the same chunk map as the forward sweep, or (AINV) the
  // varying entries of A_minus (none at stage N, whose slot keeps what it holds)
  auto load_m = [&](V (&r)[AINV ? 1 : CH_AM], V (&rc)[AINV ? CHD : 1], int t) __attribute__((always_inline)) {
    if constexpr (AINV) {
      if (t < N) ac_load(rc, t);
    } else if constexpr (GRES) {
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<V*>(am_run(t)), (short)0, nch_am * 16, kBufferFlags);
#pragma unroll
      for (int c = 0; c < CH_AM; ++c)
        r[c] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(rs, fa_off[c], 0, 0));
    } else {
      load_run<V, CH_AM>(r, am_run(t), nch_am);
    }
  };
  auto store_m = [&](const V (&r)[AINV ? 1 : CH_AM], const V (&rc)[AINV ? CHD : 1], R* slot, int t)
                     __attribute__((always_inline)) {
    (void)t;
    if constexpr (AINV) {
      if (t < N) ac_store(rc, slot);
    } else if constexpr (GRES) {
      V* dst = reinterpret_cast<V*>(slot);
#pragma unroll
      for (int c = 0; c < CH_AM; ++c) *(fa_off[c] >= 0 ? dst + (fa_off[c] >> 4) : spl) = r[c];
    } else {
      store_run<V, CH_AM>(r, reinterpret_cast<V*>(slot), nch_am, spl);
    }
  };

  // ---- LDS starts zeroed (the column products rely on finite data past the
  // blocks); resident data: A0 in LDS, c0 / y_f0 in registers ---------------
  for (int e = tid; e < L.total / W; e += kWave) reinterpret_cast<V*>(lds)[e] = V{};
  lds_order();
  for (int e = tid; e < nprob * n0 * n; e += kWave) lds[L.a0 + e] = a.A0[(size_t)b0 * n0 * n + e];
  // GRES: the G rows of every M slot (slot s at L.am + s amp), from stage 0
  // of the wavefront's first problem; written again after each residual
  // reduction, whose scratch (from L.th) may reach into the slots
  // AINV: also the A_minus rows of every M slot, from each problem's own
  // stage-0 record (the invariant entries; the varying ones are overwritten
  // before use)
  auto fill_g = [&]() __attribute__((always_inline)) {
    if constexpr (GRES) {
      const R* g0 = a.am + (size_t)b0 * amp + nx * n;
      const int gl = m * n, nslot = (DPF > 2 ? DPF : 2) * P;
      for (int e = tid; e < nslot * gl; e += kWave) {
        const int sl = e / gl, k = e - sl * gl;
        lds[L.am + sl * amp + nx * n + k] = g0[k];
      }
    }
    if constexpr (AINV) {
      const int al = nx * n, nslot = (DPF > 2 ? DPF : 2) * P;
      for (int e = tid; e < nslot * al; e += kWave) {
        const int sl = e / al, k = e - sl * al, pp = sl % P;
        if (pp < nprob) lds[L.am + sl * amp + k] = a.am[(size_t)(b0 + pp) * amp + k];
      }
    }
  };
  fill_g();
  const R c0v = (i < n0) ? a.c0[(size_t)b * n0 + i] : R(0);
  R yf0v = (i < n0) ? a.y_f0[(size_t)b * n0 + i] : R(0);

  // ---- per-problem control state (as admm_chunk_kernel) ---------------------
  int it;
  bool done;
  R res[6];
  if (a.first_chunk) {
    it = 0;
    done = (a.chk_conv == nullptr && a.act_in) ? a.act_in[b] == 0 : false;
    res[0] = res[1] = res[4] = res[5] = rinf<R>();
    res[2] = res[3] = R(1);
    if (G.live && i == 0) a.ctl[b * 4 + 2] = 0;
  } else {
    it = a.ctl[b * 4 + 0];
    done = a.ctl[b * 4 + 1] != 0;
#pragma unroll
    for (int k = 0; k < 6; ++k) res[k] = a.res[b * 8 + k];
  }
  R rho = a.rho[b];
  const bool slack = a.use_slack && m > 0;
  const R gs = (slack && a.slack_w) ? a.slack_w[b] : R(0);
  lds_order();

  // ---- gamma_t for the current state and rho (compute_gamma, admm.py:157-174),
  // and, in the first chunk of an SQP step, the first-order check of the input
  // iterate against this QP (_compute_first_order_convergence_error,
  // turbompc_solver.py:1158-1225) from the same stage records:
  //   stationarity P x + q + C^T y_f + G^T y_g, equality C x - c, inequality
  //   violation of g = G x (+ slack), slack stationarity gamma_s xi + y_g.
  const bool fochk = a.first_chunk && a.chk_conv != nullptr;
  {
    struct GRegs {
      V am[CH_AM], rv[CH_RV], dm[CH_TH];
    };
    const R rho_f = rho * a.rho_f_factor;
    R scp = R(0);
    R c_st = R(0), c_eq = R(0), c_iq = R(0), c_sl = R(0);  // this lane's maxima
    R pend = R(0);  // (A_minus_{t-1} x_{t-1} - c_{t-1})[i], awaiting -x_t
    R yfp = R(0);   // y_f_{t-1}[i]
    const GVec<R, DV> vc0 = gvec<DV, NL>(rho_f * c0v - yf0v, sc0, i);  // 0 past n0
    GVec<R, DV> vy0{};
    if (fochk) vy0 = gvec<DV, NL>(yf0v, sy0, i);  // 0 past n0
    run_sweep<1, GRegs>(
        T, true,
        [&](GRegs& r, int t) {
          load_run<V, CH_AM>(r.am, am_run(t), nch_am);
          load_run<V, CH_RV>(r.rv, rv_run(t), nch_rv);
          if (fochk) load_run<V, CH_TH>(r.dm, dm_run(t), nch_dm);
        },
        [&](GRegs& r, int j) {
          store_run<V, CH_AM>(r.am, reinterpret_cast<V*>(amS(j)), nch_am, spl);
          store_run<V, CH_RV>(r.rv, reinterpret_cast<V*>(rvS(j)), nch_rv, spl);
          if (fochk) store_run<V, CH_TH>(r.dm, reinterpret_cast<V*>(dmS(j)), nch_dm, spl);
        },
        [&](int j, int t) {
          if constexpr (AINV) {
            // the first chunk writes the compressed runs from the staged records
            if (a.first_chunk && t < N) {
              const R* sl = amS(j);
#pragma unroll
              for (int c = 0; c < CHD; ++c) {
                if (c > 0 && nrow <= c) break;
                V v;
#pragma unroll
                for (int k = 0; k < W; ++k) v[k] = sl[ad(c, k)];
                typedef int i32x4 __attribute__((ext_vector_type(4)));
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), acr, (int)((c * kWave + tid) * 16u),
                                                       (int)((unsigned)t * sacb), 0);
              }
            }
          }
          const R* mt = amS(j) + p * amp;
          const R* rv = rvS(j) + p * rvp;
          const bool crow = (dyn && t < N) || ineq;  // a live stacked constraint row
          // stacked [rho_f c - y_f; rho z - y_g] (dynamics rows vanish at t = N)
          const R czv = rv[rg.cz + icr], yv = crow ? rv[rg.y + icr] : R(0);
          const R sct = crow ? (dyn ? rho_f : rho) * czv - yv : R(0);
          const R xv = rv[rg.x + icn];
          const auto vc = gvec<DV, NL>(sct, sc, i);  // 0 past nr
          GVec<R, DV> vx{}, vy{};
          if (fochk) {
            vx = gvec<DV, NL>(xv, sx, i);
            vy = gvec<DV, NL>(yv, sy, i);  // [y_f_t; y_g], 0 past nr
          }
          lds_order();
          {
            R gv = sigma * xv - rv[rg.q + icn];
            gv += mcol<R, NC, NL, DV>(mt, icn, vc);
            if (t > 0) gv -= (i < nx) ? scp : R(0);  // A_plus_{t-1}^T = [-I; 0]
            if (t == 0) gv += mcol<R, NC, NC, DV>(a0p, icn, vc0);
            if (i < n) wgp[t * n + i] = gv;
          }
          if (fochk) {
            const R* dmt = dmS(j) + p * dmp;
            R px;
            if (diagD)
              px = dmt[icn] * xv;
            else
              px = msym<R, NC, DV>(dmt, icn, vx);
            R aty = mcol<R, NC, NL, DV>(mt, icn, vy);  // A_minus_t^T y_f_t + G_t^T y_g
            if (t == 0) aty += mcol<R, NC, NC, DV>(a0p, icn, vy0);
            if (t > 0) aty -= dyn ? yfp : R(0);  // A_plus_{t-1}^T y_f_{t-1}
            c_st = rmax(c_st, i < n ? rabs(px + rv[rg.q + icn] + aty) : R(0));
            const R mxv = mrow<R, NC, DV>(mt, icr, vx);
            // dynamics row t-1 is complete with -x_t
            if (t > 0) c_eq = rmax(c_eq, dyn ? rabs(pend - xv) : R(0));
            pend = (dyn && t < N) ? mxv - czv : R(0);
            if (t == 0) {  // every lane computes (DPP); rows past n0 are discarded
              const R a0x = mrow<R, NC, DV>(a0p, min(i, n0 - 1), vx);
              if (i < n0) c_eq = rmax(c_eq, rabs(a0x - c0v));
            }
            const R xiv = rv[rg.xi + ji];
            const R g = mxv + (slack ? xiv : R(0));
            const R viol = rmax(rmax(rv[rg.l + ji] - g, g - rv[rg.u + ji]), R(0));
            c_iq = rmax(c_iq, ineq ? viol : R(0));
            if (slack) c_sl = rmax(c_sl, ineq ? rabs(gs * xiv + yv) : R(0));
            if (a.chk_g && ineq && G.live) a.chk_g[((size_t)b * T + t) * m + ji] = g;
            yfp = (dyn && t < N) ? yv : R(0);
          }
          scp = sct;
          lds_order();
        });
    if constexpr (AINV) {  // the sweep staged whole records (stage N's A_minus rows are zero)
      fill_g();
      lds_order();
    }
    if (fochk) {
      // group maxima (every lane of a group reduces its group: the result
      // decides whether the problem iterates), then the activity of the step
      R* red = lds + L.th;
      red[0 * kWave + tid] = c_st;
      red[1 * kWave + tid] = c_eq;
      red[2 * kWave + tid] = c_iq;
      red[3 * kWave + tid] = c_sl;
      lds_order();
      R mxs[4] = {R(0), R(0), R(0), R(0)};
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int l = 0; l < NL; ++l) mxs[k] = rmax(mxs[k], red[k * kWave + base + l]);
      lds_order();
      fill_g();  // the reduction's scratch may have reached the M slots
      const R conv = rmax(rmax(mxs[0], mxs[1]), rmax(mxs[2], mxs[3]));
      const bool act = (a.act_in ? a.act_in[b] != 0 : true) && conv > a.chk_tol;
      if (G.live && i == 0) {
        a.chk_conv[b] = conv;
        if (a.chk_eq) a.chk_eq[b] = mxs[1];
        if (a.chk_iq) a.chk_iq[b] = mxs[2];
        if (a.act_out) a.act_out[b] = act ? 1 : 0;
      }
      done = !act;  // a stopped problem keeps its input iterate (zero iterations)
    }
  }

  for (int iter = a.it_lo; iter < a.it_hi; ++iter) {
    // cond_fun (admm.py:843-851)
    bool active = false;
    if (!done) {
      const bool sc_ = mod_zero(iter, a.check_every);
      const bool tl = (res[0] > a.eps_abs + a.eps_rel * res[2]) || (res[1] > a.eps_abs + a.eps_rel * res[3]);
      active = (iter < a.max_iter) && (!sc_ || tl);
      active = active || iter < 1;
      if (!active) done = true;
    }
    const bool commit = active && G.live;
    if (__ballot(active && G.real) == 0) break;
    const R rho_f = rho * a.rho_f_factor;

    // ---- forward sweep: w_t = Theta_t^{-1} (gamma_t + rho_f [A_minus_{t-1} w_{t-1}; 0])
    {
      struct FRegs {
        V th[CH_TH], am[AINV ? 1 : CH_AM], ac[AINV ? CHD : 1];
      };
      R v = R(0);  // (A_minus_{t-1} w_{t-1})[i], i < nx
      run_sweep<DPF, FRegs>(
          T, true,
          [&](FRegs& r, int t) {
            load_run<V, CH_TH>(r.th, th_run(t), nch_th);
            if constexpr (AINV) {
              if (t < N) ac_load(r.ac, t);
            } else if (t < N) {  // the A_minus rows of M_t only
              const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                  const_cast<V*>(am_run(t)), (short)0, nch_am * 16, kBufferFlags);
#pragma unroll
              for (int c = 0; c < CH_AM; ++c)
                r.am[c] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(rs, fa_off[c], 0, 0));
            }
          },
          [&](FRegs& r, int j) {
            store_run<V, CH_TH>(r.th, reinterpret_cast<V*>(thS(j)), nch_th, spl);
            if constexpr (AINV) {
              ac_store(r.ac, amS(j));  // at stage N: stage N-1's entries, unused
            } else {
              V* dst = reinterpret_cast<V*>(amS(j));
#pragma unroll
              for (int c = 0; c < CH_AM; ++c)
                *(fa_off[c] >= 0 ? dst + (fa_off[c] >> 4) : spl) = r.am[c];
            }
          },
          [&](int j, int t) {
            // lanes past n compute throwaway values in their own vector slots
            R rr = i < n ? wgp[t * n + i] : R(0);
            if (t > 0) rr += (i < nx) ? rho_f * v : R(0);
            const auto vr = gvec<DV, NL>(rr, sr, i);
            lds_order();
            const R wv = msym<R, NC, DV>(thS(j) + p * PITCH, icn, vr);
            if (i < n) wgp[t * n + i] = wv;
            const auto vw = gvec<DV, NL>(wv, sx, i);
            lds_order();
            if (t < N) v = mrow<R, NC, DV>(amS(j) + p * amp, icr, vw);
          });
    }

    // ---- backward sweep fused with the ADMM updates, the next gamma and (on
    // checking iterations) the residuals of the new iterate (admm.py:392-556).
    //
    // Software-pipelined over two stages: step t runs the recursion part of
    // stage t-1 (A: xt_{t-1} = w_{t-1} - Theta_{t-1}^{-1} rho_f A_minus_{t-1}^T
    // (-xt_t), the only dependence between stages) together with the rest of
    // stage t (B: constraint products, relaxation, projection, duals, the next
    // gamma_t, residual terms), which needs xt_t only.  A and B share each of
    // the three regions of a step (separated by LDS ordering points), so
    // their LDS round trips overlap.  LDS slots: Theta^{-1} of stage t-1; M of
    // stages t and t-1 (by stage parity); rv and D of stage t.  Registers
    // prefetch the runs of step t - PFD (Theta^{-1}, M of t-PFD-1; rv, D of
    // t-PFD) while step t computes.
    const bool chk = mod_zero(iter, a.check_every);
    R rp = 0, nCx = 0, nc = 0, nGx = 0, nz = 0, rd = 0, nPx = 0, nAty = 0, nq = 0, nxi = 0, nyg = 0;
    // per-iteration constants of the projection: y / rho as y * (1 / rho)
    const R inv_rho = R(1) / rho;
    const R frac = slack ? gs / (gs + rho) : R(0), xi_f = slack ? rho / (gs + rho) : R(0);
    {
      // PFD register sets, used by turns: the runs of step t - PFD are loaded
      // while step t computes (two sets where the registers allow)
      constexpr int PFD = P <= 2 ? 2 : 1;
      struct BRegs {
        V th[CH_TH], am[AINV ? 1 : CH_AM], rv[CH_RV], dm[CH_TH], ac[AINV ? CHD : 1];
      };
      BRegs ra, rb;
      auto amP = [&](int t) { return lds + L.am + (t & 1) * (P * amp); };
      R* th_slot = thS(0);
      R* rv_slot = rvS(0);
      R* dm_slot = dmS(0);
      // prologue: M_{T-1} into its slot; ra <- Theta^{-1}, M of T-2 and rv, D
      // of T-1 (step T-1); with two sets rb <- those of T-3 and T-2 (step T-2)
      load_m(ra.am, ra.ac, T - 1);
      store_m(ra.am, ra.ac, amP(T - 1), T - 1);
      if (T >= 2) {
        load_run<V, CH_TH>(ra.th, th_run(T - 2), nch_th);
        load_m(ra.am, ra.ac, T - 2);
      }
      load_run<V, CH_RV>(ra.rv, rv_run(T - 1), nch_rv);
      if (chk) load_run<V, CH_TH>(ra.dm, dm_run(T - 1), nch_dm);
      if constexpr (PFD == 2) {
        if (T >= 2) {
          load_run<V, CH_RV>(rb.rv, rv_run(T - 2), nch_rv);
          if (chk) load_run<V, CH_TH>(rb.dm, dm_run(T - 2), nch_dm);
        }
        if (T >= 3) {
          load_run<V, CH_TH>(rb.th, th_run(T - 3), nch_th);
          load_m(rb.am, rb.ac, T - 3);
        }
      }
      R xa = i < n ? wgp[N * n + i] : R(0);  // xt_t for the coming step (xt_N = w_N)
      R xn = R(0);   // xt_{t+1}[i]
      R xnn = R(0);  // relaxed x_{t+1}[i]
      R gp = R(0);   // gamma_{t+1}[i] awaiting its A_plus_t^T term
      // dual residual row t+1 awaiting its A_plus_t^T y_f_t term (i < nx):
      // P x + q and the rest of C^T y + G^T y_g
      R pq_p = R(0), aty_p = R(0);
      auto step = [&](const int t, BRegs& pr) {
        const bool hasA = t >= 1;  // the recursion part of stage t-1 runs in this step
        // ---- region 1: stage the runs; su for A, sx for B.  Lanes past a
        // vector's length write zeros or throwaway values into their own
        // group's slot (never read as part of the vector).
        if (hasA) {
          store_run<V, CH_TH>(pr.th, reinterpret_cast<V*>(th_slot), nch_th, spl);
          store_m(pr.am, pr.ac, amP(t - 1), t - 1);
        }
        store_run<V, CH_RV>(pr.rv, reinterpret_cast<V*>(rv_slot), nch_rv, spl);
        if (chk) store_run<V, CH_TH>(pr.dm, reinterpret_cast<V*>(dm_slot), nch_dm, spl);
        const auto vu = gvec<DV, NL>(dyn ? -xa : R(0), su, i);  // A_plus_{t-1} xt_t, 0 past nx
        const auto vx = gvec<DV, NL>(xa, sx, i);
        lds_order();
        // this set's next use is step t - PFD
        if (t >= PFD + 1) {
          load_run<V, CH_TH>(pr.th, th_run(t - PFD - 1), nch_th);
          load_m(pr.am, pr.ac, t - PFD - 1);
        }
        if (t >= PFD) {
          load_run<V, CH_RV>(pr.rv, rv_run(t - PFD), nch_rv);
          if (chk) load_run<V, CH_TH>(pr.dm, dm_run(t - PFD), nch_dm);
        }
        // ---- region 2
        const R* mA = amP(t - 1) + p * amp;  // M_{t-1} (A)
        const R* mt = amP(t) + p * amp;      // M_t = [A_minus_t; G_t] (B)
        const R* rv = rv_slot + p * rvp;
        // this wavefront's rv records of stage t in HBM; stores outside the
        // masks go past the range and are dropped
        const __amdgpu_buffer_rsrc_t rsg = __builtin_amdgcn_make_buffer_rsrc(
            rv0 + (unsigned)t * srv, (short)0, (int)(nprob * rvp * sizeof(R)), kBufferFlags);
        GVec<R, DV> vs{};
        if (hasA) vs = gvec<DV, NL>(rho_f * mcol<R, NC, NL, DV>(mA, icn, vu), ss, i);
        const bool drow = dyn && t < N;  // a live dynamics row of stage t
        const R u = drow ? -xn : R(0);   // (A_plus_t xt_{t+1})[i]
        // stacked C and G products of the pre-relaxation iterate
        const R mx = mrow<R, NC, DV>(mt, icr, vx);
        R cx0 = R(0);
        if (t == 0) {  // every lane computes (DPP); rows past n0 are discarded
          const R a0x = mrow<R, NC, DV>(a0p, min(i, n0 - 1), vx);
          cx0 = i < n0 ? a0x : R(0);
        }
        // over-relaxation
        const R xnew = alpha * xa + one_m_alpha * rv[rg.x + icn];
        buf_store(xnew, rsg, commit && i < n, rv_lane + rg.x + i);
        // constraint row i: the dual, the next gamma's entry, and (inequality
        // rows) the box projection / slack
        const R zo = rv[rg.cz + icr], yo = rv[rg.y + icr];
        const R zt = alpha * mx + one_m_alpha * zo + yo * inv_rho;
        const R proj = rmin(rmax(zt, rv[rg.l + ji]), rv[rg.u + ji]);
        R zn = proj, xin = R(0);
        if (slack) {
          zn = (R(1) - frac) * zt + frac * proj;
          xin = xi_f * (proj - zt);
        }
        const R ygn = yo + rho * (alpha * mx + one_m_alpha * zo - zn);
        const R cv = zo;  // c_t[i] on a dynamics row
        const R yf = yo + rho_f * (alpha * (mx + u) + one_m_alpha * cv - cv);
        const R y_r = ineq ? ygn : (drow ? yf : R(0));
        const R tgt = ineq ? rho * zn - ygn : (drow ? rho_f * cv - yf : R(0));
        const R z_r = zn, xi_r = xin;
        buf_store(y_r, rsg, commit && (ineq || drow), rv_lane + rg.y + i);
        buf_store(zn, rsg, commit && ineq, rv_lane + rg.cz + i);
        buf_store(xin, rsg, commit && ineq, rv_lane + rg.xi + ji);
        R ct0 = R(0), yf0_r = R(0);
        if (t == 0 && i < n0) {
          const R yf0 = yf0v + rho_f * (alpha * cx0 + one_m_alpha * c0v - c0v);
          if (commit) {
            a.y_f0[(size_t)b * n0 + i] = yf0;
            yf0v = yf0;
          }
          ct0 = rho_f * c0v - yf0;
          yf0_r = yf0;
        }
        // next iteration's gamma (valid while rho is unchanged)
        const auto vc = gvec<DV, NL>(tgt, sc, i);  // 0 past nr
        GVec<R, DV> vc0{}, vxn{}, vy{}, vy0{};
        if (t == 0) vc0 = gvec<DV, NL>(ct0, sc0, i);  // 0 past n0
        if (chk) {
          vxn = gvec<DV, NL>(xnew, sxn, i);
          vy = gvec<DV, NL>(y_r, sy, i);                  // 0 past nr
          if (t == 0) vy0 = gvec<DV, NL>(yf0_r, sy0, i);  // 0 past n0
        }
        lds_order();
        // ---- region 3
        R xa_next = R(0);
        if (hasA) {
          const R xv = wgp[(t - 1) * n + icn] - msym<R, NC, DV>(th_slot + p * PITCH, icn, vs);
          xa_next = i < n ? xv : R(0);
        }
        if (t < N) {
          gp -= dyn ? tgt : R(0);  // A_plus_t^T = [-I; 0]
          if (i < n) wgp[(t + 1) * n + i] = gp;
        }
        {
          R gv = sigma * xnew - rv[rg.q + icn];
          gv += mcol<R, NC, NL, DV>(mt, icn, vc);
          if (t == 0) gv += mcol<R, NC, NC, DV>(a0p, icn, vc0);
          gp = gv;
        }
        if (chk) {
          const bool cl = i < n;  // a lane of an n-vector
          // dual residual row t+1 is complete with -[y_f_t; 0]
          {
            const R aty = aty_p - y_r;
            rd = rmax(rd, drow ? rabs(pq_p + aty) : R(0));
            nAty = rmax(nAty, drow ? rabs(aty) : R(0));
          }
          // stacked primal rows of the relaxed iterate
          const R m1 = mrow<R, NC, DV>(mt, icr, vxn);
          {
            const R cx1 = m1 - xnn;  // A_minus_t x_t - x_{t+1}, dynamics rows
            rp = rmax(rp, drow ? rabs(cx1 - cv) : (ineq ? rabs(m1 - z_r) : R(0)));
            nCx = rmax(nCx, drow ? rabs(cx1) : R(0));
            nc = rmax(nc, drow ? rabs(cv) : R(0));
            nGx = rmax(nGx, ineq ? rabs(m1) : R(0));
            nz = rmax(nz, ineq ? rabs(z_r) : R(0));
            if (slack) {
              rd = rmax(rd, ineq ? rabs(gs * xi_r + y_r) : R(0));
              nxi = rmax(nxi, ineq ? rabs(xi_r) : R(0));
              nyg = rmax(nyg, ineq ? rabs(y_r) : R(0));
            }
          }
          if (t == 0) {  // every lane computes (DPP); rows past n0 are discarded
            const R cx1 = mrow<R, NC, DV>(a0p, min(i, n0 - 1), vxn);
            if (i < n0) {
              rp = rmax(rp, rabs(cx1 - c0v));
              nCx = rmax(nCx, rabs(cx1));
              nc = rmax(nc, rabs(c0v));
            }
          }
          {
            const R* dmt = dm_slot + p * dmp;
            R px;
            if (diagD)
              px = dmt[icn] * xnew;
            else
              px = msym<R, NC, DV>(dmt, icn, vxn);
            R aty = R(0);
            if (t == 0) aty += mcol<R, NC, NC, DV>(a0p, icn, vy0);
            aty += mcol<R, NC, NL, DV>(mt, icn, vy);  // A_minus_t^T y_f_t + G_t^T y_g_t
            const R qv = rv[rg.q + icn];
            const bool wait = t > 0 && dyn;  // awaits -y_f_{t-1}[i]
            pq_p = px + qv;
            aty_p = aty;
            rd = rmax(rd, (cl && !wait) ? rabs(px + qv + aty) : R(0));
            nAty = rmax(nAty, (cl && !wait) ? rabs(aty) : R(0));
            nPx = rmax(nPx, cl ? rabs(px) : R(0));
            nq = rmax(nq, cl ? rabs(qv) : R(0));
          }
        }
        xn = xa;
        xnn = xnew;
        xa = xa_next;
        lds_order();
      };
      for (int t = T - 1; t >= 0; t -= PFD) {
        step(t, ra);
        if constexpr (PFD == 2)
          if (t >= 1) step(t - 1, rb);
      }
      if (i < n) wgp[i] = gp;
      lds_order();
    }

    // ---- residual reductions and adaptive rho (admm.py:392-556) --------------
    if (chk) {
      // group max-reductions (the slot region is free now)
      R* red = lds + L.th;
      const R vals[11] = {rp, nCx, nc, nGx, nz, rd, nPx, nAty, nq, nxi, nyg};
#pragma unroll
      for (int k = 0; k < 11; ++k) red[k * kWave + tid] = (i < NL) ? vals[k] : R(0);
      lds_order();
      // lane i of each group reduces values k = i, i + NL, ... over the group's
      // NL lanes (lanes past NL that land on k < 11 repeat a value of lane k - NL)
      R mx[(11 + NL - 1) / NL];
#pragma unroll
      for (int q = 0; q < (11 + NL - 1) / NL; ++q) {
        const int k = i + q * NL;
        mx[q] = R(0);
        if (k < 11)
#pragma unroll
          for (int l = 0; l < NL; ++l) mx[q] = rmax(mx[q], red[k * kWave + base + l]);
      }
      lds_order();
#pragma unroll
      for (int q = 0; q < (11 + NL - 1) / NL; ++q)
        if (i + q * NL < 11) red[(i + q * NL) * kWave + base] = mx[q];
      lds_order();
      R r[11];
#pragma unroll
      for (int k = 0; k < 11; ++k) r[k] = red[k * kWave + base];
      lds_order();
      fill_g();  // the reduction's scratch may have reached the M slots
      const R np = rmax(rmax(r[1], r[3]), rmax(r[2], r[4]));
      R nd = rmax(rmax(r[6], r[7]), r[8]);
      if (slack) nd = rmax(nd, rmax(gs * r[9], r[10]));
      const R rv6[6] = {r[0], r[5], np, nd, r[0] / (R(1e-10) + np), r[5] / (R(1e-10) + nd)};
      if (active) {
#pragma unroll
        for (int k = 0; k < 6; ++k) res[k] = rv6[k];
        const R cand = rmin(rmax(rho * r_sqrt(rv6[4] / rv6[5]), a.rho_min), a.rho_max);
        const R ratio = rmax(cand / rho, rho / cand);
        const bool conv = !((rv6[0] > a.eps_abs + a.eps_rel * rv6[2]) || (rv6[1] > a.eps_abs + a.eps_rel * rv6[3]));
        bool keep = iter < 2 || !mod_zero(iter, a.adapt_every);
        keep = keep || conv;
        keep = keep || ratio < a.rho_tol;
        if (!keep) {
          rho = cand;
          if (G.live && i == 0) {
            a.rho[b] = cand;
            a.ctl[b * 4 + 2] = 1;
          }
        }
      }
    }
    if (active) it = iter + 1;
  }
  if (G.live && i == 0) {
    a.ctl[b * 4 + 0] = it;
    a.ctl[b * 4 + 1] = done ? 1 : 0;
#pragma unroll
    for (int k = 0; k < 6; ++k) a.res[b * 8 + k] = res[k];
    a.iters_out[b] = (uint32_t)it;
  }
}

// ---- factorization of S for the explicit-integrator structure ---------------
//
// factor_kernel's recursion (factor.hpp) specialised to A_plus_t = [-I 0],
// E_t = 0, where phi_{t-1} = -rho_f [A_minus_{t-1}; 0]:
//   theta_t = D_t + sigma I + rho G_t^T G_t
//             + rho_f (A_minus_t^T A_minus_t [t < N] + diag(I_nx, 0) [t > 0] + A0^T A0 [t = 0])
//   Theta_t = theta_t - rho_f^2 [A_minus_{t-1} Theta_{t-1}^{-1} A_minus_{t-1}^T, 0; 0, 0]
// so the Schur update touches the leading nx x nx block only.  fp64 throughout.
//
// A wavefront holds P problems; lane i of a group keeps row i of Theta_t in
// registers and the rows it needs from the other lanes come through LDS:
// A_minus blocks (double-buffered across stages), Theta_{t-1}^{-1} (full), the
// Gauss-Jordan pivot row.  Reads the stage records of stage_pack_kernel.

// LDS of factor_std_kernel, in bytes: fp64 work area [P][n n] Theta_{t-1}^{-1}
// and [P][2 n] pivot rows, then the staged stage runs in the storage type R:
// M_t = [A_minus_t; G_t] double-buffered [2][P][amp], D_t [P][pitch],
// A0 [P][n0 n].
struct FactorLayout {
  int th, piv;          // fp64 offsets (elements)
  int am, dm, a0;       // R offsets (elements, from the start of the R region)
  size_t r_base;        // byte offset of the R region
  size_t bytes;
};

template <typename R>
__host__ __device__ inline FactorLayout factor_layout(const Dims& d, int P, bool diag) {
  const RecGeom g = rec_geom(d, diag);
  FactorLayout L;
  const int n = d.n;
  L.th = 0;
  L.piv = P * n * n;
  const int c_elems = L.piv + 2 * P * n;
  L.r_base = ((size_t)c_elems * sizeof(double) + 15) / 16 * 16;
  L.am = 0;
  L.dm = 2 * P * g.amp;
  L.a0 = L.dm + P * g.dmp;
  L.bytes = L.r_base + (size_t)(L.a0 + P * d.n0 * n) * sizeof(R);
  return L;
}

template <typename R, int NC, int P, int NL = NC, int MM = kMaxStreamM>
__global__ __launch_bounds__(kWave, 2) void factor_std_kernel(Dims d, const R* __restrict__ am, const R* __restrict__ dm, const R* __restrict__ A0,
                                                          const R* __restrict__ rho, R sigma, R rho_f_factor,
                                                          int32_t* __restrict__ ctl, R* __restrict__ thinv,
                                                          int diag) {
  using C = double;
  using V = typename Vec16<R>::T;
  using K = StreamShape<R, NC, P, NL, MM>;  // stage-run chunk counts
  constexpr int n = NC, PITCH = K::PITCH, W = K::W;
  constexpr int CH_TH = K::CH_TH, CH_AM = K::CH_AM;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const Dims dd = d;
  const int T = dd.T, N = dd.N, nx = dd.nx, n0 = dd.n0, m = dd.m, B = dd.B;
  const RecGeom rg = rec_geom(dd, diag != 0);
  const FactorLayout FL = factor_layout<R>(dd, P, diag != 0);
  C* lds = reinterpret_cast<C*>(smem_raw);
  R* ldr = reinterpret_cast<R*>(smem_raw + FL.r_base);
  const Group G = make_group_strided(n, P, B);
  const int b = G.prob, i = G.lane, p = G.gid, tid = threadIdx.x;
  const int b0 = blockIdx.x * P, nprob = min(P, B - b0);
  if (ctl != nullptr && __ballot(G.real && ctl[b * 4 + 2] != 0) == 0) return;  // nothing flagged here
  const int n0n = n0 * n;
  const int nch_am = nprob * rg.amp / W, nch_dm = nprob * rg.dmp / W;
  C* th = lds + FL.th + p * n * n;
  C* piv = lds + FL.piv + p * 2 * n;  // two pivot rows
  const R* dmt = ldr + FL.dm + p * rg.dmp;
  const R* a0 = ldr + FL.a0 + p * n0n;
  for (int e = tid; e < nprob * n0n; e += kWave) ldr[FL.a0 + e] = A0[(size_t)b0 * n0n + e];
  // stage runs of the next stage are loaded into registers while the current
  // stage computes (as in admm_stream_kernel)
  auto run = [&](const R* arr, int pitch, int t) {
    return reinterpret_cast<const V*>(arr + ((size_t)t * B + b0) * pitch);
  };
  struct Regs {
    V am[CH_AM], dm[CH_TH];
  } nxt;
  auto load = [&](int t) {
    load_run<V, CH_AM>(nxt.am, run(am, rg.amp, t), nch_am);
    load_run<V, CH_TH>(nxt.dm, run(dm, rg.dmp, t), nch_dm);
  };
  load(0);
  const C rho_i = (C)rho[b];
  const C rho_f = rho_i * (C)rho_f_factor;
  const C sig = (C)sigma;

  C a[NC];  // row i of Theta_t, then of Theta_t^{-1}
  for (int t = 0; t < T; ++t) {
    const int cur = (t & 1) * (P * rg.amp), prv = ((t & 1) ^ 1) * (P * rg.amp);
    store_run<V, CH_AM>(nxt.am, reinterpret_cast<V*>(ldr + FL.am + cur), nch_am);
    store_run<V, CH_TH>(nxt.dm, reinterpret_cast<V*>(ldr + FL.dm), nch_dm);
    wsync();
    if (t + 1 < T) load(t + 1);
    const R* amc = ldr + FL.am + cur + p * rg.amp;
    const R* amq = ldr + FL.am + prv + p * rg.amp;
    if (i < n) {
      // theta_t row i.  Every loop body below issues its LDS reads, then a
      // scheduling barrier, then its FMAs, so the reads of a body share one
      // round trip.
      C c[NC];
      {
        R dk[NC];
        if (diag) {
#pragma unroll
          for (int k = 0; k < NC; ++k) dk[k] = k == i ? dmt[i] : R(0);
        } else {
#pragma unroll
          for (int k = 0; k < NC; ++k) dk[k] = dmt[pidx(i, k)];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < NC; ++k) {
          a[k] = (C)dk[k] + (k == i ? sig : C(0));
          c[k] = C(0);
        }
      }
      // c += sum_r w_r M[r][i] M[r][:] over rows r0..r1-1 of an (rows x n)
      // block, two rows per round trip; w_r = rho_f below row wsplit, rho from it
      auto gram = [&](const R* M, int r0, int r1, int wsplit) {
        for (int r = r0; r < r1; r += 2) {
          const bool two = r + 1 < r1;
          R m0[NC], m1[NC];
          const R a0v = M[r * n + i];
          const R a1v = M[(two ? r + 1 : r) * n + i];
#pragma unroll
          for (int k = 0; k < NC; ++k) {
            m0[k] = M[r * n + k];
            m1[k] = M[(two ? r + 1 : r) * n + k];
          }
          __builtin_amdgcn_sched_barrier(0);
          const C s0 = (C)a0v * (r < wsplit ? rho_f : rho_i);
          const C s1 = two ? (C)a1v * (r + 1 < wsplit ? rho_f : rho_i) : C(0);
#pragma unroll
          for (int k = 0; k < NC; ++k) c[k] += s0 * (C)m0[k] + s1 * (C)m1[k];
        }
      };
      if (t == 0) gram(a0, 0, n0, n0);
      gram(amc, t < N ? 0 : nx, nx + m, nx);  // [A_minus_t; G_t]
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        if (t > 0 && k == i && i < nx) c[k] += rho_f;  // rho_f A_plus_{t-1}^T A_plus_{t-1} = rho_f diag(I_nx, 0)
        a[k] += c[k];
      }
      // Schur update of the leading nx x nx block
      if (t > 0 && i < nx) {
        C mr[NC];
        R aq[NC];
#pragma unroll
        for (int k = 0; k < NC; ++k) aq[k] = amq[i * n + k];
#pragma unroll
        for (int j = 0; j < NC; ++j) mr[j] = C(0);
#pragma unroll
        for (int k = 0; k < NC; ++k) {
          C tk[NC];
#pragma unroll
          for (int j = 0; j < NC; ++j) tk[j] = th[k * n + j];
          __builtin_amdgcn_sched_barrier(0);
          const C ak = (C)aq[k];
#pragma unroll
          for (int j = 0; j < NC; ++j) mr[j] += ak * tk[j];
        }
        const C f2 = rho_f * rho_f;
#pragma unroll
        for (int s = 0; s < NC; ++s) {
          if (s < nx) {
            R qs[NC];
#pragma unroll
            for (int k = 0; k < NC; ++k) qs[k] = amq[s * n + k];
            __builtin_amdgcn_sched_barrier(0);
            C sv = C(0);
#pragma unroll
            for (int k = 0; k < NC; ++k) sv += mr[k] * (C)qs[k];
            a[s] -= f2 * sv;
          }
        }
      }
    }
    // Gauss-Jordan inversion without pivoting, rows in lanes (the pivots of an
    // SPD matrix stay positive), two pivots per LDS round trip: rows k and k+1
    // are broadcast together and every lane replays the two single-pivot steps
    // itself, forming row k+1 after step k from the pair, so the arithmetic is
    // that of one pivot at a time (a closed-form 2x2 block inverse instead
    // loses digits on strongly coupled pivot pairs).  The pivot row of a step
    // is not normalized at its step: its lane keeps the pivot as a scale
    // (myip) and normalizes after the last step, so every lane runs the same
    // instructions.
    C myip = C(1);
#pragma unroll
    for (int k = 0; k < NC; k += 2) {
      const bool pair = k + 1 < NC;
      wsync();
      if (i == k || (pair && i == k + 1))
#pragma unroll
        for (int j = 0; j < NC; ++j) piv[(i - k) * NC + j] = a[j];
      wsync();
      if (i < n) {
        C p1[NC], p2[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          p1[j] = piv[j];
          p2[j] = pair ? piv[NC + j] : C(0);
        }
        __builtin_amdgcn_sched_barrier(0);
        const bool m0 = i == k, m1 = pair && i == k + 1;
        // step k
        const C ip = C(1) / p1[k];
        myip = m0 ? ip : myip;
        const C g = m0 ? C(0) : a[k] * ip;
#pragma unroll
        for (int j = 0; j < NC; ++j) a[j] = (j == k) ? (m0 ? C(1) : -g) : a[j] - g * p1[j];
        if (pair) {
          // row k+1 after step k (what lane k+1 now holds), in place of p2
          const C gq = p2[k] * ip;
#pragma unroll
          for (int j = 0; j < NC; ++j) p2[j] = (j == k) ? -gq : p2[j] - gq * p1[j];
          // step k+1
          const C ip2 = C(1) / p2[k + 1];
          myip = m1 ? ip2 : myip;
          const C g2 = m1 ? C(0) : a[k + 1] * ip2;
#pragma unroll
          for (int j = 0; j < NC; ++j) a[j] = (j == k + 1) ? (m1 ? C(1) : -g2) : a[j] - g2 * p2[j];
        }
      }
    }
    wsync();
    if (i < n)
#pragma unroll
      for (int j = 0; j < NC; ++j) a[j] *= myip;
    // keep the symmetric part of the computed inverse (row i averaged with
    // column i): mirroring one triangle of the slightly asymmetric result
    // breaks its small residual at cond(Theta) ~ 1e9 (large rho_f), and the
    // ADMM iteration then diverges
    if (i < n)
#pragma unroll
      for (int j = 0; j < NC; ++j) th[i * n + j] = a[j];
    wsync();
    if (i < n) {
      C col[NC];
#pragma unroll
      for (int k = 0; k < NC; ++k) col[k] = th[k * n + i];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < NC; ++k) a[k] = C(0.5) * (a[k] + col[k]);
    }
    wsync();
    if (i < n) {
#pragma unroll
      for (int j = 0; j < NC; ++j) th[i * n + j] = a[j];
      if (G.live) {
        R* out = thinv + ((size_t)t * B + b) * PITCH + ((i * (i + 1)) >> 1);
#pragma unroll
        for (int k = 0; k < NC; ++k)
          if (k <= i) out[k] = (R)a[k];
      }
    }
    wsync();
  }
  if (ctl != nullptr && G.live && i == 0) ctl[b * 4 + 2] = 0;
}

}  // namespace tmpc
