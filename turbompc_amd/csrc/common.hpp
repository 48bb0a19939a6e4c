// Shared device-side types and helpers for the gfx950 MPC kernels.
//
// Data at the boundary keeps the reference's batched layout: a leading problem
// axis and row-major blocks per problem (turbompc/solvers/qp_data.py:11-100 as
// seen by the FFI under vmap "broadcast_all",
// turbompc/solvers/admm/admm_cudss_ffi_backend.py:131-155).  Internal
// workspaces are stage-major ([t][b][...]) so the problems that share a
// wavefront read one contiguous run of HBM per stage.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace tmpc {

constexpr int kWave = 64;

// n: the block width of the kernels' records; nq: the row length of the QP
// and state arrays (nq <= n: the streaming path rounds n up to a width it is
// built for, the extra variables being decoupled dummies; nq = n elsewhere).
struct Dims {
  int B, T, N, n, nx, n0, m, nq;
};

template <typename R>
struct QPDev {
  const R *D, *E, *q, *A0, *Am, *Ap, *G, *l, *u, *c0, *c;
  const R* slack_w;  // (B,) or null (= 0)
};

template <typename R>
struct StateDev {
  R *x, *z, *y_g, *y_f0, *y_f, *xi, *rho;
};

// packed symmetric (lower) index of element (i, k)
__device__ __forceinline__ int pidx(int i, int k) {
  return i >= k ? ((i * (i + 1)) >> 1) + k : ((k * (k + 1)) >> 1) + i;
}
__host__ __device__ __forceinline__ constexpr int packed_size(int n) { return (n * (n + 1)) / 2; }
// Stored pitch of one packed Theta^{-1} block: padded to a multiple of four
// elements so that every block starts on a 16-byte boundary and the blocks of
// consecutive problems load as one run of 128-bit accesses.
__host__ __device__ __forceinline__ constexpr int th_pitch(int n) { return (packed_size(n) + 3) & ~3; }

// `it % k == 0` with XLA's integer remainder convention (x % 0 == x), which is
// what the reference's jnp expressions evaluate to when k == 0.
__device__ __forceinline__ bool mod_zero(int it, int k) {
  return k > 0 ? (it % k) == 0 : it == 0;
}

// max / min / abs as single instructions (v_max, v_min, and the |x| source
// modifier).  On finite operands they equal the reference's jnp.maximum /
// jnp.minimum / jnp.abs; a NaN operand yields the other operand.
__device__ __forceinline__ float rmax(float a, float b) { return __builtin_fmaxf(a, b); }
__device__ __forceinline__ double rmax(double a, double b) { return __builtin_fmax(a, b); }
__device__ __forceinline__ float rmin(float a, float b) { return __builtin_fminf(a, b); }
__device__ __forceinline__ double rmin(double a, double b) { return __builtin_fmin(a, b); }
__device__ __forceinline__ float rabs(float a) { return __builtin_fabsf(a); }
__device__ __forceinline__ double rabs(double a) { return __builtin_fabs(a); }
// the square root in the value's own precision (not its reciprocal)
__device__ __forceinline__ float r_sqrt(float a) { return sqrtf(a); }
__device__ __forceinline__ double r_sqrt(double a) { return sqrt(a); }

template <typename R>
__device__ __forceinline__ R rinf() {
  return __builtin_huge_val();
}

// Wavefront-wide sum / max by butterfly shuffles: every lane ends with the
// same value, combined in the same fixed order on every run.
// v moved across lanes by the DPP control CTRL (a VALU move, no LDS)
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ double dpp_move(double v) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, 0xF, 0xF, true);
  const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, 0xF, 0xF, true);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ float read_lane(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double read_lane(double v, int l) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, l);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), l);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// Sum over each 16-lane row, the same value in every lane of the row: pairs,
// quads, half rows, rows (every step adds two equal-shaped partials, so all
// lanes of a row end with the same bits).  Every lane must be active.
template <typename R>
__device__ __forceinline__ R row_sum(R v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_move<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  return v;
}

// Sum over the 64 lanes, the same value in every lane, in a fixed order:
// within each 16-lane row by DPP moves (pairs, quads, half rows, rows; every
// step adds two equal-shaped partials, so all lanes of a row end with the same
// bits), then the four row sums.  Every lane must be active.
template <typename R>
__device__ __forceinline__ R wave_sum(R v) {
  v = row_sum(v);
  return (read_lane(v, 0) + read_lane(v, 16)) + (read_lane(v, 32) + read_lane(v, 48));
}

template <typename R>
__device__ __forceinline__ R wave_max(R v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = rmax(v, __shfl_xor(v, off));
  return v;
}

// Lane K of each 16-lane row of the wavefront, broadcast to the whole row
// (DPP row_newbcast; a VALU move, no LDS).  Every lane of the wavefront must
// be active where it is used.
template <int K>
__device__ __forceinline__ float row_bcast(float v) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + K, 0xF, 0xF, true));
}
template <int K>
__device__ __forceinline__ double row_bcast(double v) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)u, 0x150 + K, 0xF, 0xF, true);
  const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), 0x150 + K, 0xF, 0xF, true);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// row_bcast with a lane index that is a constant after unrolling
template <typename R>
__device__ __forceinline__ R row_bcast_at(R v, int k) {
  switch (k) {
    case 0: return row_bcast<0>(v);
    case 1: return row_bcast<1>(v);
    case 2: return row_bcast<2>(v);
    case 3: return row_bcast<3>(v);
    case 4: return row_bcast<4>(v);
    case 5: return row_bcast<5>(v);
    case 6: return row_bcast<6>(v);
    case 7: return row_bcast<7>(v);
    case 8: return row_bcast<8>(v);
    case 9: return row_bcast<9>(v);
    case 10: return row_bcast<10>(v);
    case 11: return row_bcast<11>(v);
    case 12: return row_bcast<12>(v);
    case 13: return row_bcast<13>(v);
    case 14: return row_bcast<14>(v);
    default: return row_bcast<15>(v);
  }
}

// sum_k w[k] s_k for k < NC (even and odd k summed in order, then added),
// where s_k is the value s of lane k of this lane's 16-lane row
template <typename R, int NC, int... K>
__device__ __forceinline__ R row_dot_seq(const R (&w)[NC], R s, std::integer_sequence<int, K...>) {
  R acc[2] = {R(0), R(0)};  // even and odd k: two dependence chains
  ((acc[K & 1] += w[K] * row_bcast<K>(s)), ...);
  return acc[0] + acc[1];
}
template <int NC, typename R>
__device__ __forceinline__ R row_dot(const R (&w)[NC], R s) {
  return row_dot_seq<R, NC>(w, s, std::make_integer_sequence<int, NC>{});
}

// The same sums with the broadcast folded into the arithmetic (v_*_dpp
// row_newbcast: one instruction per term instead of a move and an FMA; in
// fp32 the first term of each chain initialises it with a multiply, which has
// no DPP form in fp64).  The compiler does not form these, so they are written
// out; the s_nop before the block gives the DPP source the wait states a DPP
// read needs after a VALU write of its operand, and the one after covers a
// DPP read of the sums that follows.

__device__ __forceinline__ float row_dot_dpp(const float (&w)[6], float s) {
  float a0, a1;
  asm volatile(
      "s_nop 4\n"
      "v_mul_f32_dpp %0, %2, %3 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %1, %2, %4 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %5 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %6 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %7 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %8 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "=&v"(a0), "=&v"(a1)
      : "v"(s), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]));
  return a0 + a1;
}

__device__ __forceinline__ float row_dot_dpp(const float (&w)[9], float s) {
  float a0, a1;
  asm volatile(
      "s_nop 4\n"
      "v_mul_f32_dpp %0, %2, %3 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %1, %2, %4 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %5 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %6 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %7 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %8 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %9 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %10 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %11 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "=&v"(a0), "=&v"(a1)
      : "v"(s), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]));
  return a0 + a1;
}

__device__ __forceinline__ float row_dot_dpp(const float (&w)[16], float s) {
  float a0, a1;
  asm volatile(
      "s_nop 4\n"
      "v_mul_f32_dpp %0, %2, %3 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %1, %2, %4 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %5 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %6 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %7 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %8 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %9 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %10 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %11 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %12 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %13 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %14 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %15 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %16 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %17 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %18 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "=&v"(a0), "=&v"(a1)
      : "v"(s), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]));
  return a0 + a1;
}

__device__ __forceinline__ double row_dot_dpp(const double (&w)[6], double s) {
  double a0 = double(0), a1 = double(0);
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %2, %3 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %4 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %5 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %6 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %7 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %8 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a0), "+v"(a1)
      : "v"(s), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]));
  return a0 + a1;
}

__device__ __forceinline__ double row_dot_dpp(const double (&w)[9], double s) {
  double a0 = double(0), a1 = double(0);
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %2, %3 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %4 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %5 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %6 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %7 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %8 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %9 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %10 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %11 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a0), "+v"(a1)
      : "v"(s), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]));
  return a0 + a1;
}

__device__ __forceinline__ double row_dot_dpp(const double (&w)[16], double s) {
  double a0 = double(0), a1 = double(0);
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %2, %3 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %4 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %5 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %6 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %7 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %8 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %9 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %10 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %11 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %12 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %13 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %14 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %15 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %16 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %17 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %18 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a0), "+v"(a1)
      : "v"(s), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]));
  return a0 + a1;
}

// Fills n words with v.  Used instead of hipMemsetAsync so that a solve
// captured in a HIP graph holds kernel nodes only.
template <typename W>
__global__ void fill_kernel(W* p, size_t n, W v) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Sets bit 31 of iters[b] (TMPC_ITERS_NONFINITE) when problem b's state
// holds a NaN or an infinity.  One wavefront per problem reads its arrays
// (contiguous per problem) once; lane 0 updates the word with a plain store.
template <typename R>
__global__ __launch_bounds__(64) void nonfinite_flag_kernel(Dims d, StateDev<R> st, uint32_t* iters) {
  const int b = blockIdx.x, lane = threadIdx.x;
  bool bad = false;
  auto scan = [&](const R* p, int cnt) {
    if (p == nullptr || cnt == 0) return;
    const R* q = p + (size_t)b * cnt;
    for (int k = lane; k < cnt; k += kWave) bad |= !__builtin_isfinite(q[k]);
  };
  scan(st.x, d.T * d.n);
  scan(st.z, d.T * d.m);
  scan(st.y_g, d.T * d.m);
  scan(st.xi, d.T * d.m);
  scan(st.y_f0, d.n0);
  scan(st.y_f, d.N * d.nx);
  scan(st.rho, 1);
  if (__ballot(bad) != 0 && lane == 0) iters[b] |= 0x80000000u;
}

// One workgroup is one wavefront; LDS traffic between lanes of the wave is
// ordered by this barrier (a single-wave s_barrier is cheap on CDNA).
__device__ __forceinline__ void wsync() { __syncthreads(); }

// Orders LDS accesses between lanes of one wavefront without waiting: the LDS
// unit executes one wavefront's instructions in issue order, so a read issued
// after another lane's write returns the written value; only the compiler has
// to keep the accesses in program order (the memory clobber), and each use of
// a read still waits for its own data.  For single-wavefront workgroups only.
__device__ __forceinline__ void lds_order() { asm volatile("" ::: "memory"); }

// A wavefront is split into P = 64 / g groups of g lanes; group p owns one
// problem and lane i of the group owns row i of every stage block.
// Reads always use `prob` (clamped into [0, B) so a partially filled last
// wave never reads past the arrays); writes are predicated on `live`.  The idle
// tail lanes get lane >= g, so every row-bounded access skips them.
struct Group {
  int lane;   // lane within group, 0..g-1 (>= g for the idle tail lanes)
  int gid;    // group within wave
  int prob;   // problem index, clamped to B-1
  bool live;  // owns a real row of a real problem
  bool real;  // the group maps to a real problem (any lane, including lane >= g)
};

__device__ __forceinline__ Group make_group(int g, int P, int B) {
  Group G;
  const int tid = threadIdx.x;
  G.gid = tid / g;
  G.lane = tid - G.gid * g;
  if (G.gid >= P) {  // idle tail lanes of the wave
    G.gid = P - 1;
    G.lane = g + (tid - P * g);
  }
  const int raw = blockIdx.x * P + G.gid;
  G.prob = raw < B ? raw : B - 1;
  G.live = (G.lane < g) && (tid < P * g) && (raw < B);
  G.real = (tid < P * g) && (raw < B);
  return G;
}

// Groups at lane offsets 0, S, 2S, ... with S = 64 / P.  For P = 2 each group
// sits in its own half-wave, so the LDS accesses of different groups never
// share an LDS pass and cannot conflict on a bank.  Every lane belongs to a
// group; lanes at offset >= g inside a group are idle (lane >= g).
__device__ __forceinline__ Group make_group_strided(int g, int P, int B) {
  Group G;
  const int tid = threadIdx.x, S = kWave / P;
  G.gid = min(tid / S, P - 1);
  G.lane = tid - G.gid * S;
  const int raw = blockIdx.x * P + G.gid;
  G.prob = raw < B ? raw : B - 1;
  G.live = G.lane < g && raw < B;
  G.real = raw < B;
  return G;
}

}  // namespace tmpc
