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

namespace tmpc {

constexpr int kWave = 64;

struct Dims {
  int B, T, N, n, nx, n0, m;
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
__device__ __forceinline__ float rsqrt_(float a) { return sqrtf(a); }
__device__ __forceinline__ double rsqrt_(double a) { return sqrt(a); }

template <typename R>
__device__ __forceinline__ R rinf() {
  return __builtin_huge_val();
}

// Wavefront-wide sum / max by butterfly shuffles: every lane ends with the
// same value, combined in the same fixed order on every run.
template <typename R>
__device__ __forceinline__ R wave_sum(R v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <typename R>
__device__ __forceinline__ R wave_max(R v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = rmax(v, __shfl_xor(v, off));
  return v;
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
