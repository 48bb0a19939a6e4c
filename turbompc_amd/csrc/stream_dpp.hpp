// Group vectors through DPP row broadcasts for the streaming kernel.
//
// A problem's group holds a vector one element per lane (lane k of the group,
// k < NL <= 32).  When the group starts on a 16-lane row boundary and, for
// groups of more than 16 lanes, the row after it holds no other group (one or
// two problems per wavefront, at lane offsets 0 and 32), every lane of the
// group can read element k without LDS: v_permlane16_swap of the vector with
// itself gives
//   x: each even row's values in both rows of its pair  [r0, r0, r2, r2],
//   y: each odd row's values in both rows of its pair   [r1, r1, r3, r3],
// so element k < 16 is lane k of x's row (DPP row_newbcast:k) and element
// k >= 16 is lane k - 16 of y's row (a 32-lane group at lane offset 0 or 32
// reads its whole vector the same way).  The dot products fold the broadcast into
// v_fmac_dpp (the compiler keeps a broadcast as a separate move), so a
// product with a vector costs one VALU instruction per term and no LDS
// round trip.
#pragma once
#include "common.hpp"

namespace tmpc {

template <typename R>
struct RowPair {
  R x, y;
};

__device__ __forceinline__ RowPair<float> row_pair(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return {__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1])};
}
__device__ __forceinline__ RowPair<double> row_pair(double v) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)u, hi = (unsigned)(u >> 32);
  const auto rl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto rh = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  const auto cat = [](unsigned l, unsigned h) {
    return __builtin_bit_cast(double, ((unsigned long long)h << 32) | l);
  };
  return {cat((unsigned)rl[0], (unsigned)rh[0]), cat((unsigned)rl[1], (unsigned)rh[1])};
}

// sum_k w[k] v[k] for k < N: even and odd k in two chains (fp32 chains start
// with a multiply; fp64 has no v_mul_f64_dpp, its chains start at zero), then
// added.  Every lane of the wavefront must be active.  The s_nop before a
// block gives the DPP sources the wait states a DPP read needs after a VALU
// write; the one after covers a DPP read of the sums that follows.

__device__ __forceinline__ float dot_pair(const float (&w)[6], const RowPair<float>& v) {
  float a0, a1;
  asm volatile(
      "s_nop 4\n"
      "v_mul_f32_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "=&v"(a0), "=&v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]));
  return a0 + a1;
}

__device__ __forceinline__ float dot_pair(const float (&w)[9], const RowPair<float>& v) {
  float a0, a1;
  asm volatile(
      "s_nop 4\n"
      "v_mul_f32_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %10 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %11 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %12 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "=&v"(a0), "=&v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]));
  return a0 + a1;
}

__device__ __forceinline__ float dot_pair(const float (&w)[16], const RowPair<float>& v) {
  float a0, a1;
  asm volatile(
      "s_nop 4\n"
      "v_mul_f32_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %10 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %11 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %12 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %13 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %14 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %15 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %16 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %17 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %18 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %19 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "=&v"(a0), "=&v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]));
  return a0 + a1;
}

__device__ __forceinline__ float dot_pair(const float (&w)[17], const RowPair<float>& v) {
  float a0, a1;
  asm volatile(
      "s_nop 4\n"
      "v_mul_f32_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %10 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %11 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %12 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %13 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %14 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %15 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %16 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %17 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %18 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %19 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %20 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "=&v"(a0), "=&v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]), "v"(w[16]));
  return a0 + a1;
}

__device__ __forceinline__ double dot_pair(const double (&w)[6], const RowPair<double>& v) {
  double a0 = 0.0, a1 = 0.0;
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a0), "+v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]));
  return a0 + a1;
}

__device__ __forceinline__ double dot_pair(const double (&w)[9], const RowPair<double>& v) {
  double a0 = 0.0, a1 = 0.0;
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %10 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %11 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %12 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a0), "+v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]));
  return a0 + a1;
}

__device__ __forceinline__ double dot_pair(const double (&w)[16], const RowPair<double>& v) {
  double a0 = 0.0, a1 = 0.0;
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %10 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %11 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %12 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %13 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %14 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %15 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %16 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %17 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %18 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %19 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a0), "+v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]));
  return a0 + a1;
}

__device__ __forceinline__ double dot_pair(const double (&w)[17], const RowPair<double>& v) {
  double a0 = 0.0, a1 = 0.0;
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %10 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %11 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %12 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %13 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %14 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %15 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %16 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %17 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %18 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %19 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %3, %20 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a0), "+v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]), "v"(w[16]));
  return a0 + a1;
}

// 32-element vectors (32-lane groups): element k >= 16 is lane k - 16 of y's row.

__device__ __forceinline__ float dot_pair(const float (&w)[32], const RowPair<float>& v) {
  float a0, a1;
  asm volatile(
      "s_nop 4\n"
      "v_mul_f32_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_mul_f32_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %10 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %11 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %12 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %13 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %14 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %15 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %16 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %17 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %18 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %2, %19 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %20 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %3, %21 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %22 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %3, %23 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %24 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %3, %25 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %26 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %3, %27 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %28 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %3, %29 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %30 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %3, %31 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %32 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %3, %33 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %34 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %1, %3, %35 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "=&v"(a0), "=&v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]), "v"(w[16]), "v"(w[17]), "v"(w[18]), "v"(w[19]), "v"(w[20]), "v"(w[21]), "v"(w[22]), "v"(w[23]), "v"(w[24]), "v"(w[25]), "v"(w[26]), "v"(w[27]), "v"(w[28]), "v"(w[29]), "v"(w[30]), "v"(w[31]));
  return a0 + a1;
}

__device__ __forceinline__ double dot_pair(const double (&w)[32], const RowPair<double>& v) {
  double a0 = 0.0, a1 = 0.0;
  asm volatile(
      "s_nop 4\n"
      "v_fmac_f64_dpp %0, %2, %4 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %5 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %6 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %7 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %8 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %9 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %10 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %11 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %12 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %13 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %14 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %15 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %16 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %17 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %2, %18 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %2, %19 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %3, %20 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %3, %21 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %3, %22 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %3, %23 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %3, %24 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %3, %25 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %3, %26 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %3, %27 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %3, %28 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %3, %29 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %3, %30 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %3, %31 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %3, %32 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %3, %33 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %0, %3, %34 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f64_dpp %1, %3, %35 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
      "s_nop 1"
      : "+v"(a0), "+v"(a1)
      : "v"(v.x), "v"(v.y), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]), "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]), "v"(w[16]), "v"(w[17]), "v"(w[18]), "v"(w[19]), "v"(w[20]), "v"(w[21]), "v"(w[22]), "v"(w[23]), "v"(w[24]), "v"(w[25]), "v"(w[26]), "v"(w[27]), "v"(w[28]), "v"(w[29]), "v"(w[30]), "v"(w[31]));
  return a0 + a1;
}

}  // namespace tmpc
