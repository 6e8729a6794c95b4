// q/k RMSNorm and RoPE of one 128-element head row, held by 16 lanes x 8
// elements (the decode kernel's fused append) or by 8 lanes x 2 half rows
// (the append kernel). Every product and sum is rounded separately (the file that
// includes this must be built with -ffp-contract=off): the reference's
// chain of elementwise torch ops rounds each step (hayate/model/rope.py:44-47),
// so the results are bit-exact with it.
#pragma once

#include "hy_common.h"

namespace hy {

__device__ __forceinline__ void unpack8(const u32x4 w, float (&x)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[2 * j] = bf16_lo(w[j]);
    x[2 * j + 1] = bf16_hi(w[j]);
  }
}

__device__ __forceinline__ u32x4 pack8_rne(const float (&y)[8]) {
  u32x4 w;
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2_rne(y[2 * j], y[2 * j + 1]);
  return w;
}

// x' = bf16((x * rsqrt(mean(x^2) + eps)) * w), fp32 arithmetic, per head row
// held by 16 lanes x 8 elements (torch/_decomp/decompositions.py
// _fused_rms_norm: upcast, pow 2, mean, add eps, rsqrt, mul, mul weight,
// cast back).
// The squares of bf16 values are exact and so is their fp64 sum, so the
// mean is the correctly rounded one whatever the reduction order. sqrt and
// the reciprocal are taken in fp64 and rounded to fp32, which equals the
// correctly rounded fp32 operation (53 >= 2 * 24 + 2 makes the double
// rounding innocuous for both), independent of fp32 sqrt/div lowering.
// Lane data movement within 16-lane rows by DPP row rotations (VALU, no
// LDS round trip). A row holds a head row in full, so every lane a rotation
// reads is active whenever the destination is.
template <int N>
__device__ __forceinline__ uint32_t row_ror(uint32_t x) {
  static_assert(N >= 1 && N <= 15, "row_ror:1..15");
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x120 + N, 0xf, 0xf, false));
}
// Value of lane l ^ 8 of the row (a rotation by 8 of 16).
__device__ __forceinline__ float row_xor8(float x) {
  return __uint_as_float(row_ror<8>(__float_as_uint(x)));
}
// rsqrt(mean + eps) of a head row from its fp64 sum of squares: the mean
// rounded to fp32, then sqrt and reciprocal each correctly rounded to fp32.
__device__ __forceinline__ float rms_rstd(double ss, float eps) {
  const float mean = static_cast<float>(ss) * (1.0f / kHeadDim);
  const float root = static_cast<float>(sqrt(static_cast<double>(mean + eps)));
  return static_cast<float>(1.0 / static_cast<double>(root));
}

// Sum over the 8 lanes of an aligned group, in every lane; defined with the
// paired-half layout below.
__device__ __forceinline__ double group8_sum_f64(double x);

// wf: the 8 weights of this lane's features, already widened to fp32.
// The sum of squares is accumulated in exactly the order rms_norm16 uses
// for the same row: lane l < 8 and its partner l + 8 hold the two halves
// rms_norm16's group lane l holds, so each interleaves its own and its
// partner's squares (lo feature first) and both halves of the 16-lane row
// reduce like one 8-lane group. The fp64 sum is exact for all but rows whose
// squares span more than ~2^30; with one grouping the two layouts agree bit
// for bit even then.
__device__ __forceinline__ void rms_norm8(float (&x)[8], const float (&wf)[8], int lane,
                                          float eps) {
  const bool lo_half = lane < 8;
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const double own = static_cast<double>(x[j]);
    const double other = static_cast<double>(row_xor8(x[j]));
    const double a = lo_half ? own : other;
    const double b = lo_half ? other : own;
    ss = __builtin_fma(a, a, ss);
    ss = __builtin_fma(b, b, ss);
  }
  const float rstd = rms_rstd(group8_sum_f64(ss), eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = pack_bf16x2_rne((x[2 * j] * rstd) * wf[2 * j],
                                       (x[2 * j + 1] * rstd) * wf[2 * j + 1]);
    x[2 * j] = bf16_lo(w);
    x[2 * j + 1] = bf16_hi(w);
  }
}

__device__ __forceinline__ void rms_norm8(float (&x)[8],
                                          const uint16_t *__restrict__ w,
                                          int lane, float eps) {
  float wf[8];
  unpack8(load16(w + lane * 8), wf);
  rms_norm8(x, wf, lane, eps);
}

// y = bf16(x * cos + rotate_half(x) * sin), rotate_half(x) = cat(-x2, x1)
// (hayate/model/rope.py:31-47). Lane l holds features 8l..8l+7; its partner
// l ^ 8 holds the other half.
// c: cos of this lane's 8 features at the token's position; ss: their sin
// times -1 in lanes 0-7 (the half that rotate_half negates) and +1 in lanes
// 8-15. Negation is exact and (-o) * s rounds to o * (-s) bit for bit, so
// folding the sign into the table is the reference's arithmetic.
__device__ __forceinline__ void rope8_signed(float (&x)[8], const float (&c)[8],
                                             const float (&ss)[8]) {
  float other[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) other[j] = row_xor8(x[j]);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float a = x[j] * c[j];
    const float r = other[j] * ss[j];
    x[j] = a + r;
  }
}

// Loads this lane's 8 entries of a 128-wide fp32 table row.
__device__ __forceinline__ void load_row8(const float *__restrict__ row, int lane,
                                          float (&out)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4 *>(row + lane * 8);
  const f32x4 b = *reinterpret_cast<const f32x4 *>(row + lane * 8 + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out[j] = a[j];
    out[4 + j] = b[j];
  }
}

__device__ __forceinline__ void rope8(float (&x)[8],
                                      const float *__restrict__ cos_row,
                                      const float *__restrict__ sin_row,
                                      int lane) {
  float c[8], s[8];
  load_row8(cos_row, lane, c);
  load_row8(sin_row, lane, s);
  const float sgn = lane < 8 ? -1.0f : 1.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s[j] *= sgn;
  rope8_signed(x, c, s);
}

// ---------------------------------------------------------------------------
// Paired-half row layout: a head row is held by an aligned group of 8 lanes,
// lane l of the group holding features [8l, 8l + 8) ("lo") and
// [64 + 8l, 64 + 8l + 8) ("hi"). rotate_half pairs feature i with i + 64,
// so the rotation stays inside a lane, and the norm's row reduction spans 8
// lanes.
// ---------------------------------------------------------------------------
template <int Ctrl>
__device__ __forceinline__ double dpp_f64(double x) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(x));
  const uint64_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_mov_dpp(static_cast<int>(static_cast<uint32_t>(u)), Ctrl, 0xf, 0xf, false));
  const uint64_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_mov_dpp(static_cast<int>(static_cast<uint32_t>(u >> 32)), Ctrl, 0xf, 0xf, false));
  return __longlong_as_double(static_cast<long long>((hi << 32) | lo));
}

// Sum over the 8 lanes of an aligned group, in every lane: lane ^ 1 and
// lane ^ 2 (quad permutations), then lane i with 7 - i (half-row mirror).
// Each step adds two operands that every lane of the pair holds in swapped
// order, so all 8 lanes end with the same bits.
__device__ __forceinline__ double group8_sum_f64(double x) {
  x += dpp_f64<0xB1>(x);   // quad_perm [1, 0, 3, 2]
  x += dpp_f64<0x4E>(x);   // quad_perm [2, 3, 0, 1]
  x += dpp_f64<0x141>(x);  // row_half_mirror
  return x;
}

// RMSNorm of a row in the paired-half layout (same arithmetic as
// rms_norm8): squares of bf16 values are exact in fp64, so fma(x, x, ss)
// adds the exact square.
__device__ __forceinline__ void rms_norm16(float (&xl)[8], float (&xh)[8], const float (&wl)[8],
                                           const float (&wh)[8], float eps) {
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const double a = static_cast<double>(xl[j]);
    const double b = static_cast<double>(xh[j]);
    ss = __builtin_fma(a, a, ss);
    ss = __builtin_fma(b, b, ss);
  }
  const float rstd = rms_rstd(group8_sum_f64(ss), eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t a = pack_bf16x2_rne((xl[2 * j] * rstd) * wl[2 * j],
                                       (xl[2 * j + 1] * rstd) * wl[2 * j + 1]);
    const uint32_t b = pack_bf16x2_rne((xh[2 * j] * rstd) * wh[2 * j],
                                       (xh[2 * j + 1] * rstd) * wh[2 * j + 1]);
    xl[2 * j] = bf16_lo(a);
    xl[2 * j + 1] = bf16_hi(a);
    xh[2 * j] = bf16_lo(b);
    xh[2 * j + 1] = bf16_hi(b);
  }
}

// y = x * cos + rotate_half(x) * sin in the paired-half layout:
// lo: x_lo * c_lo + (-x_hi) * s_lo, rounded as x_lo * c_lo - x_hi * s_lo
// (negation is exact); hi: x_hi * c_hi + x_lo * s_hi.
__device__ __forceinline__ void rope16(float (&xl)[8], float (&xh)[8], const float (&cl)[8],
                                       const float (&ch)[8], const float (&sl)[8],
                                       const float (&sh)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float a = xl[j] * cl[j];
    const float b = xh[j] * sl[j];
    const float c = xh[j] * ch[j];
    const float d = xl[j] * sh[j];
    xl[j] = a - b;
    xh[j] = c + d;
  }
}

}  // namespace hy
