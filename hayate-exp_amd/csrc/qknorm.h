// q/k RMSNorm and RoPE of one 128-element head row held by 16 lanes x 8
// elements, shared by the append kernel and the decode kernel's fused
// append. Every product and sum is rounded separately (the file that
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
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x120 + N, 0xf, 0xf, false));
}
template <int N>
__device__ __forceinline__ double row_ror_f64(double x) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(x));
  const uint64_t lo = row_ror<N>(static_cast<uint32_t>(u));
  const uint64_t hi = row_ror<N>(static_cast<uint32_t>(u >> 32));
  return __longlong_as_double(static_cast<long long>((hi << 32) | lo));
}
// Value of lane l ^ 8 of the row (a rotation by 8 of 16).
__device__ __forceinline__ float row_xor8(float x) {
  return __uint_as_float(row_ror<8>(__float_as_uint(x)));
}
// Sum over the 16 lanes of a row, in every lane: rotations by 8, 4, 2, 1.
// The terms are exact squares of bf16 values and fp64 holds their sum
// exactly, so the order does not matter.
__device__ __forceinline__ double row16_sum_f64(double x) {
  x += row_ror_f64<8>(x);
  x += row_ror_f64<4>(x);
  x += row_ror_f64<2>(x);
  x += row_ror_f64<1>(x);
  return x;
}

__device__ __forceinline__ void rms_norm8(float (&x)[8],
                                          const uint16_t *__restrict__ w,
                                          int lane, float eps) {
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += static_cast<double>(x[j] * x[j]);
  ss = row16_sum_f64(ss);
  const float mean = static_cast<float>(ss) * (1.0f / kHeadDim);
  const float root = static_cast<float>(sqrt(static_cast<double>(mean + eps)));
  const float rstd = static_cast<float>(1.0 / static_cast<double>(root));
  const u32x4 wv = load16(w + lane * 8);
  float wf[8];
  unpack8(wv, wf);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float y = (x[j] * rstd) * wf[j];
    x[j] = bf16_to_f32(static_cast<uint16_t>(f32_to_bf16_rne(y)));
  }
}

// y = bf16(x * cos + rotate_half(x) * sin), rotate_half(x) = cat(-x2, x1)
// (hayate/model/rope.py:31-47). Lane l holds features 8l..8l+7; its partner
// l ^ 8 holds the other half.
__device__ __forceinline__ void rope8(float (&x)[8],
                                      const float *__restrict__ cos_row,
                                      const float *__restrict__ sin_row,
                                      int lane) {
  float other[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) other[j] = row_xor8(x[j]);
  const float sgn = lane < 8 ? -1.0f : 1.0f;
  const f32x4 c0 = *reinterpret_cast<const f32x4 *>(cos_row + lane * 8);
  const f32x4 c1 = *reinterpret_cast<const f32x4 *>(cos_row + lane * 8 + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4 *>(sin_row + lane * 8);
  const f32x4 s1 = *reinterpret_cast<const f32x4 *>(sin_row + lane * 8 + 4);
  const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float a = x[j] * c[j];
    const float r = (sgn * other[j]) * s[j];
    x[j] = a + r;
  }
}

}  // namespace hy
