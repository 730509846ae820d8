// Per-row QK-RMSNorm + NeoX RoPE of one head (D = 128) on a 32-lane group,
// shared by the fused norm/RoPE/KV-write kernel and the fused decode
// attention kernel.
//
// Reference math: qk_norm_rope_kv_prefill_raw_f16 / _decode_raw_f16
// (src/kernels.rs:4837-5452):
//   ss = sum(x^2); inv = rsqrt(ss/D + eps); n = x*inv*gamma;
//   y_lo = n_lo*cos - n_hi*sin; y_hi = n_hi*cos + n_lo*sin; f16(y)
//
// Lane j (0..31) of the group owns elements 4j..4j+3; lanes j and j^16 hold
// the RoPE partners d and d+64.  Every step is an IEEE-defined operation in a
// fixed order (no contraction: the sum of squares is the in-lane
// (a^2+b^2)+(c^2+d^2) followed by the butterfly over partners l^16, l^8,
// l^4, l^2, l^1; 1/sqrt is a fixed double-precision Newton sequence; cos/sin
// come from a host-built fp32 table), so the rotated K rows match a CPU
// restatement bit for bit.
#pragma once

#include "common.hpp"

namespace grout {

__device__ __forceinline__ float rsqrt_det(float v) {
#pragma clang fp contract(off)
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  b = 0x5f3759dfu - (b >> 1);
  double y = (double)__builtin_bit_cast(float, b);
  const double vd = (double)v;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    double t = vd * y;
    t = t * y;
    t = 0.5 * t;
    t = 1.5 - t;
    y = y * t;
  }
  return (float)y;
}

// Lane exchanges inside one 32-lane group, on the VALU (no LDS round trip):
// xor16 swaps the two 16-lane halves, ror16<N> reads lane (l+N) mod 16 of the
// same half.
__device__ __forceinline__ float xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  // r[0]: odd halves take the even half's value; r[1]: even halves take the odd half's
  return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
template <int N>
__device__ __forceinline__ float ror16(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x120 + N, 0xf, 0xf, false));
}

// Rotated, normalized row: lane j passes its 4 input halves xr (elements
// 4j..4j+3), its gamma halves gh, and the cos/sin of angle index 4(j%16)..+3
// at the row's position; returns its 4 output halves.  All 32 lanes of the
// group must be active.
__device__ __forceinline__ u32x2 norm_rope_row(u32x2 xr, half4 gh, floatx4 c, floatx4 sn, int j,
                                               float eps) {
#pragma clang fp contract(off)
  const half4 xh = __builtin_bit_cast(half4, xr);
  const float x0 = (float)xh[0], x1 = (float)xh[1], x2 = (float)xh[2], x3 = (float)xh[3];
  // After the l^16 and l^8 steps lanes l and l^8 hold equal values, so the
  // rotation partners (l+-4, l+-2, l+-1 mod 16) add exactly the values the
  // xor partners would.
  float a0 = x0 * x0, a1 = x1 * x1, a2 = x2 * x2, a3 = x3 * x3;
  float s0 = a0 + a1, s1 = a2 + a3;
  float ss = s0 + s1;
  ss = ss + xor16(ss);
  ss = ss + ror16<8>(ss);
  ss = ss + ror16<4>(ss);
  ss = ss + ror16<2>(ss);
  ss = ss + ror16<1>(ss);
  const float mean = ss / (float)kHeadDim;
  const float inv = rsqrt_det(mean + eps);

  float n[4];
  n[0] = (x0 * inv) * (float)gh[0];
  n[1] = (x1 * inv) * (float)gh[1];
  n[2] = (x2 * inv) * (float)gh[2];
  n[3] = (x3 * inv) * (float)gh[3];
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = xor16(n[i]);  // RoPE partner (d +/- 64)

  half4 y;
  if (j < 16) {  // low half: y = n_lo*c - n_hi*s
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float t0 = n[i] * c[i];
      float t1 = p[i] * sn[i];
      y[i] = (half_t)(t0 - t1);
    }
  } else {  // high half: y = n_hi*c + n_lo*s
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float t0 = n[i] * c[i];
      float t1 = p[i] * sn[i];
      y[i] = (half_t)(t0 + t1);
    }
  }
  return __builtin_bit_cast(u32x2, y);
}

// The same row on an 8-lane group (8 rows per wave): lane i (0..7) owns
// elements 8i..8i+7 ("lo", x16 bytes 16i..) and their RoPE partners
// 8i+64..8i+71 ("hi", bytes 128+16i..), so the rotation needs no exchange.
// The sum of squares pairs exactly as in norm_rope_row (and the CPU
// restatement): with group g = elements 4g..4g+3, lane i holds groups 2i,
// 2i+1 (lo) and 2i+16, 2i+17 (hi); the butterfly's distance-16 step adds them
// in-lane, distances 8, 4 and 2 are lanes i^4, i^2, i^1, distance 1 adds the
// two lane values.  IEEE addition commutes, so every sum equals the 32-lane
// tree's bit for bit.  All 8 lanes of the group must be active.
__device__ __forceinline__ float xor_lane4(float x) {
  // DPP row half-mirror then quad reversal (common.hpp), the same partner as
  // the ds_swizzle xor-4 mode without its LDS round trip
  return xor_lane<4>(x);
}
__device__ __forceinline__ float xor_lane2(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4e, 0xf, 0xf, false));
}
__device__ __forceinline__ float xor_lane1(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xb1, 0xf, 0xf, false));
}

__device__ __forceinline__ void norm_rope_row8(u32x4 xlo, u32x4 xhi, half8 glo, half8 ghi,
                                               const float (&c)[8], const float (&sn)[8],
                                               float eps, u32x4& ylo, u32x4& yhi) {
#pragma clang fp contract(off)
  const half8 l = __builtin_bit_cast(half8, xlo), hh = __builtin_bit_cast(half8, xhi);
  float xl[8], xh[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    xl[e] = (float)l[e];
    xh[e] = (float)hh[e];
  }
  auto grp = [](const float* x) {
    const float a = x[0] * x[0], b = x[1] * x[1], cc = x[2] * x[2], d = x[3] * x[3];
    const float s0 = a + b, s1 = cc + d;
    return s0 + s1;
  };
  // distance 16: group 2i + group 2i+16, group 2i+1 + group 2i+17
  float u0 = grp(xl) + grp(xh);
  float u1 = grp(xl + 4) + grp(xh + 4);
  u0 = u0 + xor_lane4(u0);
  u1 = u1 + xor_lane4(u1);
  u0 = u0 + xor_lane2(u0);
  u1 = u1 + xor_lane2(u1);
  u0 = u0 + xor_lane1(u0);
  u1 = u1 + xor_lane1(u1);
  const float ss = u0 + u1;
  const float mean = ss / (float)kHeadDim;
  const float inv = rsqrt_det(mean + eps);

  half8 yl, yh;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float nl = (xl[e] * inv) * (float)glo[e];
    const float nh = (xh[e] * inv) * (float)ghi[e];
    const float a = nl * c[e], b = nh * sn[e];
    yl[e] = (half_t)(a - b);
    const float f = nh * c[e], g = nl * sn[e];
    yh[e] = (half_t)(f + g);
  }
  ylo = __builtin_bit_cast(u32x4, yl);
  yhi = __builtin_bit_cast(u32x4, yh);
}

}  // namespace grout
