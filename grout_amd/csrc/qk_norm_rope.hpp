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

}  // namespace grout
