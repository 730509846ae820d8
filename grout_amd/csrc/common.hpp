// Device-side helpers shared by the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace grout {

typedef _Float16 half_t;
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;  // the reference enforces head_dim == 128 (src/model.rs:1446)
constexpr int kWave = 64;

// v_mfma_f32_16x16x32_f16.  Operand layout (lane l, 64 lanes):
//   A (16 x 32): row l%16, k-slot l/16 holding 8 consecutive k values
//   B (32 x 16): col l%16, same k-slot convention
//   C (16 x 16): col l%16, rows 4*(l/16) + i, i = 0..3
// Only the C layout matters for correctness as long as A and B fill their
// k-slots with the same index order; that is how every kernel here uses it.
__device__ __forceinline__ floatx4 mfma16x16x32(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }
__device__ __forceinline__ u32x4 as_u32x4(half8 v) { return __builtin_bit_cast(u32x4, v); }

// 16-byte global load that bypasses cache allocation for streamed data.
__device__ __forceinline__ u32x4 load_stream16(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Headroom (log2 units) of the fp16 probabilities that feed P.V.  The
// attention kernels form p = 2^(s - m) against m = running max - kPHeadroom
// rather than the max itself.  Then a tile whose p stay below
// 2^(8 + kPHeadroom) = 2^15 fits fp16 (65504 at most), and a weight down to
// 2^-31 of the largest still lands in fp16's range (subnormals reach 2^-24).
// Against the max itself, the weights below 2^-25 round to zero: with one key
// ~26 units above a long N(0,1) background, fp16 rounding drops ~27% of the
// background's mass, and none up to ~30 units with the headroom.  The factor
// 2^kPHeadroom is in every l and acc alike, so it cancels in acc / l and in
// the merges, which take (m, l) as a reference point and the sum of
// 2^(s - m).
constexpr float kPHeadroom = 7.0f;

// x / d for every x < 2^31 without a runtime division (one is ~20 dependent
// instructions with a reciprocal round trip, in front of every load whose
// address needs it): (x * m) >> sh with l = ceil(log2 d), m = ceil(2^(31+l) /
// d) < 2^32, sh = 31 + l (Granlund and Montgomery, "Division by invariant
// integers using multiplication", 1994, Thm 4.2: m d - 2^(31+l) < d <= 2^l).
// The host computes (m, sh) once per launch with make_div.
struct DivBy {
  uint32_t m;
  int sh;
};
__host__ __device__ inline uint32_t div_by(uint32_t x, DivBy d) {
  return (uint32_t)(((uint64_t)x * d.m) >> d.sh);
}
inline DivBy make_div(int d) {
  int l = 0;
  while ((1ll << l) < d) ++l;
  return DivBy{(uint32_t)(((1ull << (31 + l)) + (uint64_t)d - 1) / (uint64_t)d), 31 + l};
}

// Lane l ends with f(x[l], x[l ^ 16]) and then f(.., x[l ^ 32]): the reduction
// over the four 16-lane groups that hold one MFMA column, on the VALU
// (v_permlane16/32_swap, gfx950) instead of two LDS round trips.
__device__ __forceinline__ float col_max(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float col_sum(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Cross-lane xor shuffle within the wave (ds_bpermute based).
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

}  // namespace grout
