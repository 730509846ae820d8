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

// x of lane (lane ^ OFF), i.e. __shfl_xor(x, OFF) over the 64-lane wave, on
// the VALU instead of an LDS round trip (ds_bpermute): across 16-lane rows
// with v_permlane32/16_swap (each lane keeps the one of the two results
// that came from its partner), within a row with DPP: row_ror:8 is xor 8,
// the row half-mirror (i -> 7 - i in each 8 lanes) followed by the quad
// reversal (i -> 3 - i in each 4) is xor 4, quad_perm [2,3,0,1] and
// [1,0,3,2] are xor 2 and xor 1.  Every lane reads the same partner as with
// the shuffle, so reductions built on it give the same bits.  All 64 lanes
// must be active.
template <int OFF>
__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t x) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32,
                "xor offsets 1..32");
  if constexpr (OFF == 32 || OFF == 16) {
    const auto a = OFF == 32 ? __builtin_amdgcn_permlane32_swap(x, x, false, false)
                             : __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (__lane_id() & OFF) ? a[0] : a[1];
  } else if constexpr (OFF == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);
  } else if constexpr (OFF == 4) {
    const int hm = __builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false);
    return (uint32_t)__builtin_amdgcn_update_dpp(0, hm, 0x1B, 0xF, 0xF, false);
  } else {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, OFF == 2 ? 0x4E : 0xB1, 0xF, 0xF,
                                                 false);
  }
}
template <int OFF>
__device__ __forceinline__ float xor_lane(float x) {
  return __uint_as_float(xor_lane_u32<OFF>(__float_as_uint(x)));
}
// Sum over the wave in the butterfly order of x += __shfl_xor(x, off), off =
// 32, 16, ..., 1 (the same bits).
__device__ __forceinline__ float wave_xor_sum(float x) {
  x += xor_lane<32>(x);
  x += xor_lane<16>(x);
  x += xor_lane<8>(x);
  x += xor_lane<4>(x);
  x += xor_lane<2>(x);
  x += xor_lane<1>(x);
  return x;
}


}  // namespace grout
