// Fused per-head QK-RMSNorm + NeoX RoPE + KV-cache write (prefill and decode).
//
// Reference: qk_norm_rope_kv_prefill_raw_f16 (src/kernels.rs:4837-5168) and
// qk_norm_rope_kv_decode_raw_f16 (src/kernels.rs:5170-5452).  Same math:
//   ss = sum(x^2); inv = rsqrt(ss/D + eps); n = x*inv*gamma;
//   y_lo = n_lo*cos - n_hi*sin; y_hi = n_hi*cos + n_lo*sin; f16(y)
// Q rows go to q_out, K rows to k_cache[kvh][pos][:], V rows are copied to
// v_cache[kvh][pos][:].
//
// Layout of the work: one row (one head of one token, D = 128 halves = 256 B)
// per 32 lanes; lane j owns elements 4j..4j+3 (one 8-byte load), so a wave
// moves two contiguous rows per instruction.  Lanes j and j^16 hold the RoPE
// partners d and d+64.  Eight row groups per 256-thread workgroup, each taking
// kRowsPerGroup heads of one token; lane exchanges use v_permlane16_swap and
// DPP row rotations (no LDS round trip, no integer division).
//
// Bit-exact K rows: this file is compiled with -ffp-contract=off, the sum of
// squares uses the fixed tree (in-lane (a^2+b^2)+(c^2+d^2), then xor butterfly
// 16,8,4,2,1), 1/sqrt uses a fixed double-precision Newton sequence, and the
// cos/sin come from a host-built fp32 table [max_ctx][D/2], so every step is
// an IEEE-defined operation that a CPU performs identically.
#include "common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace grout {

__device__ __forceinline__ float rsqrt_det(float v) {
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

// Lane exchanges inside one 32-lane row group, on the VALU (no LDS round
// trip): xor16 swaps the two 16-lane halves, ror(N) reads lane (l+N) mod 16 of
// the same half.
__device__ __forceinline__ float xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  // r[0]: odd halves take the even half's value; r[1]: even halves take the odd half's
  return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
template <int N>
__device__ __forceinline__ float ror16(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x120 + N, 0xf, 0xf, false));
}

// Grid (tokens, ceil((Hq+Hkv)/(8R))): 32-lane group g of the 256-thread
// workgroup takes heads h = 8R*blockIdx.y + g + 8r (r < R) of token
// blockIdx.x.  The cos/sin row is loaded once per group, every load is issued
// before any row is computed, and the R rows' reduction and Newton chains are
// independent, so they overlap.  One row per group measured fastest on MI355X
// (S=2048, 4B: 13.4 us at R = 1, 14.3 us at R = 5): more, smaller workgroups
// keep more independent HBM requests in flight.
constexpr int kRowsPerGroup = 1;

template <bool kDecode, int R>
__global__ __launch_bounds__(256) void qk_norm_rope_kv_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k, const half_t* __restrict__ v,
    const half_t* __restrict__ gamma_q, const half_t* __restrict__ gamma_k,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    half_t* __restrict__ q_out, half_t* __restrict__ k_cache, half_t* __restrict__ v_cache,
    const uint32_t* __restrict__ d_pos, int pos0, int Hq, int Hkv, long head_stride,
    int max_ctx, float eps) {
  const int s = blockIdx.x;
  const int h0 = blockIdx.y * 8 * R + (threadIdx.x >> 5);
  const int j = threadIdx.x & 31;
  const int H = Hq + Hkv;
  if (h0 >= H) return;  // uniform across the 32 lanes of a row group
  const int pos = kDecode ? (int)d_pos[0] : pos0 + s;
  if (pos < 0 || pos >= max_ctx) return;  // never write outside the cache

  // All loads first.
  const size_t trow = (size_t)pos * (kHeadDim / 2) + 4 * (j & 15);
  const floatx4 c = *reinterpret_cast<const floatx4*>(rope_cos + trow);
  const floatx4 sn = *reinterpret_cast<const floatx4*>(rope_sin + trow);
  const half4 gq = __builtin_bit_cast(half4, *reinterpret_cast<const u32x2*>(gamma_q + 4 * j));
  const half4 gk = __builtin_bit_cast(half4, *reinterpret_cast<const u32x2*>(gamma_k + 4 * j));
  u32x2 xr[R], vr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int h = h0 + 8 * r;
    xr[r] = u32x2{0u, 0u};
    vr[r] = u32x2{0u, 0u};
    if (h >= H) continue;
    const bool is_q = h < Hq;
    const int kvh = h - Hq;
    const half_t* x;
    if (kDecode) {
      x = q + (size_t)h * kHeadDim;  // qkv = [Q | K | V], K rows follow Q rows
    } else {
      x = is_q ? q + ((size_t)s * Hq + h) * kHeadDim : k + ((size_t)s * Hkv + kvh) * kHeadDim;
    }
    xr[r] = *reinterpret_cast<const u32x2*>(x + 4 * j);
    if (!is_q) {
      const half_t* vrow = kDecode ? v + (size_t)(Hq + Hkv + kvh) * kHeadDim
                                   : v + ((size_t)s * Hkv + kvh) * kHeadDim;
      vr[r] = *reinterpret_cast<const u32x2*>(vrow + 4 * j);
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int h = h0 + 8 * r;
    if (h >= H) continue;  // uniform across the group
    const bool is_q = h < Hq;
    const int kvh = h - Hq;
    const half4 xh = __builtin_bit_cast(half4, xr[r]);
    const float x0 = (float)xh[0], x1 = (float)xh[1], x2 = (float)xh[2], x3 = (float)xh[3];

    // Sum of squares: fixed tree, in-lane (a^2+b^2)+(c^2+d^2) then the
    // butterfly over partners l^16, l^8, l^4, l^2, l^1.  After the l^16 and
    // l^8 steps lanes l and l^8 hold equal values, so the rotation partners
    // (l+-4, l+-2, l+-1 mod 16) add exactly the values the xor partners would.
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

    const half4 gh = is_q ? gq : gk;
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
    const u32x2 yr = __builtin_bit_cast(u32x2, y);
    if (is_q) {
      half_t* dst = kDecode ? q_out + (size_t)h * kHeadDim : q_out + ((size_t)s * Hq + h) * kHeadDim;
      *reinterpret_cast<u32x2*>(dst + 4 * j) = yr;
    } else {
      const size_t coff = (size_t)kvh * head_stride + (size_t)pos * kHeadDim + 4 * j;
      *reinterpret_cast<u32x2*>(k_cache + coff) = yr;
      *reinterpret_cast<u32x2*>(v_cache + coff) = vr[r];
    }
  }
}

hipError_t launch_qk_norm_rope_kv_prefill(const void* q, const void* k, const void* v,
                                          const void* gamma_q, const void* gamma_k,
                                          const float* rope_cos, const float* rope_sin,
                                          void* q_out, void* k_cache, void* v_cache, int pos0,
                                          int seq_len, int Hq, int Hkv, long head_stride,
                                          int max_ctx, float eps, hipStream_t stream) {
  const dim3 grid((unsigned)seq_len, (unsigned)((Hq + Hkv + 8 * kRowsPerGroup - 1) / (8 * kRowsPerGroup)));
  qk_norm_rope_kv_kernel<false, kRowsPerGroup><<<grid, 256, 0, stream>>>(
      (const half_t*)q, (const half_t*)k, (const half_t*)v, (const half_t*)gamma_q,
      (const half_t*)gamma_k, rope_cos, rope_sin, (half_t*)q_out, (half_t*)k_cache,
      (half_t*)v_cache, nullptr, pos0, Hq, Hkv, head_stride, max_ctx, eps);
  return hipGetLastError();
}

hipError_t launch_qk_norm_rope_kv_decode(const void* qkv, const void* gamma_q,
                                         const void* gamma_k, const float* rope_cos,
                                         const float* rope_sin, void* q_out, void* k_cache,
                                         void* v_cache, const uint32_t* d_pos, int Hq, int Hkv,
                                         long head_stride, int max_ctx, float eps,
                                         hipStream_t stream) {
  const dim3 grid(1u, (unsigned)((Hq + Hkv + 7) / 8));
  qk_norm_rope_kv_kernel<true, 1><<<grid, 256, 0, stream>>>(
      (const half_t*)qkv, nullptr, (const half_t*)qkv, (const half_t*)gamma_q,
      (const half_t*)gamma_k, rope_cos, rope_sin, (half_t*)q_out, (half_t*)k_cache,
      (half_t*)v_cache, d_pos, 0, Hq, Hkv, head_stride, max_ctx, eps);
  return hipGetLastError();
}

}  // namespace grout
