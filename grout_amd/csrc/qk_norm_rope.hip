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
// partners d and d+64.  Eight rows per 256-thread workgroup.
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

template <bool kDecode>
__global__ __launch_bounds__(256) void qk_norm_rope_kv_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k, const half_t* __restrict__ v,
    const half_t* __restrict__ gamma_q, const half_t* __restrict__ gamma_k,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    half_t* __restrict__ q_out, half_t* __restrict__ k_cache, half_t* __restrict__ v_cache,
    const uint32_t* __restrict__ d_pos, int pos0, int seq_len, int Hq, int Hkv,
    long head_stride, int max_ctx, float eps) {
  const int H = Hq + Hkv;
  const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int j = threadIdx.x & 31;
  if (row >= seq_len * H) return;  // uniform across the 32 lanes of a row
  const int s = row / H;
  const int h = row - s * H;
  const int pos = kDecode ? (int)d_pos[0] : pos0 + s;
  if (pos < 0 || pos >= max_ctx) return;  // never write outside the cache
  const bool is_q = h < Hq;
  const int kvh = h - Hq;

  const half_t* x;
  if (kDecode) {
    x = q + (size_t)h * kHeadDim;  // qkv = [Q | K | V], K rows follow Q rows
  } else {
    x = is_q ? q + ((size_t)s * Hq + h) * kHeadDim : k + ((size_t)s * Hkv + kvh) * kHeadDim;
  }
  const u32x2 xr = *reinterpret_cast<const u32x2*>(x + 4 * j);
  const half4 xh = __builtin_bit_cast(half4, xr);
  const float x0 = (float)xh[0], x1 = (float)xh[1], x2 = (float)xh[2], x3 = (float)xh[3];

  // Sum of squares: fixed tree.
  float a0 = x0 * x0, a1 = x1 * x1, a2 = x2 * x2, a3 = x3 * x3;
  float s0 = a0 + a1, s1 = a2 + a3;
  float ss = s0 + s1;
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) ss = ss + __shfl_xor(ss, off, 64);
  const float mean = ss / (float)kHeadDim;
  const float inv = rsqrt_det(mean + eps);

  const half_t* g = is_q ? gamma_q : gamma_k;
  const half4 gh = __builtin_bit_cast(half4, *reinterpret_cast<const u32x2*>(g + 4 * j));
  float n[4];
  n[0] = (x0 * inv) * (float)gh[0];
  n[1] = (x1 * inv) * (float)gh[1];
  n[2] = (x2 * inv) * (float)gh[2];
  n[3] = (x3 * inv) * (float)gh[3];
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = __shfl_xor(n[i], 16, 64);  // RoPE partner (d +/- 64)

  const size_t trow = (size_t)pos * (kHeadDim / 2) + 4 * (j & 15);
  const floatx4 c = *reinterpret_cast<const floatx4*>(rope_cos + trow);
  const floatx4 sn = *reinterpret_cast<const floatx4*>(rope_sin + trow);
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
    const half_t* vrow = kDecode ? v + (size_t)(Hq + Hkv + kvh) * kHeadDim
                                 : v + ((size_t)s * Hkv + kvh) * kHeadDim;
    *reinterpret_cast<u32x2*>(v_cache + coff) = *reinterpret_cast<const u32x2*>(vrow + 4 * j);
  }
}

hipError_t launch_qk_norm_rope_kv_prefill(const void* q, const void* k, const void* v,
                                          const void* gamma_q, const void* gamma_k,
                                          const float* rope_cos, const float* rope_sin,
                                          void* q_out, void* k_cache, void* v_cache, int pos0,
                                          int seq_len, int Hq, int Hkv, long head_stride,
                                          int max_ctx, float eps, hipStream_t stream) {
  const long rows = (long)seq_len * (Hq + Hkv);
  const unsigned blocks = (unsigned)((rows + 7) / 8);
  qk_norm_rope_kv_kernel<false><<<blocks, 256, 0, stream>>>(
      (const half_t*)q, (const half_t*)k, (const half_t*)v, (const half_t*)gamma_q,
      (const half_t*)gamma_k, rope_cos, rope_sin, (half_t*)q_out, (half_t*)k_cache,
      (half_t*)v_cache, nullptr, pos0, seq_len, Hq, Hkv, head_stride, max_ctx, eps);
  return hipGetLastError();
}

hipError_t launch_qk_norm_rope_kv_decode(const void* qkv, const void* gamma_q,
                                         const void* gamma_k, const float* rope_cos,
                                         const float* rope_sin, void* q_out, void* k_cache,
                                         void* v_cache, const uint32_t* d_pos, int Hq, int Hkv,
                                         long head_stride, int max_ctx, float eps,
                                         hipStream_t stream) {
  const unsigned blocks = (unsigned)((Hq + Hkv + 7) / 8);
  qk_norm_rope_kv_kernel<true><<<blocks, 256, 0, stream>>>(
      (const half_t*)qkv, nullptr, (const half_t*)qkv, (const half_t*)gamma_q,
      (const half_t*)gamma_k, rope_cos, rope_sin, (half_t*)q_out, (half_t*)k_cache,
      (half_t*)v_cache, d_pos, 0, 1, Hq, Hkv, head_stride, max_ctx, eps);
  return hipGetLastError();
}

}  // namespace grout
