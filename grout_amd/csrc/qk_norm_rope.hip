// Fused per-head QK-RMSNorm + NeoX RoPE + KV-cache write (prefill and decode).
//
// Reference: qk_norm_rope_kv_prefill_raw_f16 (src/kernels.rs:4837-5168) and
// qk_norm_rope_kv_decode_raw_f16 (src/kernels.rs:5170-5452).  Same math:
//   ss = sum(x^2); inv = rsqrt(ss/D + eps); n = x*inv*gamma;
//   y_lo = n_lo*cos - n_hi*sin; y_hi = n_hi*cos + n_lo*sin; f16(y)
// Q rows go to q_out, K rows to k_cache[kvh][pos][:], V rows are copied to
// v_cache[kvh][pos][:].
//
// Layout of the work.  Prefill: one row (one head of one token, D = 128
// halves = 256 B) per 8 lanes, lane i owning elements 8i..8i+7 and their RoPE
// partners 8i+64..8i+71 (two 16-byte loads), 32 rows per 256-thread workgroup
// from the flattened (token, head) order; see norm_rope_row8.  Decode (one
// token): one row per 32 lanes, lane j owning elements 4j..4j+3 (8-byte
// loads), lanes j and j^16 the partners d and d+64, exchanged with
// v_permlane16_swap and DPP row rotations; see norm_rope_row.  Both forms
// reduce the sum of squares in the same pairing order.
//
// Bit-exact K rows: this file is compiled with -ffp-contract=off, the sum of
// squares uses the fixed tree (in-lane (a^2+b^2)+(c^2+d^2), then xor butterfly
// 16,8,4,2,1), 1/sqrt uses a fixed double-precision Newton sequence, and the
// cos/sin come from a host-built fp32 table [max_ctx][D/2], so every step is
// an IEEE-defined operation that a CPU performs identically.
#include "common.hpp"
#include "kernels.hpp"
#include "qk_norm_rope.hpp"

#pragma clang fp contract(off)

namespace grout {

// Decode: grid (1, ceil((Hq+Hkv)/8)): 32-lane group g of the 256-thread
// workgroup takes heads h = 8R*blockIdx.y + g + 8r (r < R) of the token at
// d_pos[0].  The cos/sin row is loaded once per group, every load is issued
// before any row is computed, and the R rows' reduction and Newton chains are
// independent, so they overlap.
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
    const u32x2 yr = norm_rope_row(xr[r], is_q ? gq : gk, c, sn, j, eps);
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

// Prefill: one head row per 8-lane group (norm_rope_row8), 32 rows per
// 256-thread workgroup taken from the flattened (token, head) sequence, so a
// wave covers 8 consecutive heads (2 KiB of contiguous input).  Q rows go to
// q_out; K rows to the cache slot, with their V row copied alongside.  The
// per-row work (the reduction, the fp64 Newton sequence of 1/sqrt) runs once
// per 8 rows of a wave instead of once per 2 with 32 lanes per row.
__global__ __launch_bounds__(256) void qk_norm_rope_kv_prefill8_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k, const half_t* __restrict__ v,
    const half_t* __restrict__ gamma_q, const half_t* __restrict__ gamma_k,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin,
    half_t* __restrict__ q_out, half_t* __restrict__ k_cache, half_t* __restrict__ v_cache,
    int pos0, int rows, int Hq, int Hkv, long head_stride, float eps, long ldq, long ldkv) {
  const int r = (int)blockIdx.x * 32 + (int)(threadIdx.x >> 3);
  if (r >= rows) return;  // uniform across the 8 lanes of a row group
  const int i = threadIdx.x & 7;
  const int H = Hq + Hkv;
  const int s = r / H, h = r - s * H;
  const int pos = pos0 + s;
  const bool is_q = h < Hq;
  const int kvh = h - Hq;
  // all loads first
  // token s's rows start ldq (q) / ldkv (k, v) elements apart
  const half_t* x = is_q ? q + (size_t)s * ldq + (size_t)h * kHeadDim
                         : k + (size_t)s * ldkv + (size_t)kvh * kHeadDim;
  const u32x4 xlo = load16(x + 8 * i), xhi = load16(x + 64 + 8 * i);
  const half_t* gm = is_q ? gamma_q : gamma_k;
  const half8 glo = as_half8(load16(gm + 8 * i)), ghi = as_half8(load16(gm + 64 + 8 * i));
  const float* crow = rope_cos + (size_t)pos * (kHeadDim / 2) + 8 * i;
  const float* srow = rope_sin + (size_t)pos * (kHeadDim / 2) + 8 * i;
  const floatx4 c0 = *reinterpret_cast<const floatx4*>(crow);
  const floatx4 c1 = *reinterpret_cast<const floatx4*>(crow + 4);
  const floatx4 s0 = *reinterpret_cast<const floatx4*>(srow);
  const floatx4 s1 = *reinterpret_cast<const floatx4*>(srow + 4);
  u32x4 vlo = {0u, 0u, 0u, 0u}, vhi = {0u, 0u, 0u, 0u};
  if (!is_q) {
    const half_t* vr = v + (size_t)s * ldkv + (size_t)kvh * kHeadDim;
    vlo = load16(vr + 8 * i);
    vhi = load16(vr + 64 + 8 * i);
  }
  const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  u32x4 ylo, yhi;
  norm_rope_row8(xlo, xhi, glo, ghi, c, sn, eps, ylo, yhi);
  if (is_q) {
    half_t* dst = q_out + ((size_t)s * Hq + h) * kHeadDim;
    *reinterpret_cast<u32x4*>(dst + 8 * i) = ylo;
    *reinterpret_cast<u32x4*>(dst + 64 + 8 * i) = yhi;
  } else {
    const size_t coff = (size_t)kvh * head_stride + (size_t)pos * kHeadDim;
    *reinterpret_cast<u32x4*>(k_cache + coff + 8 * i) = ylo;
    *reinterpret_cast<u32x4*>(k_cache + coff + 64 + 8 * i) = yhi;
    *reinterpret_cast<u32x4*>(v_cache + coff + 8 * i) = vlo;
    *reinterpret_cast<u32x4*>(v_cache + coff + 64 + 8 * i) = vhi;
  }
}

hipError_t launch_qk_norm_rope_kv_prefill(const void* q, const void* k, const void* v,
                                          const void* gamma_q, const void* gamma_k,
                                          const float* rope_cos, const float* rope_sin,
                                          void* q_out, void* k_cache, void* v_cache, int pos0,
                                          int seq_len, int Hq, int Hkv, long head_stride,
                                          int max_ctx, float eps, hipStream_t stream, long ldq,
                                          long ldkv) {
  (void)max_ctx;  // the caller checked pos0 + seq_len <= max_ctx
  const long rows = (long)seq_len * (Hq + Hkv);
  if (rows <= 0 || rows > 0x7fffffffL) return hipErrorInvalidValue;
  if (ldq == 0) ldq = (long)Hq * kHeadDim;
  if (ldkv == 0) ldkv = (long)Hkv * kHeadDim;
  if (ldq < (long)Hq * kHeadDim || ldkv < (long)Hkv * kHeadDim || ldq % 8 || ldkv % 8)
    return hipErrorInvalidValue;
  // 32 rows per 256-thread workgroup measured fastest on MI355X (S=2048, 4B:
  // 8.6-8.7 us; 64/128/512 threads 8.9-9.5 us; two rows per lane group 9.8-10.9 us)
  qk_norm_rope_kv_prefill8_kernel<<<(unsigned)((rows + 31) / 32), 256, 0, stream>>>(
      (const half_t*)q, (const half_t*)k, (const half_t*)v, (const half_t*)gamma_q,
      (const half_t*)gamma_k, rope_cos, rope_sin, (half_t*)q_out, (half_t*)k_cache,
      (half_t*)v_cache, pos0, (int)rows, Hq, Hkv, head_stride, eps, ldq, ldkv);
  return hipGetLastError();
}

hipError_t launch_qk_norm_rope_kv_decode(const void* qkv, const void* gamma_q,
                                         const void* gamma_k, const float* rope_cos,
                                         const float* rope_sin, void* q_out, void* k_cache,
                                         void* v_cache, const uint32_t* d_pos, int Hq, int Hkv,
                                         long head_stride, int max_ctx, float eps,
                                         hipStream_t stream) {
  constexpr int rows = 8 * kRowsPerGroup;  // heads per workgroup
  const dim3 grid(1u, (unsigned)((Hq + Hkv + rows - 1) / rows));
  qk_norm_rope_kv_kernel<true, kRowsPerGroup><<<grid, 256, 0, stream>>>(
      (const half_t*)qkv, nullptr, (const half_t*)qkv, (const half_t*)gamma_q,
      (const half_t*)gamma_k, rope_cos, rope_sin, (half_t*)q_out, (half_t*)k_cache,
      (half_t*)v_cache, d_pos, 0, Hq, Hkv, head_stride, max_ctx, eps);
  return hipGetLastError();
}

}  // namespace grout
