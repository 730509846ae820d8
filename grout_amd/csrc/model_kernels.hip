// Kernels of the Qwen3 decode/prefill step around the attention path:
// embedding gather, RMSNorm (plain and fused residual add), SiLU * up, the
// decode GEMV (f16 weights, fp32 accumulation) and the two-stage greedy
// argmax.
//
// Reference: embedding_f16 / embedding_batch_f16 (src/kernels.rs:1893-1938),
// rms_norm_f16 (1530-1569), add_rms_norm_decode_raw_f16 (4518-4657),
// silu_mul_2d_f16 (1493-1522), argmax_blocks_f16 and
// argmax_reduce_blocks_to_u32 (1571-1740); the decode GEMVs are cuBLAS in the
// reference (src/cublas.rs:434-570).  Same math:
//   rms_norm:      out = f16(x * rsqrt(sum(x^2)/N + eps) * w)
//   add_rms_norm:  c = residual + x (fp32); out = f16(c * rsqrt(sum(c^2)/N + eps) * w);
//                  residual_out = f16(c)
//   silu_mul:      out = f16(g * sigmoid(g) * u)
//   argmax:        largest logit, ties to the smallest index.
#include "common.hpp"
#include "kernels.hpp"

namespace grout {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// acc + <w, x> over 8 halves with v_dot2_f32_f16 (fp32 accumulation).
__device__ __forceinline__ float dot8(u32x4 w, half8 x, float acc) {
  const half8 wh = as_half8(w);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 0, 1),
                               __builtin_shufflevector(x, x, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 2, 3),
                               __builtin_shufflevector(x, x, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 4, 5),
                               __builtin_shufflevector(x, x, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 6, 7),
                               __builtin_shufflevector(x, x, 6, 7), acc, false);
  return acc;
}

// ------------------------------------------------------------- embedding

// out[s][:] = table[ids[s]][:]; ids past the vocabulary give a zero row (the
// host API rejects them before they get here).
__global__ __launch_bounds__(256) void embedding_kernel(const uint32_t* __restrict__ ids,
                                                       const half_t* __restrict__ table,
                                                       half_t* __restrict__ out, int H, int vocab) {
  const int s = blockIdx.x;
  const uint32_t id = ids[s];
  const int nvec = H / 8;
  for (int i = threadIdx.x; i < nvec; i += blockDim.x) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (id < (uint32_t)vocab) v = load16(table + (size_t)id * H + 8 * i);
    *reinterpret_cast<u32x4*>(out + (size_t)s * H + 8 * i) = v;
  }
}

// ------------------------------------------------------------- RMSNorm

// One 256-thread workgroup per row; H a multiple of 8.
template <bool kAdd>
__global__ __launch_bounds__(256) void rms_norm_kernel(const half_t* __restrict__ residual,
                                                      const half_t* __restrict__ x,
                                                      const half_t* __restrict__ w,
                                                      half_t* __restrict__ out,
                                                      half_t* __restrict__ residual_out, int H,
                                                      float eps) {
  __shared__ float s_part[4];
  const size_t row = blockIdx.x;
  const int nvec = H / 8;
  constexpr int kMaxVec = 4;  // up to 4 x 8 x 256 = 8192 elements per row held in registers
  float c[kMaxVec][8];
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < kMaxVec; ++it) {
    const int i = threadIdx.x + it * 256;
    if (i < nvec) {
      const half8 xv = as_half8(load16(x + row * H + 8 * i));
      half8 rv = {};
      if (kAdd) rv = as_half8(load16(residual + row * H + 8 * i));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        c[it][e] = kAdd ? (float)rv[e] + (float)xv[e] : (float)xv[e];
        ss += c[it][e] * c[it][e];
      }
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
  const float inv = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
  for (int it = 0; it < kMaxVec; ++it) {
    const int i = threadIdx.x + it * 256;
    if (i < nvec) {
      const half8 wv = as_half8(load16(w + 8 * i));
      half8 o, r;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o[e] = (half_t)(c[it][e] * inv * (float)wv[e]);
        r[e] = (half_t)c[it][e];
      }
      *reinterpret_cast<u32x4*>(out + row * H + 8 * i) = as_u32x4(o);
      if (kAdd) *reinterpret_cast<u32x4*>(residual_out + row * H + 8 * i) = as_u32x4(r);
    }
  }
}

// ------------------------------------------------------------- SiLU * up

// gate_up rows are [gate (I) | up (I)]; out rows are I wide.
__global__ __launch_bounds__(256) void silu_mul_kernel(const half_t* __restrict__ gate_up,
                                                      half_t* __restrict__ out, int I,
                                                      long total_vec) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total_vec) return;
  const int nvec = I / 8;
  const long row = i / nvec;
  const int v = (int)(i - row * nvec);
  const half8 g = as_half8(load16(gate_up + row * 2 * I + 8 * v));
  const half8 u = as_half8(load16(gate_up + row * 2 * I + I + 8 * v));
  half8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gf = (float)g[e];
    const float sig = 1.0f / (1.0f + expf(-gf));
    o[e] = (half_t)(sig * gf * (float)u[e]);
  }
  *reinterpret_cast<u32x4*>(out + row * I + 8 * v) = as_u32x4(o);
}

// ------------------------------------------------------------- GEMV

// y[n] = sum_k W[n][k] x[k] (W row-major [N][K] f16, fp32 accumulation, f16
// out).  A 256-thread workgroup owns kGemvRows rows; its 4 waves split K in
// steps of 512 elements (wave w takes steps w, w+4, ...), each lane reads 16
// bytes of every row per step, partial sums meet in LDS.  K a multiple of 8.
constexpr int kGemvRows = 4;

__global__ __launch_bounds__(256) void gemv_kernel(const half_t* __restrict__ W,
                                                  const half_t* __restrict__ x,
                                                  half_t* __restrict__ y, int N, int K) {
  __shared__ float s_part[4][kGemvRows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * kGemvRows;
  const int nsteps = (K + 511) / 512;
  float acc[kGemvRows];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r) acc[r] = 0.f;
  for (int t = wave; t < nsteps; t += 4) {
    const int k = t * 512 + lane * 8;
    if (k < K) {
      const half8 xv = as_half8(load16(x + k));
      u32x4 wv[kGemvRows];
#pragma unroll
      for (int r = 0; r < kGemvRows; ++r)
        wv[r] = n0 + r < N ? load_stream16(W + (size_t)(n0 + r) * K + k) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int r = 0; r < kGemvRows; ++r) acc[r] = dot8(wv[r], xv, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r) {
    const float s = wave_sum(acc[r]);
    if (lane == 0) s_part[wave][r] = s;
  }
  __syncthreads();
  if (threadIdx.x < kGemvRows && n0 + (int)threadIdx.x < N) {
    const int r = threadIdx.x;
    const float s = (s_part[0][r] + s_part[1][r]) + (s_part[2][r] + s_part[3][r]);
    y[n0 + r] = (half_t)s;
  }
}

// ------------------------------------------------------------- argmax

constexpr int kArgmaxBlock = 2048;  // logits per first-stage workgroup (256 x 8)

__device__ __forceinline__ void argmax_combine(float& m, uint32_t& i, float m2, uint32_t i2) {
  if (m2 > m || (m2 == m && i2 < i)) {
    m = m2;
    i = i2;
  }
}
__device__ __forceinline__ void argmax_wave(float& m, uint32_t& i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const uint32_t i2 = (uint32_t)__shfl_xor((int)i, off, 64);
    argmax_combine(m, i, m2, i2);
  }
}

__global__ __launch_bounds__(256) void argmax_blocks_kernel(const half_t* __restrict__ logits,
                                                           float* __restrict__ block_max,
                                                           uint32_t* __restrict__ block_idx,
                                                           int V) {
  __shared__ float s_m[4];
  __shared__ uint32_t s_i[4];
  const long base = (long)blockIdx.x * kArgmaxBlock + threadIdx.x * 8;
  float m = -3.0e38f;
  uint32_t idx = 0xffffffffu;
  if (base + 8 <= V) {
    const half8 v = as_half8(load16(logits + base));
#pragma unroll
    for (int e = 0; e < 8; ++e) argmax_combine(m, idx, (float)v[e], (uint32_t)(base + e));
  } else {
    for (int e = 0; e < 8; ++e)
      if (base + e < V) argmax_combine(m, idx, (float)logits[base + e], (uint32_t)(base + e));
  }
  argmax_wave(m, idx);
  if ((threadIdx.x & 63) == 0) {
    s_m[threadIdx.x >> 6] = m;
    s_i[threadIdx.x >> 6] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) argmax_combine(m, idx, s_m[w], s_i[w]);
    block_max[blockIdx.x] = m;
    block_idx[blockIdx.x] = idx;
  }
}

__global__ __launch_bounds__(256) void argmax_reduce_kernel(const float* __restrict__ block_max,
                                                           const uint32_t* __restrict__ block_idx,
                                                           int nblocks, uint32_t* __restrict__ out) {
  __shared__ float s_m[4];
  __shared__ uint32_t s_i[4];
  float m = -3.0e38f;
  uint32_t idx = 0xffffffffu;
  for (int b = threadIdx.x; b < nblocks; b += 256) argmax_combine(m, idx, block_max[b], block_idx[b]);
  argmax_wave(m, idx);
  if ((threadIdx.x & 63) == 0) {
    s_m[threadIdx.x >> 6] = m;
    s_i[threadIdx.x >> 6] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) argmax_combine(m, idx, s_m[w], s_i[w]);
    out[0] = idx;
  }
}

// ------------------------------------------------------------- launchers

hipError_t launch_embedding(const uint32_t* ids, const void* table, void* out, int rows, int H,
                            int vocab, hipStream_t stream) {
  embedding_kernel<<<rows, 256, 0, stream>>>(ids, (const half_t*)table, (half_t*)out, H, vocab);
  return hipGetLastError();
}

hipError_t launch_rms_norm(const void* residual, const void* x, const void* w, void* out,
                           void* residual_out, int rows, int H, float eps, hipStream_t stream) {
  if (H % 8 != 0 || H > 8192) return hipErrorInvalidValue;
  if (residual)
    rms_norm_kernel<true><<<rows, 256, 0, stream>>>((const half_t*)residual, (const half_t*)x,
                                                    (const half_t*)w, (half_t*)out,
                                                    (half_t*)residual_out, H, eps);
  else
    rms_norm_kernel<false><<<rows, 256, 0, stream>>>(nullptr, (const half_t*)x, (const half_t*)w,
                                                     (half_t*)out, nullptr, H, eps);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const void* gate_up, void* out, int rows, int I, hipStream_t stream) {
  if (I % 8 != 0) return hipErrorInvalidValue;
  const long total = (long)rows * (I / 8);
  silu_mul_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>((const half_t*)gate_up,
                                                                      (half_t*)out, I, total);
  return hipGetLastError();
}

hipError_t launch_gemv(const void* W, const void* x, void* y, int N, int K, hipStream_t stream) {
  if (K % 8 != 0) return hipErrorInvalidValue;
  gemv_kernel<<<(unsigned)((N + kGemvRows - 1) / kGemvRows), 256, 0, stream>>>(
      (const half_t*)W, (const half_t*)x, (half_t*)y, N, K);
  return hipGetLastError();
}

int argmax_num_blocks(int V) { return (V + kArgmaxBlock - 1) / kArgmaxBlock; }

hipError_t launch_argmax(const void* logits, float* block_max, uint32_t* block_idx, int V,
                         uint32_t* out, hipStream_t stream) {
  const int nb = argmax_num_blocks(V);
  argmax_blocks_kernel<<<nb, 256, 0, stream>>>((const half_t*)logits, block_max, block_idx, V);
  argmax_reduce_kernel<<<1, 256, 0, stream>>>(block_max, block_idx, nb, out);
  return hipGetLastError();
}

}  // namespace grout
