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

// Butterfly sum over the wave (x += x of lane ^ off, off = 32 .. 1) on the
// VALU: it ends every GEMV, so two LDS round trips per step were on each
// launch's critical path.
__device__ __forceinline__ float wave_sum(float x) { return wave_xor_sum(x); }

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

// y = W x' (W row-major [rows][K] f16, fp32 accumulation, f16 out).  The
// input x' is produced on the fly (IN):
//   kPlain:   x' = x
//   kNorm:    x' = f16(x * inv * gamma),             inv = 1/rms(x)
//   kAddNorm: c = residual + x (fp32), x' = f16(c * inv * gamma), inv = 1/rms(c);
//             the first wave also stores residual_out = f16(c)
// and the output (OUT):
//   kRows:      y[n] = f16(W[n] . x') for n < N
//   kSiluPairs: W holds 2N rows [gate | up]; y[n] = f16(silu(g) * u) with
//               g = f16(W[n] . x'), u = f16(W[N + n] . x')
// so the decode step's input / post-attention RMSNorms run inside the QKV and
// gate_up GEMVs and SiLU * up in the gate_up epilogue, with the rounding
// points of the separate kernels (src/kernels.rs:1493-1522, 1530-1569,
// 4518-4657).
//
// Work split: a wave owns R weight rows over the whole K; lane l covers
// k = 512c + 8l of chunk c.  The wave first issues its input reads (L2 hits),
// then all R x CH weight reads (16 bytes per lane each, HBM), and only then
// computes: the norm of the input overlaps the weight stream, and every wave
// has its whole share of HBM reads in flight at once.  Partial sums meet in a
// wave reduction; with a plain input the waves are independent (no LDS, no
// barrier), with a norm input the workgroup shares x' through LDS
// (gemv_norm_lds_kernel), and at the long plain K of the larger models
// (16-50 chunks) the waves of a workgroup split one row pair's chunks
// (gemv_splitk_kernel).  The decode
// shapes compile with CH = the exact chunk count, so no branch separates the
// loads (a branch there makes the compiler wait for every outstanding load
// before issuing the next); other K loop over batches of 8 chunks.
enum GemvInMode { kPlain = 0, kNorm = 1, kAddNorm = 2 };
enum GemvOutMode { kRows = 0, kSiluPairs = 1 };

struct GemvArgs {
  const half_t* x;
  const half_t* res;
  const half_t* gamma;
  half_t* res_out;
  float eps;
};

constexpr int kGemvLoopBatch = 8;

__device__ __forceinline__ float silu_mul1(float g, float u) {
  const float sig = 1.0f / (1.0f + expf(-g));
  return sig * g * u;
}

// The wave's weight rows: kRows takes rows row0 .. row0+R-1 (clamped to
// N - 1 for the loads), kSiluPairs rows n and N + n.
template <int R, int OUT>
__device__ __forceinline__ void gemv_rows(const half_t* W, int gwave, int N, int K,
                                          const half_t* (&wrow)[R]) {
  if (OUT == kSiluPairs) {
    wrow[0] = W + (size_t)gwave * K;
    wrow[R - 1] = W + (size_t)(N + gwave) * K;
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = gwave * R + r;
      wrow[r] = W + (size_t)(row < N ? row : N - 1) * K;
    }
  }
}

template <int R, int OUT>
__device__ __forceinline__ void gemv_store(float (&acc)[R], half_t* y, int gwave, int N,
                                           int lane) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  if (OUT == kSiluPairs) {
    if (lane == 0) {
      const half_t g = (half_t)acc[0], u = (half_t)acc[R - 1];
      y[gwave] = (half_t)silu_mul1((float)g, (float)u);
    }
  } else {
    const int row0 = gwave * R;
    if (lane < R && row0 + lane < N) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) v = acc[r];
      y[row0 + lane] = (half_t)v;
    }
  }
}

// Exactly CH chunks (K in (512 (CH - 1), 512 CH]): one pass.
template <int R, int IN, int OUT, int CH>
__device__ __forceinline__ void gemv_exact(const half_t* __restrict__ W, const GemvArgs& a,
                                           half_t* __restrict__ y, int N, int K, int gwave,
                                           int lane) {
  const half_t* wrow[R];
  gemv_rows<R, OUT>(W, gwave, N, K, wrow);
  // 1. input reads
  u32x4 xa[CH], xr[CH], xg[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int k = j * 512 + lane * 8;
    const int kk = k < K ? k : 0;
    xa[j] = load16(a.x + kk);
    if (IN == kAddNorm) xr[j] = load16(a.res + kk);
    if (IN != kPlain) xg[j] = load16(a.gamma + kk);
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. weight reads
  u32x4 wv[CH][R];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int k = j * 512 + lane * 8;
    const int kk = k < K ? k : 0;
#pragma unroll
    for (int r = 0; r < R; ++r) wv[j][r] = load_stream16(wrow[r] + kk);
  }
  __builtin_amdgcn_sched_barrier(0);
  // 3. x' (overlaps the weight reads: they return after the input reads)
  half8 xp[CH];
  if (IN == kPlain) {
#pragma unroll
    for (int j = 0; j < CH; ++j) xp[j] = as_half8(xa[j]);
  } else {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const half8 xh = as_half8(xa[j]);
      const half8 rh = IN == kAddNorm ? as_half8(xr[j]) : half8{};
      half8 co;
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float cv = IN == kAddNorm ? (float)rh[e] + (float)xh[e] : (float)xh[e];
        part += cv * cv;
        co[e] = (half_t)cv;
      }
      const int k = j * 512 + lane * 8;
      ss += k < K ? part : 0.f;
      if (IN == kAddNorm && gwave == 0 && k < K)
        *reinterpret_cast<u32x4*>(a.res_out + k) = as_u32x4(co);
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const half8 xh = as_half8(xa[j]);
      const half8 rh = IN == kAddNorm ? as_half8(xr[j]) : half8{};
      const half8 gh = as_half8(xg[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float cv = IN == kAddNorm ? (float)rh[e] + (float)xh[e] : (float)xh[e];
        xp[j][e] = (half_t)(cv * inv * (float)gh[e]);
      }
    }
  }
  // 4. dot products
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int k = j * 512 + lane * 8;
    const half8 xh = k < K ? xp[j] : half8{};
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = dot8(wv[j][r], xh, acc[r]);
  }
  gemv_store<R, OUT>(acc, y, gwave, N, lane);
}

// Any K: 1/rms in a first pass, then batches of kGemvLoopBatch chunks with
// clamped, always-issued loads.
template <int R, int IN, int OUT>
__device__ __forceinline__ void gemv_loop(const half_t* __restrict__ W, const GemvArgs& a,
                                          half_t* __restrict__ y, int N, int K, int gwave,
                                          int lane) {
  constexpr int B = kGemvLoopBatch;
  const half_t* wrow[R];
  gemv_rows<R, OUT>(W, gwave, N, K, wrow);
  const int nchunks = (K + 511) / 512;
  float inv = 0.f;
  if (IN != kPlain) {
    float ss = 0.f;
    for (int k = lane * 8; k < K; k += 512) {
      const half8 xh = as_half8(load16(a.x + k));
      const half8 rh = IN == kAddNorm ? as_half8(load16(a.res + k)) : half8{};
      half8 co;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float cv = IN == kAddNorm ? (float)rh[e] + (float)xh[e] : (float)xh[e];
        ss += cv * cv;
        co[e] = (half_t)cv;
      }
      if (IN == kAddNorm && gwave == 0) *reinterpret_cast<u32x4*>(a.res_out + k) = as_u32x4(co);
    }
    ss = wave_sum(ss);
    inv = 1.0f / sqrtf(ss / (float)K + a.eps);
  }
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int c0 = 0; c0 < nchunks; c0 += B) {
    u32x4 wv[B][R], xa[B], xr[B], xg[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int c = c0 + j < nchunks ? c0 + j : nchunks - 1;
      const int k = c * 512 + lane * 8;
      const int kk = k < K ? k : 0;
      xa[j] = load16(a.x + kk);
      if (IN == kAddNorm) xr[j] = load16(a.res + kk);
      if (IN != kPlain) xg[j] = load16(a.gamma + kk);
#pragma unroll
      for (int r = 0; r < R; ++r) wv[j][r] = load_stream16(wrow[r] + kk);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int k = (c0 + j) * 512 + lane * 8;
      const bool ok = c0 + j < nchunks && k < K;
      half8 xh = as_half8(xa[j]);
      if (IN != kPlain) {
        const half8 rh = IN == kAddNorm ? as_half8(xr[j]) : half8{};
        const half8 gh = as_half8(xg[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float cv = IN == kAddNorm ? (float)rh[e] + (float)xh[e] : (float)xh[e];
          xh[e] = (half_t)(cv * inv * (float)gh[e]);
        }
      }
      if (!ok) xh = half8{};
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = dot8(wv[j][r], xh, acc[r]);
    }
  }
  gemv_store<R, OUT>(acc, y, gwave, N, lane);
}

// Norm inputs (kNorm / kAddNorm) with exactly CH chunks: the kNormWaves waves
// of a workgroup compute x' once, into LDS, instead of every wave re-reading
// x, residual and gamma and redoing the norm (for two rows per wave that was
// 1.5 input bytes through L1 per weight byte).  Each thread loads its share
// of the inputs, then its wave's R x CH weight reads are issued, so the norm
// (two barriers) overlaps the weight stream as before.  R weight rows per
// wave; kSiluPairs: R / 2 (gate, up) pairs.  Measured on MI355X at the
// Qwen3-4B shapes (HIP events, rotating weights): QKV 6144 x 2560 6.95 vs
// 7.83 us, gate_up 19456 x 2560 16.4 vs 20.9 us.
constexpr int kNormWaves = 4;  // the wave sums below add exactly four partials

template <int R, int IN, int OUT, int CH>
__global__ __launch_bounds__(kNormWaves * 64) void gemv_norm_lds_kernel(
    const half_t* __restrict__ W, GemvArgs a, half_t* __restrict__ y, int N, int K) {
  constexpr int T = kNormWaves * 64;
  constexpr int NV = (CH * 64 + T - 1) / T;  // input vectors (8 halves) per thread
  constexpr int P = OUT == kSiluPairs ? R / 2 : R;  // outputs per wave
  __shared__ __attribute__((aligned(16))) half_t s_x[CH * 512];
  __shared__ float s_ss[kNormWaves];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int gwave = blockIdx.x * kNormWaves + w;
  // weight rows (clamped for the loads; waves past N still join the barriers)
  const half_t* wrow[R];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int o = gwave * P + i;
    const int oc = o < N ? o : N - 1;
    if (OUT == kSiluPairs) {
      wrow[2 * i] = W + (size_t)oc * K;
      wrow[2 * i + 1] = W + (size_t)(N + oc) * K;
    } else {
      wrow[i] = W + (size_t)oc * K;
    }
  }
  // 1. input reads: vector v = threadIdx.x + T i covers k = 8v .. 8v+7
  u32x4 xa[NV], xr[NV], xg[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = threadIdx.x + T * i;
    const int kk = v < CH * 64 && 8 * v < K ? 8 * v : 0;
    xa[i] = load16(a.x + kk);
    if (IN == kAddNorm) xr[i] = load16(a.res + kk);
    xg[i] = load16(a.gamma + kk);
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. weight reads
  u32x4 wv[CH][R];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int k = j * 512 + lane * 8;
    const int kk = k < K ? k : 0;
#pragma unroll
    for (int r = 0; r < R; ++r) wv[j][r] = load_stream16(wrow[r] + kk);
  }
  __builtin_amdgcn_sched_barrier(0);
  // 3. x' into LDS: sum of squares per thread, per wave, then over the waves
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = threadIdx.x + T * i;
    const bool ok = v < CH * 64 && 8 * v < K;
    const half8 xh = as_half8(xa[i]);
    const half8 rh = IN == kAddNorm ? as_half8(xr[i]) : half8{};
    half8 co;
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float cv = IN == kAddNorm ? (float)rh[e] + (float)xh[e] : (float)xh[e];
      part += cv * cv;
      co[e] = (half_t)cv;
    }
    ss += ok ? part : 0.f;
    if (IN == kAddNorm && blockIdx.x == 0 && ok)
      *reinterpret_cast<u32x4*>(a.res_out + 8 * v) = as_u32x4(co);
  }
  ss = wave_sum(ss);
  if (lane == 0) s_ss[w] = ss;
  __syncthreads();
  static_assert(kNormWaves == 4, "fixed summation order of the wave partials");
  ss = (s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]);
  const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = threadIdx.x + T * i;
    if (v < CH * 64) {
      const half8 xh = as_half8(xa[i]);
      const half8 rh = IN == kAddNorm ? as_half8(xr[i]) : half8{};
      const half8 gh = as_half8(xg[i]);
      half8 xp;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float cv = IN == kAddNorm ? (float)rh[e] + (float)xh[e] : (float)xh[e];
        xp[e] = (half_t)(cv * inv * (float)gh[e]);
      }
      if (8 * v >= K) xp = half8{};
      *reinterpret_cast<u32x4*>(&s_x[8 * v]) = as_u32x4(xp);
    }
  }
  __syncthreads();
  // 4. dot products
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const half8 xh = as_half8(*reinterpret_cast<const u32x4*>(&s_x[j * 512 + lane * 8]));
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = dot8(wv[j][r], xh, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  const int o0 = gwave * P;
  if (lane < P && o0 + lane < N) {
    float g = acc[0], u = acc[R > 1 ? 1 : 0];
#pragma unroll
    for (int i = 1; i < P; ++i)
      if (lane == i) {
        g = acc[OUT == kSiluPairs ? 2 * i : i];
        u = acc[OUT == kSiluPairs ? 2 * i + 1 : i];
      }
    if (OUT == kSiluPairs)
      y[o0 + lane] = (half_t)silu_mul1((float)(half_t)g, (float)(half_t)u);
    else
      y[o0 + lane] = (half_t)g;
  }
}

// CH > 0: exactly CH chunks; CH == 0: any K.  N = output rows.  WAVES waves
// per workgroup: one for the layer projections (measured 5-10% faster than
// four on MI355X: finished waves free their CU slot at once), four for the
// 150k-row lm_head (keeps the workgroup count, and dispatch time, bounded).
template <int R, int IN, int OUT, int CH, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(const half_t* __restrict__ W, GemvArgs a,
                                                          half_t* __restrict__ y, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int gwave = blockIdx.x * WAVES + (threadIdx.x >> 6);
  const int outs_per_wave = OUT == kSiluPairs ? 1 : R;
  if (gwave * outs_per_wave >= N) return;  // whole wave
  if (CH > 0)
    gemv_exact<R, IN, OUT, (CH > 0 ? CH : 1)>(W, a, y, N, K, gwave, lane);
  else
    gemv_loop<R, IN, OUT>(W, a, y, N, K, gwave, lane);
}

// Long K, plain input: the W waves of a workgroup share its R rows and split
// the chunks (wave w takes chunks [w CHW, (w + 1) CHW), k < K; input reads,
// then all of its weight reads in flight at once); the waves' row sums meet
// in LDS and are added in wave order.  Measured on MI355X against one wave
// per row (pair) over the whole K (us, rotating weight copies): 5120 x 25600
// 40.2 vs 44.1, 5120 x 17408 27.9 vs 31.3, 4096 x 12288 17.2 vs 17.7, 5120 x
// 8192 14.3 vs 15.2; at 2560 x 9728 and below the one-wave forms stay faster.
template <int R, int CHW, int W>
__global__ __launch_bounds__(W * 64) void gemv_splitk_kernel(const half_t* __restrict__ Wm,
                                                             const half_t* __restrict__ x,
                                                             half_t* __restrict__ y, int N,
                                                             int K) {
  __shared__ float part[W][R];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const half_t* wrow[R];
  gemv_rows<R, kRows>(Wm, blockIdx.x, N, K, wrow);
  u32x4 xa[CHW];
#pragma unroll
  for (int j = 0; j < CHW; ++j) {
    const int k = (w * CHW + j) * 512 + lane * 8;
    xa[j] = load16(x + (k < K ? k : 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 wv[CHW][R];
#pragma unroll
  for (int j = 0; j < CHW; ++j) {
    const int k = (w * CHW + j) * 512 + lane * 8;
#pragma unroll
    for (int r = 0; r < R; ++r) wv[j][r] = load_stream16(wrow[r] + (k < K ? k : 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int j = 0; j < CHW; ++j) {
    const int k = (w * CHW + j) * 512 + lane * 8;
    const half8 xh = k < K ? as_half8(xa[j]) : half8{};
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = dot8(wv[j][r], xh, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = wave_sum(acc[r]);
    if (lane == 0) part[w][r] = acc[r];
  }
  __syncthreads();
  const int row = blockIdx.x * R + lane;
  if (w == 0 && lane < R && row < N) {
    float s = part[0][lane];
#pragma unroll
    for (int i = 1; i < W; ++i) s += part[i][lane];
    y[row] = (half_t)s;
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
template <int OFF>
__device__ __forceinline__ void argmax_step(float& m, uint32_t& i) {
  const float m2 = xor_lane<OFF>(m);
  const uint32_t i2 = xor_lane_u32<OFF>(i);
  argmax_combine(m, i, m2, i2);
}
// The butterfly over the wave (partner = lane ^ off, off = 32 .. 1).
__device__ __forceinline__ void argmax_wave(float& m, uint32_t& i) {
  argmax_step<32>(m, i);
  argmax_step<16>(m, i);
  argmax_step<8>(m, i);
  argmax_step<4>(m, i);
  argmax_step<2>(m, i);
  argmax_step<1>(m, i);
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
                                                           int nblocks, uint32_t* __restrict__ out,
                                                           uint32_t* __restrict__ advance_pos) {
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
    if (advance_pos != nullptr) advance_pos[0] += 1u;
  }
}

// ------------------------------------------------------------- weight cast

// Checkpoint tensors to f16 the way the reference's loader casts them
// (src/loader.rs:702-740): bf16 -> f32 (exact) -> f16, f32 -> f16,
// f64 -> f32 -> f16, each step round to nearest even (v_cvt_f16_f32 in the
// default rounding mode; overflow becomes inf).
__global__ __launch_bounds__(256) void convert_to_f16_kernel(const void* __restrict__ src,
                                                            int dtype, size_t n,
                                                            half_t* __restrict__ dst) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    float f;
    if (dtype == 1) {
      f = __uint_as_float((uint32_t)static_cast<const uint16_t*>(src)[i] << 16);
    } else if (dtype == 2) {
      f = static_cast<const float*>(src)[i];
    } else if (dtype == 3) {
      f = (float)static_cast<const double*>(src)[i];
    } else {
      dst[i] = static_cast<const half_t*>(src)[i];
      continue;
    }
    dst[i] = (half_t)f;
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

template <int R, int IN, int OUT, int CH>
static void gemv_launch(const void* W, const GemvArgs& a, void* y, int N, int K,
                        hipStream_t stream) {
  const int outs = OUT == kSiluPairs ? 1 : R;
  const long waves = (N + outs - 1) / outs;
  if (waves <= 32768) {
    gemv_kernel<R, IN, OUT, CH, 1><<<(unsigned)waves, 64, 0, stream>>>((const half_t*)W, a,
                                                                       (half_t*)y, N, K);
  } else {
    gemv_kernel<R, IN, OUT, CH, 4><<<(unsigned)((waves + 3) / 4), 256, 0, stream>>>(
        (const half_t*)W, a, (half_t*)y, N, K);
  }
}

template <int IN, int OUT>
static hipError_t launch_gemv_mode(const void* W, const GemvArgs& a, void* y, int N, int K,
                                   hipStream_t stream) {
  if (K % 8 != 0 || N < 1 || K < 8) return hipErrorInvalidValue;
  const int nchunks = (K + 511) / 512;
  // kRows: two rows per wave (both rows' loads in flight) when that still
  // gives >= 2048 waves; kSiluPairs: always the (gate, up) pair.
  constexpr int RP = OUT == kSiluPairs ? 2 : 1;
  const bool two = OUT == kSiluPairs || (N + 7) / 8 >= 512;
  // Exact-chunk kernels for the Qwen3 decode shapes: hidden 2560 / 4096 /
  // 5120 (5, 8, 10 chunks), attention width 4096 / 8192 (8, 16), MLP width
  // 9728 / 12288 (19, 24).
  if constexpr (IN != kPlain) {
    // norm inputs: x' shared through LDS; two rows per wave, two (gate, up)
    // pairs per wave at 5 chunks (one pair at 8 and 10: register budget)
    auto lds = [&](auto ch, auto r) {
      constexpr int CH = decltype(ch)::value, R = decltype(r)::value;
      constexpr int P = OUT == kSiluPairs ? R / 2 : R;
      const long waves = (N + P - 1) / P;
      gemv_norm_lds_kernel<R, IN, OUT, CH>
          <<<(unsigned)((waves + kNormWaves - 1) / kNormWaves), kNormWaves * 64, 0, stream>>>(
              (const half_t*)W, a, (half_t*)y, N, K);
      return hipGetLastError();
    };
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    switch (nchunks) {
      case 5:
        if constexpr (OUT == kSiluPairs) return lds(std::integral_constant<int, 5>{}, I4{});
        else return lds(std::integral_constant<int, 5>{}, I2{});
      case 8:
        return lds(std::integral_constant<int, 8>{}, I2{});
      case 10:
        return lds(std::integral_constant<int, 10>{}, I2{});
      default:
        break;
    }
  }
  switch (nchunks) {
    case 5:
      if (two) gemv_launch<2, IN, OUT, 5>(W, a, y, N, K, stream);
      else gemv_launch<1, IN, OUT, 5>(W, a, y, N, K, stream);
      return hipGetLastError();
    case 8:
      if (two) gemv_launch<2, IN, OUT, 8>(W, a, y, N, K, stream);
      else gemv_launch<1, IN, OUT, 8>(W, a, y, N, K, stream);
      return hipGetLastError();
    case 10:
      gemv_launch<RP, IN, OUT, 10>(W, a, y, N, K, stream);
      return hipGetLastError();
    default:
      break;
  }
  // Long K occurs only for plain inputs (attention width, MLP width).
  if constexpr (IN == kPlain && OUT == kRows) {
    auto splitk = [&](auto r, auto chw, auto w) {
      constexpr int R = decltype(r)::value, CHW = decltype(chw)::value,
                    WV = decltype(w)::value;
      static_assert(R >= 1 && CHW >= 1 && WV >= 1, "split-K shape");
      gemv_splitk_kernel<R, CHW, WV><<<(unsigned)((N + R - 1) / R), WV * 64, 0, stream>>>(
          (const half_t*)W, (const half_t*)a.x, (half_t*)y, N, K);
      return hipGetLastError();
    };
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    switch (nchunks) {
      // attention width 8192 (Qwen3-32B o_proj), MLP widths 12288 / 17408 /
      // 25600 (8B / 14B / 32B down): the chunks split over the waves of a
      // workgroup
      case 16:
        return splitk(I2{}, I4{}, I4{});
      case 24:
        return splitk(I2{}, std::integral_constant<int, 6>{}, I4{});
      case 34:
        return splitk(I2{}, std::integral_constant<int, 17>{}, I2{});
      case 50:
        return splitk(I2{}, std::integral_constant<int, 13>{}, I4{});
      // two rows per wave over the whole K at 19 chunks (down 2560 x 9728:
      // 9.5 vs 10.3 us with one row; the split forms measured 9.6-10.6)
      case 19:
        gemv_launch<2, IN, OUT, 19>(W, a, y, N, K, stream);
        return hipGetLastError();
      default:
        break;
    }
  }
  gemv_launch<RP, IN, OUT, 0>(W, a, y, N, K, stream);
  return hipGetLastError();
}

hipError_t launch_gemv(const void* W, const void* x, void* y, int N, int K, hipStream_t stream) {
  const GemvArgs a{(const half_t*)x, nullptr, nullptr, nullptr, 0.f};
  return launch_gemv_mode<kPlain, kRows>(W, a, y, N, K, stream);
}

hipError_t launch_gemv_norm(const void* W, const void* residual, const void* x, const void* gamma,
                            void* residual_out, float eps, void* y, int N, int K, bool silu_pairs,
                            hipStream_t stream) {
  const GemvArgs a{(const half_t*)x, (const half_t*)residual, (const half_t*)gamma,
                   (half_t*)residual_out, eps};
  if (silu_pairs) {
    if (residual) return launch_gemv_mode<kAddNorm, kSiluPairs>(W, a, y, N, K, stream);
    return launch_gemv_mode<kNorm, kSiluPairs>(W, a, y, N, K, stream);
  }
  if (residual) return launch_gemv_mode<kAddNorm, kRows>(W, a, y, N, K, stream);
  return launch_gemv_mode<kNorm, kRows>(W, a, y, N, K, stream);
}

int argmax_num_blocks(int V) { return (V + kArgmaxBlock - 1) / kArgmaxBlock; }

hipError_t launch_convert_to_f16(const void* src, int dtype, size_t n, void* dst,
                                 hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + 255) / 256;
  convert_to_f16_kernel<<<(unsigned)(blocks < 16384 ? blocks : 16384), 256, 0, stream>>>(
      src, dtype, n, (half_t*)dst);
  return hipGetLastError();
}

hipError_t launch_argmax(const void* logits, float* block_max, uint32_t* block_idx, int V,
                         uint32_t* out, hipStream_t stream, uint32_t* advance_pos) {
  const int nb = argmax_num_blocks(V);
  argmax_blocks_kernel<<<nb, 256, 0, stream>>>((const half_t*)logits, block_max, block_idx, V);
  argmax_reduce_kernel<<<1, 256, 0, stream>>>(block_max, block_idx, nb, out, advance_pos);
  return hipGetLastError();
}

}  // namespace grout
