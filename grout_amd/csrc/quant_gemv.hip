// Low-bit decode GEMVs over ggml-quantized weights (Q8_0, Q4_K, Q6_K).
//
// Reference: gemv_q8_0_f16 / gemv_q4k_f16 / gemv_q6k_f16 and their SoA
// variants (src/kernels.rs:259-428, 564-804) over the weights GGUF files hold
// (dequantization rules: src/dequant.rs:211-335).  Same math: every weight
// is dequantized in fp32 from its block (Q8_0: d*q; Q4_K: d*sc*q - dmin*m;
// Q6_K: d*sc*(q-32)), multiplied by the fp16 input and accumulated in fp32;
// the output row is rounded to f16.
//
// GPU layout (grout_qweight_repack): the ggml blocks are split into aligned
// arrays, bytes unchanged, so every dequantized value is the reference's and
// HBM traffic stays at the native bits per weight:
//   Q8_0: q  int8 [N][K]          d  f16 [N][K/32]
//   Q4_K: q  u8   [N][K/2] (each superblock's 128 qs bytes in ggml order)
//         h  16 B [N][K/256] (d, dmin, the 12 packed 6-bit scale/min bytes)
//   Q6_K: ql u8 [N][K/2], qh u8 [N][K/4], sc int8 [N][K/16], d f16 [N][K/256]
//
// Kernel: a 256-thread workgroup owns 16 weight rows (for SiLU pairs: 8 gate
// rows and their 8 up rows) and stages x in LDS.  The rows are cut into
// 16-byte pieces of the primary payload (Q8_0: 16 weights; Q4_K / Q6_K: 32
// weights as two runs of 16) and the threads take pieces round robin; each
// thread issues all weight loads of a batch before it consumes any.  A run of
// 16 quantized values becomes exact f16 integers (byte | 0x6400 is the f16
// 1024 + byte), its dot product with x uses v_dot2_f32_f16, and the run's
// scale (and min) is applied once: scale * sum(q x) - min * sum(x).  Partial
// sums go to LDS per piece and each row is summed in a fixed order, so the
// result does not depend on scheduling.
#include "common.hpp"
#include "kernels.hpp"

namespace grout {

constexpr int kQRows = 16;        // weight rows per workgroup
constexpr int kQThreads = 256;
constexpr int kQBatch = 8;        // pieces per thread issued before any is consumed
constexpr int kQMaxK = 16384;     // x staged in LDS (at most 32 KiB)
constexpr int kQMaxPieces = 16 * 1024;  // kQRows x pieces per row (at most 64 KiB of fp32)

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__host__ __device__ inline size_t qalign(size_t b) { return (b + 255) / 256 * 256; }

// Byte offsets of the repacked arrays of an [n][k] matrix and its total size.
struct QLayout {
  size_t off[4];
  size_t total;
};
__host__ __device__ inline QLayout qlayout(int fmt, size_t n, size_t k) {
  QLayout L{};
  size_t sz[4] = {0, 0, 0, 0};
  if (fmt == 8) {
    sz[0] = n * k;
    sz[1] = n * (k / 32) * 2;
  } else if (fmt == 12) {
    sz[0] = n * k / 2;
    sz[1] = n * (k / 256) * 16;
  } else if (fmt == 14) {
    sz[0] = n * k / 2;
    sz[1] = n * k / 4;
    sz[2] = n * k / 16;
    sz[3] = n * (k / 256) * 2;
  }
  size_t o = 0;
  for (int i = 0; i < 4; ++i) {
    L.off[i] = o;
    o += qalign(sz[i]);
  }
  L.total = o;
  return L;
}

// ---------------------------------------------------------------- repack

// One thread per ggml block.
__global__ __launch_bounds__(256) void qrepack_kernel(int fmt, const uint8_t* __restrict__ src,
                                                     size_t nblocks, int blocks_per_row, int k,
                                                     uint8_t* __restrict__ dst, QLayout L) {
  const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const size_t row = b / blocks_per_row, j = b % blocks_per_row;
  if (fmt == 8) {
    const uint8_t* s = src + b * 34;
    uint8_t* q = dst + L.off[0] + row * k + j * 32;
    for (int i = 0; i < 32; ++i) q[i] = s[2 + i];
    uint8_t* d = dst + L.off[1] + (row * blocks_per_row + j) * 2;
    d[0] = s[0];
    d[1] = s[1];
  } else if (fmt == 12) {
    const uint8_t* s = src + b * 144;
    uint8_t* q = dst + L.off[0] + row * (k / 2) + j * 128;
    for (int i = 0; i < 128; ++i) q[i] = s[16 + i];
    uint8_t* h = dst + L.off[1] + (row * blocks_per_row + j) * 16;
    for (int i = 0; i < 16; ++i) h[i] = s[i];
  } else {
    const uint8_t* s = src + b * 210;
    uint8_t* ql = dst + L.off[0] + row * (k / 2) + j * 128;
    uint8_t* qh = dst + L.off[1] + row * (k / 4) + j * 64;
    uint8_t* sc = dst + L.off[2] + row * (k / 16) + j * 16;
    uint8_t* d = dst + L.off[3] + (row * blocks_per_row + j) * 2;
    for (int i = 0; i < 128; ++i) ql[i] = s[i];
    for (int i = 0; i < 64; ++i) qh[i] = s[128 + i];
    for (int i = 0; i < 16; ++i) sc[i] = s[192 + i];
    d[0] = s[208];
    d[1] = s[209];
  }
}

// ---------------------------------------------------------------- piece decode

// Four bytes (each an integer 0..255) -> two f16 pairs holding (1024 + byte);
// `bias` is subtracted exactly (1024 for unsigned values, 1152 for int8 that
// were offset by 128, 1056 for 6-bit values stored with +32).
__device__ __forceinline__ void bytes_to_f16(uint32_t v, half2v bias, half2v& lo, half2v& hi) {
  const uint32_t a = (v & 0xFFu) | ((v & 0xFF00u) << 8) | 0x64006400u;
  const uint32_t b = ((v >> 16) & 0xFFu) | ((v >> 8) & 0xFF0000u) | 0x64006400u;
  lo = __builtin_bit_cast(half2v, a) - bias;
  hi = __builtin_bit_cast(half2v, b) - bias;
}

// sum over 16 values: q (4 words of 4 bytes, bias removed) . x (16 f16)
__device__ __forceinline__ float dot16(const uint32_t (&w)[4], half2v bias, const half8& x0,
                                       const half8& x1, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    half2v lo, hi;
    bytes_to_f16(w[i], bias, lo, hi);
    const half8& xs = i < 2 ? x0 : x1;
    const int e = (i & 1) * 4;
    acc = __builtin_amdgcn_fdot2(lo, half2v{xs[e], xs[e + 1]}, acc, false);
    acc = __builtin_amdgcn_fdot2(hi, half2v{xs[e + 2], xs[e + 3]}, acc, false);
  }
  return acc;
}

__device__ __forceinline__ float sum16(const half8& x0, const half8& x1) {
  const half2v one = {(half_t)1.0f, (half_t)1.0f};
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    s = __builtin_amdgcn_fdot2(half2v{x0[e], x0[e + 1]}, one, s, false);
    s = __builtin_amdgcn_fdot2(half2v{x1[e], x1[e + 1]}, one, s, false);
  }
  return s;
}

__device__ __forceinline__ float h2f_bits(uint16_t b) { return (float)__builtin_bit_cast(half_t, b); }

// Raw bytes of one piece (row, j).
struct QRaw {
  u32x4 a;  // primary payload: Q8_0 q, Q4_K q, Q6_K ql
  u32x4 b;  // Q6_K: the 16 qh bytes of the piece's runs
};

template <int FMT>
__device__ __forceinline__ QRaw qload(const uint8_t* __restrict__ W, const QLayout& L, int row,
                                      int j, int K) {
  QRaw r;
  if (FMT == 8) {
    r.a = load_stream16(W + L.off[0] + (size_t)row * K + (size_t)j * 16);
  } else if (FMT == 12) {
    r.a = load_stream16(W + L.off[0] + (size_t)row * (K / 2) + (size_t)j * 16);
  } else {
    r.a = load_stream16(W + L.off[0] + (size_t)row * (K / 2) + (size_t)j * 16);
    const int sb = j >> 3, o = (j & 7) * 16, n = o >> 6, h = o & 63;
    r.b = load_stream16(W + L.off[1] + (size_t)row * (K / 4) + sb * 64 + 32 * n + (h & 31));
  }
  return r;
}

// Contribution of piece j of `row` with its raw bytes, x staged in LDS.
template <int FMT>
__device__ __forceinline__ float qpiece(const QRaw& r, const uint8_t* __restrict__ W,
                                        const QLayout& L, int row, int j, int K,
                                        const half_t* __restrict__ xs) {
  if (FMT == 8) {
    // 16 int8 weights k = 16j .. 16j+15, block j/2
    const half8 x0 = *reinterpret_cast<const half8*>(xs + 16 * j);
    const half8 x1 = *reinterpret_cast<const half8*>(xs + 16 * j + 8);
    uint32_t w[4] = {r.a[0] ^ 0x80808080u, r.a[1] ^ 0x80808080u, r.a[2] ^ 0x80808080u,
                     r.a[3] ^ 0x80808080u};
    const half2v bias = {(half_t)1152.0f, (half_t)1152.0f};
    const float dot = dot16(w, bias, x0, x1, 0.f);
    const uint16_t db = *reinterpret_cast<const uint16_t*>(W + L.off[1] +
                                                           ((size_t)row * (K / 32) + (j >> 1)) * 2);
    return h2f_bits(db) * dot;
  } else if (FMT == 12) {
    const int sb = j >> 3, g = (j & 7) >> 1, l0 = (j & 1) * 16;
    const int e0 = sb * 256 + 64 * g + l0;
    const half8 xl0 = *reinterpret_cast<const half8*>(xs + e0);
    const half8 xl1 = *reinterpret_cast<const half8*>(xs + e0 + 8);
    const half8 xh0 = *reinterpret_cast<const half8*>(xs + e0 + 32);
    const half8 xh1 = *reinterpret_cast<const half8*>(xs + e0 + 40);
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = r.a[i] & 0x0F0F0F0Fu;
      hi[i] = (r.a[i] >> 4) & 0x0F0F0F0Fu;
    }
    const half2v bias = {(half_t)1024.0f, (half_t)1024.0f};
    const float dlo = dot16(lo, bias, xl0, xl1, 0.f);
    const float dhi = dot16(hi, bias, xh0, xh1, 0.f);
    // header: d, dmin, then the packed 6-bit (scale, min) of sub-blocks 2g, 2g+1
    const uint8_t* hb = W + L.off[1] + ((size_t)row * (K / 256) + sb) * 16;
    const u32x4 hv = *reinterpret_cast<const u32x4*>(hb);
    const uint8_t* sc = reinterpret_cast<const uint8_t*>(&hv) + 4;
    const float d = h2f_bits((uint16_t)(hv[0] & 0xFFFF)), dmin = h2f_bits((uint16_t)(hv[0] >> 16));
    int s1, m1, s2, m2;
    const int j1 = 2 * g, j2 = 2 * g + 1;
    if (j1 < 4) {
      s1 = sc[j1] & 63;
      m1 = sc[j1 + 4] & 63;
    } else {
      s1 = (sc[j1 + 4] & 0xF) | ((sc[j1 - 4] >> 6) << 4);
      m1 = (sc[j1 + 4] >> 4) | ((sc[j1] >> 6) << 4);
    }
    if (j2 < 4) {
      s2 = sc[j2] & 63;
      m2 = sc[j2 + 4] & 63;
    } else {
      s2 = (sc[j2 + 4] & 0xF) | ((sc[j2 - 4] >> 6) << 4);
      m2 = (sc[j2 + 4] >> 4) | ((sc[j2] >> 6) << 4);
    }
    const float d1 = d * (float)s1, mn1 = dmin * (float)m1;
    const float d2 = d * (float)s2, mn2 = dmin * (float)m2;
    return (d1 * dlo - mn1 * sum16(xl0, xl1)) + (d2 * dhi - mn2 * sum16(xh0, xh1));
  } else {
    const int sb = j >> 3, o = (j & 7) * 16, n = o >> 6, h = o & 63;
    const int base = sb * 256 + 128 * n + (h & 31);
    // h < 32: runs i = 0 (ql low, qh bits 0-1) and i = 2 (ql high, bits 4-5);
    // h >= 32: runs i = 1 (bits 2-3) and i = 3 (bits 6-7)
    const int ilo = h < 32 ? 0 : 1, ihi = ilo + 2;
    const int e_lo = base + 32 * ilo, e_hi = base + 32 * ihi;
    const half8 xl0 = *reinterpret_cast<const half8*>(xs + e_lo);
    const half8 xl1 = *reinterpret_cast<const half8*>(xs + e_lo + 8);
    const half8 xh0 = *reinterpret_cast<const half8*>(xs + e_hi);
    const half8 xh1 = *reinterpret_cast<const half8*>(xs + e_hi + 8);
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = (r.a[i] & 0x0F0F0F0Fu) | (((r.b[i] >> (2 * ilo)) & 0x03030303u) << 4);
      hi[i] = ((r.a[i] >> 4) & 0x0F0F0F0Fu) | (((r.b[i] >> (2 * ihi)) & 0x03030303u) << 4);
    }
    const half2v bias = {(half_t)1056.0f, (half_t)1056.0f};  // 1024 + 32: q - 32
    const float dlo = dot16(lo, bias, xl0, xl1, 0.f);
    const float dhi = dot16(hi, bias, xh0, xh1, 0.f);
    const int8_t* scp = reinterpret_cast<const int8_t*>(W + L.off[2] + (size_t)row * (K / 16));
    const float d = h2f_bits(
        *reinterpret_cast<const uint16_t*>(W + L.off[3] + ((size_t)row * (K / 256) + sb) * 2));
    const float s_lo = d * (float)scp[(e_lo - 0) / 16];
    const float s_hi = d * (float)scp[(e_hi - 0) / 16];
    return s_lo * dlo + s_hi * dhi;
  }
}

// ---------------------------------------------------------------- GEMV

// SILU: rows are 8 gate rows g0.. and their up rows N + g0.. (N = outputs);
// otherwise 16 consecutive rows.  pieces per row P = K / (FMT == 8 ? 16 : 32).
template <int FMT, bool SILU>
__global__ __launch_bounds__(kQThreads) void gemv_q_kernel(const uint8_t* __restrict__ W,
                                                          const half_t* __restrict__ x,
                                                          half_t* __restrict__ y, int N, int K,
                                                          QLayout L) {
  // Dynamic LDS: x (K halves), then one fp32 partial per piece (kQRows x P).
  extern __shared__ __attribute__((aligned(16))) unsigned char s_dyn[];
  half_t* const s_x = reinterpret_cast<half_t*>(s_dyn);
  float* const s_part = reinterpret_cast<float*>(s_dyn + (size_t)K * 2);
  const int tid = threadIdx.x;
  const int P = K / (FMT == 8 ? 16 : 32);
  const int total = kQRows * P;
  const int out0 = blockIdx.x * (SILU ? kQRows / 2 : kQRows);
  // Local row lr -> weight row (clamped to a valid row; its output is dropped).
  auto row_of = [&](int lr) __attribute__((always_inline)) {
    if (SILU) {
      const int o = min(out0 + (lr & (kQRows / 2 - 1)), N - 1);
      return lr < kQRows / 2 ? o : N + o;
    }
    return min(out0 + lr, N - 1);
  };

  // First batch of weight loads, then x into LDS.
  QRaw raw[kQBatch];
  auto issue = [&](int p0) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < kQBatch; ++b) {
      int p = p0 + b * kQThreads;
      p = p < total ? p : total - 1;  // clamped; the consumer skips it
      raw[b] = qload<FMT>(W, L, row_of(p / P), p % P, K);
    }
  };
  issue(tid);
  __builtin_amdgcn_sched_barrier(0);
  for (int i = tid * 8; i < K; i += kQThreads * 8)
    *reinterpret_cast<u32x4*>(s_x + i) = load16(x + i);
  __syncthreads();

  for (int p0 = tid;; p0 += kQBatch * kQThreads) {
#pragma unroll
    for (int b = 0; b < kQBatch; ++b) {
      const int p = p0 + b * kQThreads;
      if (p < total) s_part[p] = qpiece<FMT>(raw[b], W, L, row_of(p / P), p % P, K, s_x);
    }
    if (p0 + kQBatch * kQThreads >= total) break;
    issue(p0 + kQBatch * kQThreads);
  }
  __syncthreads();

  // Row sums in a fixed order: 16 threads per row, each a strided partial,
  // then a butterfly over the 16.
  const int lr = tid >> 4, sub = tid & 15;
  float s = 0.f;
  for (int q = sub; q < P; q += 16) s += s_part[lr * P + q];
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) s += __shfl_xor(s, off, 16);
  if (SILU) {
    // lanes of gate row lr (< 8) and its up row lr + 8 sit 128 threads apart:
    // pass the up sums through LDS
    __syncthreads();
    if (sub == 0 && lr >= kQRows / 2) s_part[lr - kQRows / 2] = s;
    __syncthreads();
    if (sub == 0 && lr < kQRows / 2 && out0 + lr < N) {
      const half_t g = (half_t)s, u = (half_t)s_part[lr];
      const float gf = (float)g;
      const float sig = 1.0f / (1.0f + expf(-gf));
      y[out0 + lr] = (half_t)(sig * gf * (float)u);
    }
  } else if (sub == 0 && out0 + lr < N) {
    y[out0 + lr] = (half_t)s;
  }
}

// ---------------------------------------------------------------- dequant to f16

// f16 of p rounded to nearest even, with p's sign.  Rounding keeps the sign,
// so the OR changes nothing in exact arithmetic; it is there because the
// compiler folds a product followed by this rounding into a mixed-precision
// fma with a +0 addend, which turns a -0 product into +0.
__device__ __forceinline__ half_t f2h_signed(float p) {
  const uint16_t h = __builtin_bit_cast(uint16_t, (half_t)p);
  return __builtin_bit_cast(half_t,
                            (uint16_t)(h | ((__builtin_bit_cast(uint32_t, p) >> 16) & 0x8000u)));
}

// w[row][k] as f16 (for the prefill GEMMs): one thread per 16-byte piece.
template <int FMT>
__global__ __launch_bounds__(256) void qdequant_kernel(const uint8_t* __restrict__ W, int N,
                                                      int K, QLayout L, half_t* __restrict__ out) {
  // Each weight is fp32 arithmetic in the reference's order (no fused
  // multiply-add), rounded once to f16.
#pragma clang fp contract(off)
  const int P = K / (FMT == 8 ? 16 : 32);
  const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= (size_t)N * P) return;
  const int row = (int)(p / P), j = (int)(p % P);
  const QRaw r = qload<FMT>(W, L, row, j, K);
  half_t* o = out + (size_t)row * K;
  if (FMT == 8) {
    const float d = h2f_bits(*reinterpret_cast<const uint16_t*>(W + L.off[1] +
                                                                 ((size_t)row * (K / 32) + (j >> 1)) * 2));
    const int8_t* q = reinterpret_cast<const int8_t*>(&r.a);
    for (int i = 0; i < 16; ++i) o[16 * j + i] = f2h_signed((float)q[i] * d);
  } else if (FMT == 12) {
    const int sb = j >> 3, g = (j & 7) >> 1, l0 = (j & 1) * 16;
    const uint8_t* hb = W + L.off[1] + ((size_t)row * (K / 256) + sb) * 16;
    const float d = h2f_bits((uint16_t)(hb[0] | (hb[1] << 8)));
    const float dmin = h2f_bits((uint16_t)(hb[2] | (hb[3] << 8)));
    const uint8_t* sc = hb + 4;
    int s[2], m[2];
    for (int t = 0; t < 2; ++t) {
      const int jj = 2 * g + t;
      if (jj < 4) {
        s[t] = sc[jj] & 63;
        m[t] = sc[jj + 4] & 63;
      } else {
        s[t] = (sc[jj + 4] & 0xF) | ((sc[jj - 4] >> 6) << 4);
        m[t] = (sc[jj + 4] >> 4) | ((sc[jj] >> 6) << 4);
      }
    }
    const float d1 = d * (float)s[0], m1 = dmin * (float)m[0];
    const float d2 = d * (float)s[1], m2 = dmin * (float)m[1];
    const uint8_t* q = reinterpret_cast<const uint8_t*>(&r.a);
    const int e0 = sb * 256 + 64 * g + l0;
    for (int i = 0; i < 16; ++i) {
      o[e0 + i] = f2h_signed(d1 * (float)(q[i] & 0xF) - m1);
      o[e0 + 32 + i] = f2h_signed(d2 * (float)(q[i] >> 4) - m2);
    }
  } else {
    const int sb = j >> 3, o16 = (j & 7) * 16, n = o16 >> 6, h = o16 & 63;
    const int ilo = h < 32 ? 0 : 1, ihi = ilo + 2;
    const int base = sb * 256 + 128 * n + (h & 31);
    const float d = h2f_bits(
        *reinterpret_cast<const uint16_t*>(W + L.off[3] + ((size_t)row * (K / 256) + sb) * 2));
    const int8_t* scp = reinterpret_cast<const int8_t*>(W + L.off[2] + (size_t)row * (K / 16));
    const uint8_t* ql = reinterpret_cast<const uint8_t*>(&r.a);
    const uint8_t* qh = reinterpret_cast<const uint8_t*>(&r.b);
    const int e_lo = base + 32 * ilo, e_hi = base + 32 * ihi;
    const float slo = d * (float)scp[e_lo / 16], shi = d * (float)scp[e_hi / 16];
    for (int i = 0; i < 16; ++i) {
      const int qlo = (int)((ql[i] & 0xF) | (((qh[i] >> (2 * ilo)) & 3) << 4)) - 32;
      const int qhi = (int)((ql[i] >> 4) | (((qh[i] >> (2 * ihi)) & 3) << 4)) - 32;
      o[e_lo + i] = f2h_signed(slo * (float)qlo);
      o[e_hi + i] = f2h_signed(shi * (float)qhi);
    }
  }
}

// ---------------------------------------------------------------- launchers

static bool qfmt_ok(int fmt, int N, int K) {
  if (N < 1 || K < 1) return false;
  const int blk = fmt == 8 ? 32 : 256;
  if (fmt != 8 && fmt != 12 && fmt != 14) return false;
  if (K % blk != 0 || K > kQMaxK) return false;
  const int P = K / (fmt == 8 ? 16 : 32);
  return (long)kQRows * P <= kQMaxPieces;
}

size_t qweight_bytes(int fmt, int N, int K) {
  if (!qfmt_ok(fmt, N, K)) return 0;
  return qlayout(fmt, (size_t)N, (size_t)K).total;
}

hipError_t launch_qweight_repack(int fmt, const void* src, int N, int K, void* dst,
                                 hipStream_t stream) {
  if (!qfmt_ok(fmt, N, K)) return hipErrorInvalidValue;
  const int blk = fmt == 8 ? 32 : 256;
  const size_t nblocks = (size_t)N * (K / blk);
  const QLayout L = qlayout(fmt, (size_t)N, (size_t)K);
  qrepack_kernel<<<(unsigned)((nblocks + 255) / 256), 256, 0, stream>>>(
      fmt, (const uint8_t*)src, nblocks, K / blk, K, (uint8_t*)dst, L);
  return hipGetLastError();
}

template <int FMT>
static void gemv_q_launch(const void* W, const void* x, void* y, int N, int K, bool silu,
                          hipStream_t stream) {
  const QLayout L = qlayout(FMT, (size_t)(silu ? 2 * N : N), (size_t)K);
  const size_t lds = (size_t)K * 2 + (size_t)kQRows * (K / (FMT == 8 ? 16 : 32)) * 4;
  if (silu)
    gemv_q_kernel<FMT, true><<<(unsigned)((N + kQRows / 2 - 1) / (kQRows / 2)), kQThreads, lds,
                                stream>>>((const uint8_t*)W, (const half_t*)x, (half_t*)y, N, K, L);
  else
    gemv_q_kernel<FMT, false><<<(unsigned)((N + kQRows - 1) / kQRows), kQThreads, lds, stream>>>(
        (const uint8_t*)W, (const half_t*)x, (half_t*)y, N, K, L);
}

hipError_t launch_gemv_q(int fmt, const void* W, const void* x, void* y, int N, int K, bool silu,
                         hipStream_t stream) {
  if (!qfmt_ok(fmt, silu ? 2 * N : N, K)) return hipErrorInvalidValue;
  switch (fmt) {
    case 8: gemv_q_launch<8>(W, x, y, N, K, silu, stream); break;
    case 12: gemv_q_launch<12>(W, x, y, N, K, silu, stream); break;
    default: gemv_q_launch<14>(W, x, y, N, K, silu, stream); break;
  }
  return hipGetLastError();
}

hipError_t launch_qweight_dequant(int fmt, const void* W, int N, int K, void* out,
                                  hipStream_t stream) {
  if (!qfmt_ok(fmt, N, K)) return hipErrorInvalidValue;
  const QLayout L = qlayout(fmt, (size_t)N, (size_t)K);
  const size_t pieces = (size_t)N * (K / (fmt == 8 ? 16 : 32));
  const unsigned blocks = (unsigned)((pieces + 255) / 256);
  switch (fmt) {
    case 8: qdequant_kernel<8><<<blocks, 256, 0, stream>>>((const uint8_t*)W, N, K, L, (half_t*)out); break;
    case 12: qdequant_kernel<12><<<blocks, 256, 0, stream>>>((const uint8_t*)W, N, K, L, (half_t*)out); break;
    default: qdequant_kernel<14><<<blocks, 256, 0, stream>>>((const uint8_t*)W, N, K, L, (half_t*)out); break;
  }
  return hipGetLastError();
}

}  // namespace grout
