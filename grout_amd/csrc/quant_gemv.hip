// Low-bit decode GEMVs over ggml-quantized weights (Q8_0, Q4_K, Q5_K, Q6_K).
//
// Reference: gemv_q8_0_f16 / gemv_q4k_f16 / gemv_q5k_f16 / gemv_q6k_f16 and
// their SoA variants (src/kernels.rs:259-804) over the weights GGUF files hold
// (dequantization rules: src/dequant.rs:211-335).  Same math: every weight
// is dequantized in fp32 from its block (Q8_0: d*q; Q4_K: d*sc*q - dmin*m;
// Q5_K: the same with a fifth bit of q; Q6_K: d*sc*(q-32)), multiplied by the
// fp16 input and accumulated in fp32; the output row is rounded to f16.
//
// GPU layout (grout_qweight_repack): the ggml blocks are split into aligned
// arrays, bytes unchanged, so every dequantized value is the reference's and
// HBM traffic stays at the native bits per weight:
//   Q8_0: q  int8 [N][K]          d  f16 [N][K/32]
//   Q4_K: q  u8   [N][K/2] (each superblock's 128 qs bytes in ggml order)
//         h  16 B [N][K/256] (d, dmin, the 12 packed 6-bit scale/min bytes)
//   Q5_K: q and h as Q4_K, qh u8 [N][K/8] (each superblock's 32 qh bytes)
//   Q6_K: ql u8 [N][K/2], qh u8 [N][K/4], sc int8 [N][K/16], d f16 [N][K/256]
//
// GEMV kernel: one 16-lane team per weight row, x and the rows' decoded
// block scales staged in LDS (swizzled against bank conflicts), the weights
// streamed with every load of a lane in flight before its first use.  A run
// of 16 quantized values becomes exact f16 integers (v_perm inserts 0x64, the
// exponent byte of 1024, above each byte; a packed subtract removes 1024 plus
// the format's offset), its dot product with x uses v_dot2_f32_f16, and the
// run's scale (and min) is applied once: scale * sum(q x) - min * sum(x).
#include "common.hpp"
#include "kernels.hpp"

#include <atomic>

namespace grout {

constexpr int kQMaxK = 32768;  // x staged in LDS (at most 64 KiB): every Qwen3 K up to
                               // 32B's ffn_down (25600); the 4-row workgroup then needs
                               // <= 107 KiB of LDS (gfx950: 160 KiB per workgroup)

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
  } else if (fmt == 12 || fmt == 13) {
    sz[0] = n * k / 2;
    sz[1] = n * (k / 256) * 16;
    if (fmt == 13) sz[2] = n * k / 8;
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
  } else if (fmt == 13) {
    // d, dmin, scales[12] at 0, qh[32] at 16, qs[128] at 48
    const uint8_t* s = src + b * 176;
    uint8_t* q = dst + L.off[0] + row * (k / 2) + j * 128;
    for (int i = 0; i < 128; ++i) q[i] = s[48 + i];
    uint8_t* h = dst + L.off[1] + (row * blocks_per_row + j) * 16;
    for (int i = 0; i < 16; ++i) h[i] = s[i];
    uint8_t* qh = dst + L.off[2] + row * (k / 8) + j * 32;
    for (int i = 0; i < 32; ++i) qh[i] = s[16 + i];
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

// ---------------------------------------------------------------- GEMV
//
// A row team of 16 lanes owns one weight row; lane m takes the row's pieces
// p = m, m + 16, ... (a piece is 32 consecutive weights: Q8_0 one block;
// Q4_K 16 qs bytes = 16 weights of sub-block 2g in the low nibbles and 16 of
// 2g+1 in the high; Q5_K the same and the 16 qh bytes holding their fifth
// bits; Q6_K 16 ql bytes and the 16 qh bytes they pair with), so a
// team reads 256 contiguous bytes per load and p % 8 == m % 8 fixes each
// lane's place inside a superblock.  Workgroups of R teams (4 for short
// matrices so the grid covers every CU, 16 for tall ones); before the
// barrier a workgroup stages x and its rows' decoded block scales in LDS,
// with those loads issued ahead of the weight loads.  Each lane sums its
// pieces in order and the team reduces with a fixed butterfly, so results do
// not depend on scheduling.

constexpr int kQTeam = 16;  // lanes per weight row

__device__ __forceinline__ float h2f_bits(uint16_t b) { return (float)__builtin_bit_cast(half_t, b); }

// f16 of p rounded to nearest even, with p's sign.  Rounding keeps the sign,
// so the OR changes nothing in exact arithmetic; it is there because the
// compiler folds a product followed by this rounding into a mixed-precision
// fma with a +0 addend, which turns a -0 product into +0.
__device__ __forceinline__ half_t f2h_signed(float p) {
  const uint16_t h = __builtin_bit_cast(uint16_t, (half_t)p);
  return __builtin_bit_cast(half_t,
                            (uint16_t)(h | ((__builtin_bit_cast(uint32_t, p) >> 16) & 0x8000u)));
}

// LDS granule (8 halves of x) for logical granule G.  Lane m of a team reads
// granules whose bits 1-5 are functions of m; the map moves the lane-varying
// bits onto bits 0-3 so any 8 or 16 lanes of a team hit distinct bank
// groups.  Linear over GF(2), confined to aligned runs of 16 granules and
// blind to bits 6 and up: xswz(G + 64 i) = xswz(G) + 64 i.
template <int FMT>
__host__ __device__ constexpr int xswz(int G) {
  return FMT == 8                  ? G ^ ((G >> 3) & 3) ^ (((G >> 5) & 1) << 3)
         : FMT == 12 || FMT == 13 ? G ^ ((G >> 3) & 1) ^ (((G >> 4) & 1) << 2) ^ (((G >> 5) & 1) << 3)
                                  : G ^ ((G >> 4) & 1) ^ (((G >> 5) & 1) << 3);
}

// Slot of 16-run r in the Q4_K and Q5_K x sums (runs r and r + 2 of one piece side by
// side) and in the Q6_K scales and x sums (runs r and r + 4 side by side).
__host__ __device__ constexpr int xsum_slot(int r) { return (r & ~3) | ((r & 1) << 1) | ((r >> 1) & 1); }
__host__ __device__ constexpr int q6_slot(int r) { return (r & ~7) | ((r & 3) << 1) | ((r >> 2) & 1); }

// Weight row of local row lr and the output it feeds.  SILU: in each wave the
// teams are gate rows o, o+1 then the up rows o, o+1 (up row = N + o).
template <bool SILU, int R>
__device__ __forceinline__ int qrow(int lr, int N, int& out) {
  if (SILU) {
    const int t = lr & 3;
    out = (int)blockIdx.x * (R / 2) + 2 * (lr >> 2) + (t & 1);
    const int o = min(out, N - 1);
    return t < 2 ? o : N + o;
  }
  out = (int)blockIdx.x * R + lr;
  return min(out, N - 1);
}

// Raw bytes of one piece.
struct QPc {
  u32x4 a;  // Q8_0 q[0..15]; Q4_K, Q5_K qs; Q6_K ql
  u32x4 b;  // Q8_0 q[16..31]; Q5_K, Q6_K qh
};

template <int FMT>
__device__ __forceinline__ QPc qpc_load(const uint8_t* __restrict__ W, const QLayout& L, int row,
                                        int p, int K) {
  QPc r;
  if (FMT == 8) {
    const uint8_t* q = W + L.off[0] + (size_t)row * K + (size_t)p * 32;
    r.a = load_stream16(q);
    r.b = load_stream16(q + 16);
  } else if (FMT == 12) {
    r.a = load_stream16(W + L.off[0] + (size_t)row * (K / 2) + (size_t)p * 16);
    r.b = r.a;
  } else if (FMT == 13) {
    r.a = load_stream16(W + L.off[0] + (size_t)row * (K / 2) + (size_t)p * 16);
    // qh bytes 16 l0 .. +15 of superblock p / 8 (l0 = bit 0 of p)
    r.b = load_stream16(W + L.off[2] + (size_t)row * (K / 8) + (size_t)(p >> 3) * 32 + (p & 1) * 16);
  } else {
    r.a = load_stream16(W + L.off[0] + (size_t)row * (K / 2) + (size_t)p * 16);
    // qh bytes 32n + 16 l0 .. +15 of superblock p / 8 (n = bit 2 of p, l0 = bit 0)
    r.b = load_stream16(W + L.off[1] + (size_t)row * (K / 4) + (size_t)(p >> 3) * 64 +
                        ((p >> 2) & 1) * 32 + (p & 1) * 16);
  }
  return r;
}

// Two bytes of v as an f16 pair of denormals, byte * 2^-24 (exact; v_perm
// selector 0x0C is a zero byte): sel 0x0C010C00 takes bytes 0, 1 and
// 0x0C030C02 bytes 2, 3.
__device__ __forceinline__ half2v dpair(uint32_t v, uint32_t sel) {
  return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(v, v, sel));
}

// acc + 2^-24 * sum_t byte_t * x_t over the 16 little-endian bytes of w and
// x0 (t < 8), x1: products of f16 values are exact in the fp32 accumulation.
__device__ __forceinline__ float ddot16(const uint32_t (&w)[4], half8 x0, half8 x1, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const half8& xs = i < 2 ? x0 : x1;
    const int e = (i & 1) * 4;
    acc = __builtin_amdgcn_fdot2(dpair(w[i], 0x0C010C00u), half2v{xs[e], xs[e + 1]}, acc, false);
    acc = __builtin_amdgcn_fdot2(dpair(w[i], 0x0C030C02u), half2v{xs[e + 2], xs[e + 3]}, acc,
                                 false);
  }
  return acc;
}

// Per-lane LDS offsets for piece i = 0 (piece i adds 64 i granules, and 16 i
// (Q8_0) or 32 i (Q4_K, Q5_K, Q6_K) floats of scales and x sums).
struct QLane {
  int xg[4];  // byte offsets of the x granules: Q8_0 4 of one run; else lo, lo+1, hi, hi+1
  int so;     // float offset into the row's scales
  int xo;     // float offset into the x sums
};

template <int FMT>
__device__ __forceinline__ QLane qlane(int m) {
  QLane q;
  if (FMT == 8) {
#pragma unroll
    for (int k = 0; k < 4; ++k) q.xg[k] = 16 * xswz<FMT>(4 * m + k);
    q.so = q.xo = m;
  } else if (FMT == 12 || FMT == 13) {
    // lo run: weights 256 sb + 64 g + 16 l0 (sub-block 2g), hi run +32 (2g+1)
    const int g = (m >> 1) & 3, l0 = m & 1, s3 = m >> 3;
    const int G = 32 * s3 + 8 * g + 2 * l0;
    q.xg[0] = 16 * xswz<FMT>(G);
    q.xg[1] = 16 * xswz<FMT>(G + 1);
    q.xg[2] = 16 * xswz<FMT>(G + 4);
    q.xg[3] = 16 * xswz<FMT>(G + 5);
    q.so = 16 * s3 + 4 * g;
    q.xo = 16 * s3 + 4 * g + 2 * l0;
  } else {
    // lo run: weights 256 sb + 128 n + 32 ilo + 16 l0 (qh bits 2 ilo), hi run
    // +64 (qh bits 2 ilo + 4)
    const int n = (m >> 2) & 1, ilo = (m >> 1) & 1, l0 = m & 1, s3 = m >> 3;
    const int G = 32 * s3 + 16 * n + 4 * ilo + 2 * l0;
    q.xg[0] = 16 * xswz<FMT>(G);
    q.xg[1] = 16 * xswz<FMT>(G + 1);
    q.xg[2] = 16 * xswz<FMT>(G + 8);
    q.xg[3] = 16 * xswz<FMT>(G + 9);
    q.so = q.xo = q6_slot(16 * s3 + 8 * n + 2 * ilo + l0);
  }
  return q;
}

template <int I>
__device__ __forceinline__ half8 xgran(const unsigned char* s_xb, int off) {
  return *reinterpret_cast<const half8*>(s_xb + off + 1024 * I);
}

// Contribution of piece i of lane m (piece index p = m + 16 i) to the row's
// dot product.  Staged scales carry the 2^24 of the denormal encoding.
template <int FMT, int I>
__device__ __forceinline__ float qpc_dot(const QPc& r, int m, const QLane& q,
                                         const unsigned char* s_xb, const float* s_xsum,
                                         const float* s_row) {
  if (FMT == 8) {
    // bytes hold q + 128: sum (q + 128) x - 128 sum x
    const uint32_t wa[4] = {r.a[0] ^ 0x80808080u, r.a[1] ^ 0x80808080u, r.a[2] ^ 0x80808080u,
                            r.a[3] ^ 0x80808080u};
    const uint32_t wb[4] = {r.b[0] ^ 0x80808080u, r.b[1] ^ 0x80808080u, r.b[2] ^ 0x80808080u,
                            r.b[3] ^ 0x80808080u};
    const float da = ddot16(wa, xgran<I>(s_xb, q.xg[0]), xgran<I>(s_xb, q.xg[1]), 0.f);
    const float db = ddot16(wb, xgran<I>(s_xb, q.xg[2]), xgran<I>(s_xb, q.xg[3]), 0.f);
    return s_row[q.so + 16 * I] * ((da + db) - s_xsum[q.xo + 16 * I]);
  } else if (FMT == 12) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = r.a[i] & 0x0F0F0F0Fu;
      hi[i] = r.a[i] & 0xF0F0F0F0u;  // 16 x the high nibble
    }
    const float dlo = ddot16(lo, xgran<I>(s_xb, q.xg[0]), xgran<I>(s_xb, q.xg[1]), 0.f);
    const float dhi = ddot16(hi, xgran<I>(s_xb, q.xg[2]), xgran<I>(s_xb, q.xg[3]), 0.f);
    // {2^24 d sc_2g, dmin m_2g, 2^20 d sc_2g+1, dmin m_2g+1}
    const floatx4 sc = *reinterpret_cast<const floatx4*>(s_row + q.so + 32 * I);
    const float2 xs = *reinterpret_cast<const float2*>(s_xsum + q.xo + 32 * I);
    return (sc[0] * dlo - sc[1] * xs.x) + (sc[2] * dhi - sc[3] * xs.y);
  } else if (FMT == 13) {
    // fifth bits: bit 2g of qh byte l for the lo run, bit 2g + 1 for the hi
    const int g = (m >> 1) & 3;
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t t = r.b[i] >> (2 * g);
      lo[i] = (r.a[i] & 0x0F0F0F0Fu) | ((t << 4) & 0x10101010u);
      hi[i] = ((r.a[i] >> 4) & 0x0F0F0F0Fu) | ((t << 3) & 0x10101010u);
    }
    const float dlo = ddot16(lo, xgran<I>(s_xb, q.xg[0]), xgran<I>(s_xb, q.xg[1]), 0.f);
    const float dhi = ddot16(hi, xgran<I>(s_xb, q.xg[2]), xgran<I>(s_xb, q.xg[3]), 0.f);
    // {2^24 d sc_2g, dmin m_2g, 2^24 d sc_2g+1, dmin m_2g+1}
    const floatx4 sc = *reinterpret_cast<const floatx4*>(s_row + q.so + 32 * I);
    const float2 xs = *reinterpret_cast<const float2*>(s_xsum + q.xo + 32 * I);
    return (sc[0] * dlo - sc[1] * xs.x) + (sc[2] * dhi - sc[3] * xs.y);
  } else {
    // 6-bit q held + 32: sum (q + 32) x - 32 sum x per run
    const int ilo = (m >> 1) & 1;
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = (r.a[i] & 0x0F0F0F0Fu) | ((r.b[i] << (4 - 2 * ilo)) & 0x30303030u);
      hi[i] = ((r.a[i] >> 4) & 0x0F0F0F0Fu) | ((r.b[i] >> (2 * ilo)) & 0x30303030u);
    }
    const float dlo = ddot16(lo, xgran<I>(s_xb, q.xg[0]), xgran<I>(s_xb, q.xg[1]), 0.f);
    const float dhi = ddot16(hi, xgran<I>(s_xb, q.xg[2]), xgran<I>(s_xb, q.xg[3]), 0.f);
    const float2 s = *reinterpret_cast<const float2*>(s_row + q.so + 32 * I);
    const float2 xs = *reinterpret_cast<const float2*>(s_xsum + q.xo + 32 * I);
    return s.x * (dlo - xs.x) + s.y * (dhi - xs.y);
  }
}

// Staging of x: granule c to its swizzled slot, and the x sum of each run
// (Q8_0: 32-runs = granules c..c+3, scaled by 128 * 2^-24; Q4_K, Q5_K: 16-runs;
// Q6_K: 16-runs scaled by 32 * 2^-24), the run's granules sitting in
// adjacent lanes.  Every lane calls it.
template <int FMT>
__device__ __forceinline__ void stage_x(u32x4 v, int c, int NG, half_t* s_x, float* s_xsum) {
  const half8 h = as_half8(v);
  const half2v one = {(half_t)1.0f, (half_t)1.0f};
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; e += 2) s = __builtin_amdgcn_fdot2(half2v{h[e], h[e + 1]}, one, s, false);
  s += xor_lane<1>(s);
  if (FMT == 8) {
    s += xor_lane<2>(s);
    if (c < NG && (c & 3) == 0) s_xsum[c >> 2] = s * 0x1p-17f;
  } else if (FMT == 12 || FMT == 13) {
    if (c < NG && (c & 1) == 0) s_xsum[xsum_slot(c >> 1)] = s;
  } else {
    if (c < NG && (c & 1) == 0) s_xsum[q6_slot(c >> 1)] = s * 0x1p-19f;
  }
  if (c < NG) *reinterpret_cast<u32x4*>(s_x + 8 * xswz<FMT>(c)) = v;
}

// One staging unit: Q8_0 one block scale; Q4_K, Q5_K one superblock header; Q6_K
// one superblock's 16 scales and d.
struct SRaw {
  u32x4 v;
  uint32_t d;
};

// u / UPR without an integer division (one in front of the staging loads
// would delay every load issued after them): for u < R * UPR <= 2^15,
// (u + 1/2) / UPR lies at least 1/(2 UPR) >= 2^-11 from an integer, and the
// product with the hardware reciprocal (1 ulp) is within 2^-17 of it.
__device__ __forceinline__ int unit_row(int u, float inv_upr) {
  return (int)(((float)u + 0.5f) * inv_upr);
}

template <int FMT, bool SILU, int R>
__device__ __forceinline__ SRaw stage_load(const uint8_t* __restrict__ W, const QLayout& L, int u,
                                           int UPR, float inv_upr, int N, int K) {
  const int lr = unit_row(u, inv_upr), k = u - lr * UPR;
  int o;
  const int row = qrow<SILU, R>(lr, N, o);
  SRaw s;
  s.v = u32x4{0u, 0u, 0u, 0u};
  s.d = 0;
  if (FMT == 8) {
    s.d = *reinterpret_cast<const uint16_t*>(W + L.off[1] + ((size_t)row * (K / 32) + k) * 2);
  } else if (FMT == 12 || FMT == 13) {
    s.v = load16(W + L.off[1] + ((size_t)row * (K / 256) + k) * 16);
  } else {
    s.v = load16(W + L.off[2] + (size_t)row * (K / 16) + (size_t)k * 16);
    s.d = *reinterpret_cast<const uint16_t*>(W + L.off[3] + ((size_t)row * (K / 256) + k) * 2);
  }
  return s;
}

// Scales as the reference's decode layout holds them (Q8_0 d; Q6_K d * sc in
// fp32; Q4_K the effective f16(d * sc) and f16(dmin * m); Q5_K, read in the
// native layout, d * sc and dmin * m in fp32), times the power of two that
// undoes the denormal encoding (exact).
template <int FMT>
__device__ __forceinline__ void stage_store(const SRaw& s, int u, int U, int UPR, float inv_upr,
                                            int SCW, float* s_sc) {
  if (u >= U) return;
  const int lr = unit_row(u, inv_upr), k = u - lr * UPR;
  float* dst = s_sc + lr * SCW;
  if (FMT == 8) {
    dst[k] = h2f_bits((uint16_t)s.d) * 0x1p24f;
  } else if (FMT == 12 || FMT == 13) {
    // d, dmin, then eight 6-bit (scale, min) pairs packed in 12 bytes
    const float d = h2f_bits((uint16_t)(s.v[0] & 0xFFFFu));
    const float dmin = h2f_bits((uint16_t)(s.v[0] >> 16));
    int q[12];
#pragma unroll
    for (int j = 0; j < 12; ++j) q[j] = (s.v[1 + j / 4] >> (8 * (j % 4))) & 0xFF;
    int sc[8], mn[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < 4) {
        sc[j] = q[j] & 63;
        mn[j] = q[j + 4] & 63;
      } else {
        sc[j] = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        mn[j] = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
      }
    }
    if (FMT == 12) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<floatx4*>(dst + 16 * k + 4 * g) =
            floatx4{(float)f2h_signed(d * (float)sc[2 * g]) * 0x1p24f,
                    (float)f2h_signed(dmin * (float)mn[2 * g]),
                    (float)f2h_signed(d * (float)sc[2 * g + 1]) * 0x1p20f,
                    (float)f2h_signed(dmin * (float)mn[2 * g + 1])};
    } else {  // the products are exact in fp32 (11-bit d times a 6-bit integer)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<floatx4*>(dst + 16 * k + 4 * g) =
            floatx4{(d * (float)sc[2 * g]) * 0x1p24f, dmin * (float)mn[2 * g],
                    (d * (float)sc[2 * g + 1]) * 0x1p24f, dmin * (float)mn[2 * g + 1]};
    }
  } else {
    const float d = h2f_bits((uint16_t)s.d);
    float f[16];
#pragma unroll
    for (int t = 0; t < 16; ++t)
      f[q6_slot(t)] = (d * (float)(int8_t)((s.v[t / 4] >> (8 * (t % 4))) & 0xFF)) * 0x1p24f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<floatx4*>(dst + 16 * k + 4 * i) =
          floatx4{f[4 * i], f[4 * i + 1], f[4 * i + 2], f[4 * i + 3]};
  }
}

// Weight loads in flight per lane (NPW: pieces per lane and slice, 0 = any K).
template <int FMT, int R, int NPW>
constexpr int qbatch() {
  constexpr int cap = R == 4 ? (FMT == 12 ? 20 : 8) : (FMT == 12 ? 8 : 4);
  return NPW > 0 && NPW < cap ? NPW : cap;
}

// Consumes pieces st + J.. of the lane's slice (counted from piece i0 on),
// refilling each slot B pieces ahead.
template <int FMT, int NPW, int B, int J>
__device__ __forceinline__ void qconsume(QPc (&raw)[B], float& acc, int st, int i0, int m,
                                         const QLane& q, const unsigned char* s_xb,
                                         const float* s_xsum, const float* s_row,
                                         const uint8_t* __restrict__ W, const QLayout& L, int row,
                                         int K) {
  if constexpr (J < NPW) {
    // the LDS offsets of piece st + J are compile-time steps from the base
    // pointers, which already point at piece st
    const float v = qpc_dot<FMT, J>(raw[J % B], m, q, s_xb, s_xsum, s_row);
    acc += st + J >= i0 ? v : 0.f;
    if constexpr (J + B < NPW) raw[J % B] = qpc_load<FMT>(W, L, row, m + 16 * (st + J + B), K);
    qconsume<FMT, NPW, B, J + 1>(raw, acc, st, i0, m, q, s_xb, s_xsum, s_row, W, L, row, K);
  }
}

// Input RMSNorm folded into the staging of x (the NORM kernels): c =
// residual + x in fp32 (residual NULL reads zeros: c = x exactly),
// x' = f16(c * inv * gamma), inv = 1 / rms(c), and f16(c) to residual_out
// when it is not NULL.  Every workgroup computes inv itself (in a fixed
// order: lane sums, wave butterflies, waves in order); the first writes
// residual_out.
struct QNorm {
  const half_t* res;
  const half_t* gamma;
  half_t* res_out;
  float eps;
};

// The residual of a norm without one (read-only zeros, never written).
__device__ half_t kQZero[kQMaxK];

__device__ __forceinline__ float qwave_sum(float v) { return wave_xor_sum(v); }

// c of chunk (8 values) and its contribution to sum(c^2).
__device__ __forceinline__ float qnorm_c(u32x4 xv, u32x4 rv, float (&c)[8]) {
  const half8 xh = as_half8(xv), rh = as_half8(rv);
  float part = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    c[e] = (float)rh[e] + (float)xh[e];
    part += c[e] * c[e];
  }
  return part;
}

// 1 / rms over the workgroup from each thread's partial sum (s_nrm: one float
// per wave); every thread of the workgroup calls it.
template <int T>
__device__ __forceinline__ float qnorm_inv(float ss, int K, float eps, float* s_nrm) {
  ss = qwave_sum(ss);
  if ((threadIdx.x & 63) == 0) s_nrm[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = s_nrm[0];
#pragma unroll
  for (int w = 1; w < T / 64; ++w) ss += s_nrm[w];
  return 1.0f / sqrtf(ss / (float)K + eps);
}

// x' of one chunk; the first workgroup also writes f16(c) to residual_out.
__device__ __forceinline__ u32x4 qnorm_apply(u32x4 xv, u32x4 rv, u32x4 gv, float inv, int c, int NG,
                                             const QNorm& nz) {
  float cv[8];
  (void)qnorm_c(xv, rv, cv);
  const half8 gh = as_half8(gv);
  half8 o, co;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] = (half_t)(cv[e] * inv * (float)gh[e]);
    co[e] = (half_t)cv[e];
  }
  if (nz.res_out != nullptr && blockIdx.x == 0 && c < NG)
    *reinterpret_cast<u32x4*>(nz.res_out + 8 * c) = as_u32x4(co);
  return as_u32x4(o);
}

// R weight rows per workgroup, each split into S slices of NPW pieces per
// lane (one slice per group of R teams; K a multiple of 512 with
// NPW * S >= K / 512 >= NPW), or NPW = 0: any K, S = 1.  NORM: x is the
// RMSNorm of residual + x (QNorm).
template <int FMT, bool SILU, int R, int S, int NPW, bool NORM>
__global__ __launch_bounds__(R * S * kQTeam) void gemv_q_kernel(const uint8_t* __restrict__ W,
                                                               const half_t* __restrict__ x,
                                                               half_t* __restrict__ y, int N,
                                                               int K, QLayout L, QNorm nz) {
  constexpr int T = R * S * kQTeam;
  constexpr int B = qbatch<FMT, R, NPW>();
  // LDS: x (K halves, padded to whole swizzle runs), x sums, each local row's
  // scales (SCW floats), then S x R slice partials and one float per wave
  // for the norm.
  extern __shared__ __attribute__((aligned(16))) unsigned char s_dyn[];
  const int KX = (K + 127) & ~127;
  half_t* const s_x = reinterpret_cast<half_t*>(s_dyn);
  float* const s_xsum = reinterpret_cast<float*>(s_dyn + (size_t)KX * 2);
  float* const s_sc = s_xsum + (FMT == 8 ? K / 32 : K / 16);
  const int SCW = FMT == 8 ? K / 32 : K / 16;
  const int UPR = FMT == 8 ? K / 32 : K / 256;  // staging units per row
  const float inv_upr = __builtin_amdgcn_rcpf((float)UPR);
  const int U = R * UPR, NG = K / 8, P = K / 32;
  const int tid = threadIdx.x, slice = tid / (R * kQTeam), team = (tid >> 4) % R, m = tid & 15;
  int out;
  const int row = qrow<SILU, R>(team, N, out);
  const float* const s_row = s_sc + team * SCW;
  const QLane q = qlane<FMT>(m);
  float acc = 0.f;

  if constexpr (NPW > 0) {
    // x, scale and first weight loads all in flight before any is used (the
    // per-thread counts are bounds: NP <= NPW * S pieces per lane)
    constexpr int NXJ = (NPW * S * 64 + T - 1) / T;
    constexpr int NUJ = ((FMT == 8 ? 16 : 2) * R * NPW * S + T - 1) / T;
    const int NP = K / 512;
    // slice pieces i0 .. i0 + NPW - 1 clipped to NP: a slice that would run
    // past the end starts at NP - NPW and counts only pieces >= i0
    const int i0 = slice * NPW, st = min(i0, NP - NPW);
    u32x4 xr[NXJ], rr[NORM ? NXJ : 1], gr[NORM ? NXJ : 1];
#pragma unroll
    for (int j = 0; j < NXJ; ++j) xr[j] = load16(x + 8 * min(tid + T * j, NG - 1));
    if constexpr (NORM) {
      const half_t* res = nz.res != nullptr ? nz.res : kQZero;
#pragma unroll
      for (int j = 0; j < NXJ; ++j) rr[j] = load16(res + 8 * min(tid + T * j, NG - 1));
#pragma unroll
      for (int j = 0; j < NXJ; ++j) gr[j] = load16(nz.gamma + 8 * min(tid + T * j, NG - 1));
    }
    SRaw ur[NUJ];
#pragma unroll
    for (int j = 0; j < NUJ; ++j)
      ur[j] = stage_load<FMT, SILU, R>(W, L, min(tid + T * j, U - 1), UPR, inv_upr, N, K);
    QPc raw[B];
#pragma unroll
    for (int b = 0; b < B; ++b) raw[b] = qpc_load<FMT>(W, L, row, m + 16 * (st + b), K);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < NXJ; ++j) {
        float cv[8];
        const float part = qnorm_c(xr[j], rr[j], cv);
        ss += tid + T * j < NG ? part : 0.f;
      }
      const float inv = qnorm_inv<T>(ss, K, nz.eps, s_sc + R * SCW + S * R);
#pragma unroll
      for (int j = 0; j < NXJ; ++j) xr[j] = qnorm_apply(xr[j], rr[j], gr[j], inv, tid + T * j, NG, nz);
    }
#pragma unroll
    for (int j = 0; j < NXJ; ++j) stage_x<FMT>(xr[j], tid + T * j, NG, s_x, s_xsum);
#pragma unroll
    for (int j = 0; j < NUJ; ++j) stage_store<FMT>(ur[j], tid + T * j, U, UPR, inv_upr, SCW, s_sc);
    __syncthreads();
    const int fs = FMT == 8 ? 16 : 32;  // scale / x-sum floats per piece step
    qconsume<FMT, NPW, B, 0>(raw, acc, st, i0, m, q,
                             reinterpret_cast<const unsigned char*>(s_x) + 1024 * st,
                             s_xsum + fs * st, s_row + fs * st, W, L, row, K);
  } else {
    const int nxj = (NG + T - 1) / T;
    float inv = 0.f;
    const half_t* res = nz.res != nullptr ? nz.res : kQZero;
    if constexpr (NORM) {  // a first pass for 1 / rms
      float ss = 0.f;
      for (int j = 0; j < nxj; ++j) {
        const int c = tid + T * j, cc = min(c, NG - 1);
        float cv[8];
        const float part = qnorm_c(load16(x + 8 * cc), load16(res + 8 * cc), cv);
        ss += c < NG ? part : 0.f;
      }
      inv = qnorm_inv<T>(ss, K, nz.eps, s_sc + R * SCW + S * R);
    }
    for (int j = 0; j < nxj; ++j) {
      const int c = tid + T * j, cc = min(c, NG - 1);
      u32x4 xv = load16(x + 8 * cc);
      if constexpr (NORM)
        xv = qnorm_apply(xv, load16(res + 8 * cc), load16(nz.gamma + 8 * cc), inv, c, NG, nz);
      stage_x<FMT>(xv, c, NG, s_x, s_xsum);
    }
    for (int u = tid; u < U; u += T)
      stage_store<FMT>(stage_load<FMT, SILU, R>(W, L, u, UPR, inv_upr, N, K), u, U, UPR, inv_upr,
                       SCW, s_sc);
    __syncthreads();
    const int npl = (P + 15) / 16;
    const int fs = FMT == 8 ? 16 : 32;
    const unsigned char* s_xb = reinterpret_cast<const unsigned char*>(s_x);
    for (int i = 0; i < npl; ++i) {
      const int p = m + 16 * i;
      const QPc r = qpc_load<FMT>(W, L, row, min(p, P - 1), K);
      const float v = qpc_dot<FMT, 0>(r, m, q, s_xb + 1024 * i, s_xsum + fs * i, s_row + fs * i);
      acc += p < P ? v : 0.f;
    }
  }

  // the team's 16 lanes, butterfly order (lane ^ 8, 4, 2, 1), on the VALU
  acc += xor_lane<8>(acc);
  acc += xor_lane<4>(acc);
  acc += xor_lane<2>(acc);
  acc += xor_lane<1>(acc);
  if constexpr (S > 1) {
    // slice partials summed in slice order by slice 0
    float* const s_red = s_sc + R * SCW;
    if (m == 0) s_red[slice * R + team] = acc;
    __syncthreads();
    if (slice != 0) return;
    acc = s_red[team];
#pragma unroll
    for (int w = 1; w < S; ++w) acc += s_red[w * R + team];
  }
  if (SILU) {
    const float up = xor_lane<32>(acc);  // gate teams 0, 1 <-> up teams 2, 3
    if (m == 0 && (team & 3) < 2 && out < N) {
      const half_t g = (half_t)acc, u = (half_t)up;
      const float gf = (float)g;
      const float sig = 1.0f / (1.0f + expf(-gf));
      y[out] = (half_t)(sig * gf * (float)u);
    }
  } else if (m == 0 && out < N) {
    y[out] = (half_t)acc;
  }
}

// ---------------------------------------------------------------- dequant to f16


// Raw bytes of one piece (row, j).
struct QRaw {
  u32x4 a;  // primary payload: Q8_0 q, Q4_K and Q5_K qs, Q6_K ql
  u32x4 b;  // Q5_K, Q6_K: the 16 qh bytes of the piece's runs
};

template <int FMT>
__device__ __forceinline__ QRaw qload(const uint8_t* __restrict__ W, const QLayout& L, int row,
                                      int j, int K) {
  QRaw r;
  if (FMT == 8) {
    r.a = load_stream16(W + L.off[0] + (size_t)row * K + (size_t)j * 16);
  } else if (FMT == 12) {
    r.a = load_stream16(W + L.off[0] + (size_t)row * (K / 2) + (size_t)j * 16);
    r.b = u32x4{0u, 0u, 0u, 0u};  // no fifth bits
  } else if (FMT == 13) {
    r.a = load_stream16(W + L.off[0] + (size_t)row * (K / 2) + (size_t)j * 16);
    r.b = load_stream16(W + L.off[2] + (size_t)row * (K / 8) + (size_t)(j >> 3) * 32 + (j & 1) * 16);
  } else {
    r.a = load_stream16(W + L.off[0] + (size_t)row * (K / 2) + (size_t)j * 16);
    const int sb = j >> 3, o = (j & 7) * 16, n = o >> 6, h = o & 63;
    r.b = load_stream16(W + L.off[1] + (size_t)row * (K / 4) + sb * 64 + 32 * n + (h & 31));
  }
  return r;
}



// Piece j of weight row `row` as f16 into o (the row's output).  Each weight
// is fp32 arithmetic in the reference's order (no fused multiply-add), rounded
// once to f16.  DECODE: the decode layout's Q4_K scales, f16(d * sc) and
// f16(dmin * m); otherwise the CPU rule, d * sc and dmin * m in fp32 (the
// reference's native-layout embedding gather, src/kernels.rs:1963-2007).
// Q5_K has only the CPU rule (the reference keeps it in the native layout).
template <int FMT, bool DECODE>
__device__ __forceinline__ void dequant_piece(const uint8_t* __restrict__ W, const QLayout& L,
                                              int row, int j, int K, half_t* __restrict__ o) {
#pragma clang fp contract(off)
  const QRaw r = qload<FMT>(W, L, row, j, K);
  if (FMT == 8) {
    const float d = h2f_bits(*reinterpret_cast<const uint16_t*>(W + L.off[1] +
                                                                 ((size_t)row * (K / 32) + (j >> 1)) * 2));
    const int8_t* q = reinterpret_cast<const int8_t*>(&r.a);
    for (int i = 0; i < 16; ++i) o[16 * j + i] = f2h_signed((float)q[i] * d);
  } else if (FMT == 12 || FMT == 13) {
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
    float d1 = d * (float)s[0], m1 = dmin * (float)m[0];
    float d2 = d * (float)s[1], m2 = dmin * (float)m[1];
    if (DECODE && FMT == 12) {  // effective scales of the decode layout
      d1 = (float)f2h_signed(d1);
      m1 = (float)f2h_signed(m1);
      d2 = (float)f2h_signed(d2);
      m2 = (float)f2h_signed(m2);
    }
    const uint8_t* q = reinterpret_cast<const uint8_t*>(&r.a);
    const int e0 = sb * 256 + 64 * g + l0;
    const uint8_t* qh = reinterpret_cast<const uint8_t*>(&r.b);
    for (int i = 0; i < 16; ++i) {
      const int hlo = FMT == 13 ? ((qh[i] >> (2 * g)) & 1) << 4 : 0;
      const int hhi = FMT == 13 ? ((qh[i] >> (2 * g + 1)) & 1) << 4 : 0;
      o[e0 + i] = f2h_signed(d1 * (float)((q[i] & 0xF) + hlo) - m1);
      o[e0 + 32 + i] = f2h_signed(d2 * (float)((q[i] >> 4) + hhi) - m2);
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

// w[row][k] as f16 with the decode layout's scales (for the prefill GEMMs):
// one thread per piece of 16 (Q8_0) or 32 weights.
template <int FMT>
__global__ __launch_bounds__(256) void qdequant_kernel(const uint8_t* __restrict__ W, int N,
                                                      int K, QLayout L, half_t* __restrict__ out) {
  const int P = K / (FMT == 8 ? 16 : 32);
  const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= (size_t)N * P) return;
  const int row = (int)(p / P), j = (int)(p % P);
  dequant_piece<FMT, true>(W, L, row, j, K, out + (size_t)row * K);
}

// out[t][k] = f16 of row ids[t] of the N-row matrix by the CPU rule (token
// embedding gather); ids at or past N read row N - 1.
template <int FMT>
__global__ __launch_bounds__(256) void qgather_kernel(const uint8_t* __restrict__ W, int N, int K,
                                                     QLayout L, const uint32_t* __restrict__ ids,
                                                     int rows, half_t* __restrict__ out) {
  const int P = K / (FMT == 8 ? 16 : 32);
  const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= (size_t)rows * P) return;
  const int t = (int)(p / P), j = (int)(p % P);
  const int row = (int)min(ids[t], (uint32_t)(N - 1));
  dequant_piece<FMT, false>(W, L, row, j, K, out + (size_t)t * K);
}

// ---------------------------------------------------------------- launchers

static bool qfmt_ok(int fmt, int N, int K) {
  if (N < 1 || K < 1) return false;
  const int blk = fmt == 8 ? 32 : 256;
  if (fmt != 8 && fmt != 12 && fmt != 13 && fmt != 14) return false;
  return K % blk == 0 && K <= kQMaxK;
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

// Pieces per lane and slice with an instantiated kernel: 16-row workgroups
// (S = 1) and 4-row workgroups (S = 1, 2, 4).
static bool npw_tall(int v) { return v == 5 || v == 8 || v == 10 || v == 16 || v == 19; }
static bool npw_short(int v) {
  return v == 2 || v == 3 || v == 4 || v == 5 || v == 8 || v == 10 || v == 13;
}

template <int FMT, bool SILU, int R, int S, bool NORM>
static void gemv_q_go(int npw, unsigned grid, size_t lds, const void* W, const void* x, void* y,
                      int N, int K, const QLayout& L, const QNorm& nz, hipStream_t stream) {
  const uint8_t* w = (const uint8_t*)W;
  const half_t* xi = (const half_t*)x;
  half_t* yo = (half_t*)y;
  constexpr int T = R * S * kQTeam;
#define GROUT_QGO(V) \
  case V:                                                                                     \
    gemv_q_kernel<FMT, SILU, R, S, V, NORM><<<grid, T, lds, stream>>>(w, xi, yo, N, K, L, nz); \
    break;
  if constexpr (R == 16) {
    switch (npw) {
      GROUT_QGO(5) GROUT_QGO(8) GROUT_QGO(10) GROUT_QGO(16) GROUT_QGO(19)
      default:
        gemv_q_kernel<FMT, SILU, R, 1, 0, NORM><<<grid, T, lds, stream>>>(w, xi, yo, N, K, L, nz);
    }
  } else if constexpr (SILU || S == 0) {
    gemv_q_kernel<FMT, SILU, R, 1, 0, NORM><<<grid, R * kQTeam, lds, stream>>>(w, xi, yo, N, K, L,
                                                                             nz);
  } else {
    switch (npw) {
      GROUT_QGO(2) GROUT_QGO(3) GROUT_QGO(4) GROUT_QGO(5) GROUT_QGO(8) GROUT_QGO(10)
      GROUT_QGO(13)
      default: break;
    }
  }
#undef GROUT_QGO
}

// LDS bytes of a workgroup of R rows in S slices (layout in gemv_q_kernel).
template <int FMT>
static size_t gemv_q_lds(int R, int S, int K) {
  return (size_t)((K + 127) & ~127) * 2 + (size_t)(FMT == 8 ? K / 32 : K / 16) * 4 +
         (size_t)R * (FMT == 8 ? K / 32 : K / 16) * 4 + (size_t)R * S * 4 + 4 * 4;
}

// Largest LDS allocation one workgroup may make on the current device
// (queried once per device; 64 KiB if the query fails).
static size_t qmax_lds() {
  constexpr int kDevs = 64;
  static std::atomic<int> cached[kDevs];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 65536;
  if (dev >= 0 && dev < kDevs) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return (size_t)c;
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
      v <= 0)
    return 65536;
  if (dev >= 0 && dev < kDevs) cached[dev].store(v, std::memory_order_relaxed);
  return (size_t)v;
}

template <int FMT, bool NORM>
static hipError_t gemv_q_launch(const void* W, const void* x, void* y, int N, int K, bool silu,
                                const QNorm& nz, hipStream_t stream) {
  const int rows = silu ? 2 * N : N;
  const QLayout L = qlayout(FMT, (size_t)rows, (size_t)K);
  const int np = K % 512 == 0 ? K / 512 : 0;  // pieces per lane of a whole row
  if (rows >= 16 * 1024 && gemv_q_lds<FMT>(16, 1, K) <= 65536) {
    // tall: 16 rows per workgroup (x staged once per 16 rows)
    const int per = silu ? 8 : 16;
    const unsigned grid = (unsigned)((N + per - 1) / per);
    const int npw = npw_tall(np) ? np : 0;
    if (silu) gemv_q_go<FMT, true, 16, 1, NORM>(npw, grid, gemv_q_lds<FMT>(16, 1, K), W, x, y, N, K, L, nz, stream);
    else gemv_q_go<FMT, false, 16, 1, NORM>(npw, grid, gemv_q_lds<FMT>(16, 1, K), W, x, y, N, K, L, nz, stream);
    return hipGetLastError();
  }
  // short: 4 rows per workgroup, each row split over S waves so that the grid
  // holds about 2048 waves or more
  const int per = silu ? 2 : 4;
  if (gemv_q_lds<FMT>(4, 4, K) > qmax_lds()) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)((N + per - 1) / per);
  if (silu) {
    gemv_q_go<FMT, true, 4, 0, NORM>(0, grid, gemv_q_lds<FMT>(4, 1, K), W, x, y, N, K, L, nz, stream);
    return hipGetLastError();
  }
  int S = 0, npw = 0;
  if (np > 0) {
    for (int s = grid >= 2048 ? 1 : grid >= 1024 ? 2 : 4; s <= 4 && S == 0; s *= 2) {
      const int v = (np + s - 1) / s;
      if (v <= np && npw_short(v)) S = s, npw = v;
    }
  }
  if (S == 0) gemv_q_go<FMT, false, 4, 0, NORM>(0, grid, gemv_q_lds<FMT>(4, 1, K), W, x, y, N, K, L, nz, stream);
  else if (S == 1) gemv_q_go<FMT, false, 4, 1, NORM>(npw, grid, gemv_q_lds<FMT>(4, 1, K), W, x, y, N, K, L, nz, stream);
  else if (S == 2) gemv_q_go<FMT, false, 4, 2, NORM>(npw, grid, gemv_q_lds<FMT>(4, 2, K), W, x, y, N, K, L, nz, stream);
  else gemv_q_go<FMT, false, 4, 4, NORM>(npw, grid, gemv_q_lds<FMT>(4, 4, K), W, x, y, N, K, L, nz, stream);
  return hipGetLastError();
}

hipError_t launch_gemv_q(int fmt, const void* W, const void* x, void* y, int N, int K, bool silu,
                         hipStream_t stream) {
  return launch_gemv_q_norm(fmt, W, nullptr, x, nullptr, nullptr, 0.f, y, N, K, silu, stream);
}

hipError_t launch_gemv_q_norm(int fmt, const void* W, const void* residual, const void* x,
                              const void* gamma, void* residual_out, float eps, void* y, int N,
                              int K, bool silu, hipStream_t stream) {
  const QNorm nz{(const half_t*)residual, (const half_t*)gamma, (half_t*)residual_out, eps};
  if (!qfmt_ok(fmt, silu ? 2 * N : N, K)) return hipErrorInvalidValue;
  const bool norm = gamma != nullptr;
  switch (fmt) {
    case 8:
      return norm ? gemv_q_launch<8, true>(W, x, y, N, K, silu, nz, stream)
                  : gemv_q_launch<8, false>(W, x, y, N, K, silu, nz, stream);
    case 12:
      return norm ? gemv_q_launch<12, true>(W, x, y, N, K, silu, nz, stream)
                  : gemv_q_launch<12, false>(W, x, y, N, K, silu, nz, stream);
    case 13:
      return norm ? gemv_q_launch<13, true>(W, x, y, N, K, silu, nz, stream)
                  : gemv_q_launch<13, false>(W, x, y, N, K, silu, nz, stream);
    default:
      return norm ? gemv_q_launch<14, true>(W, x, y, N, K, silu, nz, stream)
                  : gemv_q_launch<14, false>(W, x, y, N, K, silu, nz, stream);
  }
}

hipError_t launch_qgather(int fmt, const void* W, int N, int K, const uint32_t* ids, int rows,
                          void* out, hipStream_t stream) {
  if (!qfmt_ok(fmt, N, K) || rows < 1) return hipErrorInvalidValue;
  const QLayout L = qlayout(fmt, (size_t)N, (size_t)K);
  const size_t pieces = (size_t)rows * (K / (fmt == 8 ? 16 : 32));
  const unsigned blocks = (unsigned)((pieces + 255) / 256);
  const uint8_t* w = (const uint8_t*)W;
  switch (fmt) {
    case 8: qgather_kernel<8><<<blocks, 256, 0, stream>>>(w, N, K, L, ids, rows, (half_t*)out); break;
    case 12: qgather_kernel<12><<<blocks, 256, 0, stream>>>(w, N, K, L, ids, rows, (half_t*)out); break;
    case 13: qgather_kernel<13><<<blocks, 256, 0, stream>>>(w, N, K, L, ids, rows, (half_t*)out); break;
    default: qgather_kernel<14><<<blocks, 256, 0, stream>>>(w, N, K, L, ids, rows, (half_t*)out); break;
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
    case 13: qdequant_kernel<13><<<blocks, 256, 0, stream>>>((const uint8_t*)W, N, K, L, (half_t*)out); break;
    default: qdequant_kernel<14><<<blocks, 256, 0, stream>>>((const uint8_t*)W, N, K, L, (half_t*)out); break;
  }
  return hipGetLastError();
}

}  // namespace grout
