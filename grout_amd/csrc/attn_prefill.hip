// Causal GQA prefill flash attention on fp16 MFMA.
//
// Reference: fmha_prefill_causal (src/kernels.rs:2559-2725) and the GQA-packed
// LPT variant fmha_prefill_gqa_lpt (src/kernels.rs:2933-3298), dispatched by
// src/model.rs:6856-7134.  Same math: q_pos = pos0 + row attends to kv
// positions k_pos <= q_pos (kv_len = pos0 + S); fp32 online softmax in exp2
// units; output acc / l in f16.  K/V are read through an explicit
// kv_head_stride, so the engine's [Hkv][max_ctx][D] cache works for every kv
// head (the reference's LPT path assumes stride kv_len*D).
//
// gfx950 design (v_mfma_f32_16x16x32_f16, 256-thread workgroups):
//  * a workgroup owns up to 128 query rows = BQ query positions x HG heads of
//    one kv group (HG = the largest divisor of G that is <= 8, BQ =
//    floor(128/HG)), so every K/V tile staged in LDS serves HG heads; each
//    wave owns 32 rows (two 16-column MFMA blocks);
//  * S^T = K.Q^T (A = K rows from LDS, B = Q held in VGPRs for the whole
//    loop) and O^T = V^T.P^T (A = V^T rows from LDS, B = P straight from the
//    S^T accumulators): each query row is one lane column, so its softmax
//    statistics never leave the lanes that own its accumulator;
//  * K is staged row-major, V is staged transposed (d-major, with the
//    position order of the P fragments), both with padded rows;
//  * causal: tiles past the workgroup's last query are skipped, masks are
//    applied only on tiles crossing the diagonal;
//  * scheduling: block id -> (kv head = id mod Hkv, q block from the heavy
//    end), so the longest blocks start first and, with Hkv = 8, each XCD's L2
//    holds one kv head's K/V.
#include "common.hpp"
#include "kernels.hpp"

namespace grout {

constexpr int kBN = 64;                  // kv positions per tile
constexpr int kKStride = kHeadDim + 8;   // halves per K row in LDS (272 B)
constexpr int kVtStride = kBN + 8;       // halves per V^T row in LDS (144 B)
constexpr int kRowsPerWG = 128;

// Position (0..31) within a 32-position chunk -> its column in V^T, matching
// the P fragment slot order: slot (kb, j) holds position 4kb+j (j<4) or
// 16+4kb+(j-4) (j>=4).
__device__ __forceinline__ int vt_perm(int p) {
  return p < 16 ? 8 * (p >> 2) + (p & 3) : 8 * ((p - 16) >> 2) + 4 + (p & 3);
}

template <int HG>
__global__ __launch_bounds__(256) void fmha_prefill_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k_cache,
    const half_t* __restrict__ v_cache, half_t* __restrict__ out, int S, int pos0, int Hq,
    int Hkv, long head_stride, float scale_log2, int nqb) {
  constexpr int BQ = kRowsPerWG / HG;
  __shared__ __attribute__((aligned(16))) half_t k_lds[kBN * kKStride];
  __shared__ __attribute__((aligned(16))) half_t vt_lds[kHeadDim * kVtStride];

  const int G = Hq / Hkv;
  const int nsub = G / HG;
  const int bid = blockIdx.x;
  const int kvh = bid % Hkv;
  const int rest = bid / Hkv;
  const int hsub = rest % nsub;
  const int qb = nqb - 1 - rest / nsub;
  const int q0 = qb * BQ;

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, kb = lane >> 4;

  const half_t* kh = k_cache + (size_t)kvh * head_stride;
  const half_t* vh = v_cache + (size_t)kvh * head_stride;
  const int kv_len = pos0 + S;

  int qrow[2], qhead[2], qpos[2];
  bool rvalid[2];
  half8 qf[2][4];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const int r = 32 * w + 16 * mb + col;
    qrow[mb] = q0 + r / HG;
    qhead[mb] = kvh * G + hsub * HG + r % HG;
    rvalid[mb] = r < BQ * HG && qrow[mb] < S;
    qpos[mb] = pos0 + qrow[mb];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      qf[mb][c] = rvalid[mb]
                      ? as_half8(load16(q + ((size_t)qrow[mb] * Hq + qhead[mb]) * kHeadDim +
                                        c * 32 + kb * 8))
                      : as_half8(u32x4{0u, 0u, 0u, 0u});
    }
  }

  const int q_last = min(q0 + BQ, S) - 1;
  const int kv_end = pos0 + q_last + 1;
  const int ntiles = (kv_end + kBN - 1) / kBN;
  const int first_masked_kv = pos0 + q0;  // a tile needs masking if it reaches past this

  float m[2] = {-1.0e30f, -1.0e30f};
  float l[2] = {0.f, 0.f};
  floatx4 acc[2][8];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[mb][db] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Staging: thread -> K (chunk = tid%16, rows tid/16 + 16i) and V (chunk =
  // tid%16, row pairs 2a,2a+1 in each 32-row half, a = tid/16).
  const int chunk = tid & 15, rsel = tid >> 4;
  u32x4 kreg[4], vreg[4];
  auto gload = [&](int tile) {
    const int kv0 = tile * kBN;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int p = kv0 + rsel + 16 * i;
      p = p < kv_len ? p : kv_len - 1;
      kreg[i] = load16(kh + (size_t)p * kHeadDim + chunk * 8);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int p = kv0 + 32 * (i >> 1) + 2 * rsel + (i & 1);
      p = p < kv_len ? p : kv_len - 1;
      vreg[i] = load16(vh + (size_t)p * kHeadDim + chunk * 8);
    }
  };
  auto lds_store = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4*>(&k_lds[(rsel + 16 * i) * kKStride + chunk * 8]) = kreg[i];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int colp = 32 * hh + vt_perm(2 * rsel);
      const u32x4 a = vreg[2 * hh], b = vreg[2 * hh + 1];
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        const uint32_t lo = (a[wd] & 0xffffu) | (b[wd] << 16);
        const uint32_t hi = (a[wd] >> 16) | (b[wd] & 0xffff0000u);
        const int d = chunk * 8 + 2 * wd;
        *reinterpret_cast<uint32_t*>(&vt_lds[d * kVtStride + colp]) = lo;
        *reinterpret_cast<uint32_t*>(&vt_lds[(d + 1) * kVtStride + colp]) = hi;
      }
    }
  };

  gload(0);
  for (int tile = 0; tile < ntiles; ++tile) {
    __syncthreads();
    lds_store();
    __syncthreads();
    if (tile + 1 < ntiles) gload(tile + 1);

    const int kv0 = tile * kBN;
    floatx4 sc[2][4];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      half8 kf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kf[c] = *reinterpret_cast<const half8*>(&k_lds[(16 * pb + col) * kKStride + c * 32 + kb * 8]);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        floatx4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) a = mfma16x16x32(kf[c], qf[mb][c], a);
        sc[mb][pb] = a;
      }
    }

    const bool need_mask = kv0 + kBN - 1 > first_masked_kv;
    half8 pf[2][2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      if (need_mask) {
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int pos = kv0 + 16 * pb + 4 * kb + i;
            if (pos > qpos[mb]) sc[mb][pb][i] = -1.0e30f;
          }
      }
      float tmax = -1.0e30f;
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, sc[mb][pb][i]);
      tmax = fmaxf(tmax, shfl_xor(tmax, 16));
      tmax = fmaxf(tmax, shfl_xor(tmax, 32));
      const float mnew = fmaxf(m[mb], tmax * scale_log2);
      const float alpha = fast_exp2(m[mb] - mnew);
      float psum = 0.f;
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(sc[mb][pb][i] * scale_log2 - mnew);
          psum += p;
          pf[mb][pb >> 1][(pb & 1) * 4 + i] = (half_t)p;
        }
      l[mb] = l[mb] * alpha + psum;
      m[mb] = mnew;
#pragma unroll
      for (int db = 0; db < 8; ++db) acc[mb][db] *= alpha;
    }

#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const half8 vf = *reinterpret_cast<const half8*>(
            &vt_lds[(16 * db + col) * kVtStride + 32 * cc + 8 * kb]);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) acc[mb][db] = mfma16x16x32(vf, pf[mb][cc], acc[mb][db]);
      }
  }

#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    float lt = l[mb];
    lt += shfl_xor(lt, 16);
    lt += shfl_xor(lt, 32);
    if (!rvalid[mb]) continue;
    const float inv = 1.0f / lt;
    half_t* orow = out + ((size_t)qrow[mb] * Hq + qhead[mb]) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      half4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = (half_t)(acc[mb][db][i] * inv);
      *reinterpret_cast<u32x2*>(orow + 16 * db + 4 * kb) = __builtin_bit_cast(u32x2, o);
    }
  }
}

hipError_t launch_fmha_prefill(const void* q, const void* k_cache, const void* v_cache,
                               void* out, int seq_len, int pos0, int Hq, int Hkv,
                               long head_stride, float qk_scale, hipStream_t stream) {
  const float scale_log2 = qk_scale * 1.4426950408889634f;
  const int G = Hq / Hkv;
  int HG = 8;
  while (G % HG != 0) --HG;
  const int BQ = kRowsPerWG / HG;
  const int nqb = (seq_len + BQ - 1) / BQ;
  const unsigned blocks = (unsigned)(nqb * Hkv * (G / HG));
#define GROUT_PREFILL_CASE(hg)                                                              \
  case hg:                                                                                  \
    fmha_prefill_kernel<hg><<<blocks, 256, 0, stream>>>(                                   \
        (const half_t*)q, (const half_t*)k_cache, (const half_t*)v_cache, (half_t*)out,     \
        seq_len, pos0, Hq, Hkv, head_stride, scale_log2, nqb);                              \
    break;
  switch (HG) {
    GROUT_PREFILL_CASE(1)
    GROUT_PREFILL_CASE(2)
    GROUT_PREFILL_CASE(3)
    GROUT_PREFILL_CASE(4)
    GROUT_PREFILL_CASE(5)
    GROUT_PREFILL_CASE(6)
    GROUT_PREFILL_CASE(7)
    GROUT_PREFILL_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef GROUT_PREFILL_CASE
  return hipGetLastError();
}

}  // namespace grout
