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
// gfx950 design (v_mfma_f32_16x16x32_f16, 256-thread workgroups, 2 per CU):
//  * a workgroup owns up to 128 query rows = BQ query positions x HG heads of
//    one kv group (HG = the largest divisor of G that is <= 8, BQ =
//    floor(128/HG)), so every K/V tile staged in LDS serves HG heads; each
//    wave owns 32 rows (two 16-column MFMA blocks);
//  * K and V tiles (64 positions) are loaded with lane-contiguous 16-byte
//    loads and stored row-major into double-buffered, XOR-swizzled LDS; the
//    next tile is in flight while the current one is computed, with one
//    workgroup barrier per tile;
//  * S^T = K.Q^T (A = K rows from LDS, B = Q held in VGPRs for the whole
//    loop) and O^T = V^T.P^T: the V^T fragments come straight from the
//    row-major tile with ds_read_b64_tr_b16 (gfx950's transposing LDS read),
//    P comes from the S^T accumulators without any shuffle, and each query
//    row is one lane column, so its softmax statistics live in the lanes that
//    own its accumulator;
//  * the accumulator rescale is skipped when no row of the wave raised its
//    running max (most tiles once the first few are in);
//  * causal: tiles past the workgroup's last query are skipped, masks are
//    applied only on tiles crossing the diagonal;
//  * scheduling: block id -> (kv head = id mod Hkv, q block from the heavy
//    end), so the longest blocks start first and, with Hkv = 8, each XCD's L2
//    holds one kv head's K/V.
#include "common.hpp"
#include "kernels.hpp"

namespace grout {

constexpr int kBN = 64;                          // kv positions per tile
constexpr int kRowsPerWG = 128;
constexpr int kTileHalfBytes = kBN * kHeadDim * 2;  // 16 KiB: one of K or V
constexpr int kStageBytes = 2 * kTileHalfBytes;     // K + V

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;

// Byte offset of 16-byte chunk `chunk` (0..15) of row `row` in a swizzled tile.
__device__ __forceinline__ int pswz(int row, int chunk) {
  return row * 256 + ((chunk ^ (row & 15)) << 4);
}

// ds_read_b64_tr_b16: inside each 16-lane group, lane i receives element
// (i % 4) of the 8-byte chunks addressed by lanes i/4, i/4+4, i/4+8, i/4+12.
// The result is bit-cast as a whole vector and two of them are joined with
// one shuffle: extracting it element by element into a half8 was compiled
// into a duplicate-low-half permute (only element 0 survived).
__device__ __forceinline__ half4 lds_read_tr16(const unsigned char* p) {
  const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)(__attribute__((address_space(3))) unsigned char*)(p));
  return __builtin_bit_cast(half4, v);
}

template <int HG>
__global__ __launch_bounds__(256, 2) void fmha_prefill_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k_cache,
    const half_t* __restrict__ v_cache, half_t* __restrict__ out, int S, int pos0, int Hq,
    int Hkv, long head_stride, float scale_log2, int nqb) {
  constexpr int BQ = kRowsPerWG / HG;
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * kStageBytes];  // 64 KiB

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

  // Staging: instruction i of thread tid covers row 16*i + tid/16, chunk tid%16
  // (a wave instruction = 4 whole rows = 1 KiB, lane-contiguous).
  const int srow = tid >> 4, schunk = tid & 15;
  u32x4 kreg[4], vreg[4];
  auto gload = [&](int tile) {
    const int kv0 = tile * kBN;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int p = kv0 + 16 * i + srow;
      p = p < kv_len ? p : kv_len - 1;  // rows past kv_len are masked or unused
      kreg[i] = load16(kh + (size_t)p * kHeadDim + schunk * 8);
      vreg[i] = load16(vh + (size_t)p * kHeadDim + schunk * 8);
    }
  };
  auto lds_store = [&](unsigned char* st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * i + srow;
      *reinterpret_cast<u32x4*>(st + pswz(row, schunk)) = kreg[i];
      *reinterpret_cast<u32x4*>(st + kTileHalfBytes + pswz(row, schunk)) = vreg[i];
    }
  };

  gload(0);
  lds_store(smem);
  if (ntiles > 1) gload(1);
  __syncthreads();

  for (int tile = 0; tile < ntiles; ++tile) {
    const unsigned char* kst = smem + (tile & 1) * kStageBytes;
    const unsigned char* vst = kst + kTileHalfBytes;
    const int kv0 = tile * kBN;

    floatx4 sc[2][4];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      half8 kf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kf[c] = as_half8(*reinterpret_cast<const u32x4*>(kst + pswz(16 * pb + col, 4 * c + kb)));
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
    bool grew = false;
    float alpha[2];
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
      grew |= mnew > m[mb];
      alpha[mb] = fast_exp2(m[mb] - mnew);
      float psum = 0.f;
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(sc[mb][pb][i] * scale_log2 - mnew);
          psum += p;
          pf[mb][pb >> 1][(pb & 1) * 4 + i] = (half_t)p;
        }
      l[mb] = l[mb] * alpha[mb] + psum;
      m[mb] = mnew;
    }
    if (__any(grew)) {  // wave-uniform: skip the rescale when no max moved
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[mb][db] *= alpha[mb];
    }

#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        // V^T fragment rows d = 16db + col, slots (kb, 0..7) = positions
        // 32cc + {4kb..4kb+3, 16+4kb..16+4kb+3}: lane j of the 16-lane group
        // addresses row 32cc + 16h + 4kb + j/4, d-chunk 16db + 4(j%4).
        const int j = col;
        const int cbyte = 32 * db + 8 * (j & 3);
        const int r0 = 32 * cc + 4 * kb + (j >> 2);
        const half4 lo = lds_read_tr16(vst + pswz(r0, cbyte >> 4) + (cbyte & 15));
        const half4 hi = lds_read_tr16(vst + pswz(r0 + 16, cbyte >> 4) + (cbyte & 15));
        const half8 vf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) acc[mb][db] = mfma16x16x32(vf, pf[mb][cc], acc[mb][db]);
      }

    // Stage tile+1 into the other buffer (its last readers finished before the
    // barrier that ended the previous iteration), then prefetch tile+2.
    if (tile + 1 < ntiles) {
      lds_store(smem + ((tile + 1) & 1) * kStageBytes);
      if (tile + 2 < ntiles) gload(tile + 2);
    }
    __syncthreads();
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
