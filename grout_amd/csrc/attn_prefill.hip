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
//    loads and stored row-major into double-buffered LDS with padded rows
//    (K: 272 B, V: 288 B).  The padding makes both fragment reads
//    bank-conflict free (16 K rows of one 16-byte chunk shift by one chunk per
//    row; the transposing V reads touch 8 rows x 2 chunks that shift by two
//    chunks per row) and keeps every per-tile LDS offset a compile-time
//    immediate on a per-lane base.  The next tile is in flight while the
//    current one is computed, with one workgroup barrier per tile;
//  * S^T = K.Q^T (A = K rows from LDS, B = Q held in VGPRs for the whole
//    loop) and O^T = V^T.P^T: the V^T fragments come straight from the
//    row-major tile with ds_read_b64_tr_b16 (gfx950's transposing LDS read),
//    P comes from the S^T accumulators without any shuffle, and each query
//    row is one lane column, so its softmax statistics live in the lanes that
//    own its accumulator;
//  * lazy rescale: a row's running max only moves when the tile's max
//    exceeds it by more than kRescaleThreshold (log2 units), so p stays
//    <= 2^8 (exact in f16, harmless in the fp32 accumulators) and the
//    accumulator rescale is skipped on almost every tile after the first;
//  * the softmax row sums come from the MFMA unit (an all-ones A fragment
//    against the P fragment), not from VALU adds and cross-lane reductions;
//  * causal: tiles past the workgroup's last query are skipped, masks are
//    applied only on tiles crossing the diagonal;
//  * scheduling: block id -> (kv head = id mod Hkv, q block): the first half
//    of the grid takes the heavy q blocks in decreasing order, the second half
//    their complements, so co-resident workgroups balance each CU; with
//    Hkv = 8 each XCD's L2 holds one kv head's K/V.
#include "common.hpp"
#include "kernels.hpp"

namespace grout {

constexpr int kBN = 64;  // kv positions per tile
constexpr float kRescaleThreshold = 8.0f;
constexpr int kRowsPerWG = 128;
constexpr int kKRow = 272;                      // K row stride in LDS (256 B + 1 chunk)
constexpr int kVRow = 288;                      // V row stride in LDS (256 B + 2 chunks)
constexpr int kKBytes = kBN * kKRow;            // 17 KiB
constexpr int kStageBytes = kKBytes + kBN * kVRow;  // 35 KiB: K + V of one tile

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;

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
  // Two K slots and two V slots.  Iteration t reads K(t+1) and V(t); it
  // stages K(t+2) into the K slot read in iteration t-1 and V(t+1) into the V
  // slot read in iteration t-1, so one barrier per iteration suffices.
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * kStageBytes];
  unsigned char* const kslot0 = smem;
  unsigned char* const vslot0 = smem + 2 * kKBytes;
  constexpr int kVBytes = kStageBytes - kKBytes;

  const int G = Hq / Hkv;
  const int nsub = G / HG;
  const int bid = blockIdx.x;
  const int kvh = bid % Hkv;
  const int rest = bid / Hkv;
  const int hsub = rest % nsub;
  // Causal work grows with the q block.  Blocks r and r + ceil(nqb/2) of a kv
  // head take complementary q blocks (nqb-1-r and r); the heavy half is
  // dispatched first, so co-resident workgroups balance each CU's load.
  const int r = rest / nsub, half_q = (nqb + 1) / 2;
  const int qb = r < half_q ? nqb - 1 - r : r - half_q;
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
    const int rr = 32 * w + 16 * mb + col;
    qrow[mb] = q0 + rr / HG;
    qhead[mb] = kvh * G + hsub * HG + rr % HG;
    rvalid[mb] = rr < BQ * HG && qrow[mb] < S;
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

  // m: running max (log2 units) of row `col` of each block; lacc: its sum of
  // p (every element of the C fragment holds it); acc: O^T fragments.
  float m[2] = {-1.0e30f, -1.0e30f};
  floatx4 lacc[2], acc[2][8];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    lacc[mb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[mb][db] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  const half8 ones = {(half_t)1.f, (half_t)1.f, (half_t)1.f, (half_t)1.f,
                      (half_t)1.f, (half_t)1.f, (half_t)1.f, (half_t)1.f};

  // Staging: instruction i of thread tid covers row 16*i + tid/16, chunk
  // tid%16 (a wave instruction = 4 whole rows = 1 KiB, lane-contiguous).
  const int srow = tid >> 4, schunk = tid & 15;
  auto gload_rows = [&](const half_t* base, int tile, u32x4 (&reg)[4]) {
    const int kv0 = tile * kBN;
    if (kv0 + kBN <= kv_len) {  // full tile: one base, constant offsets
      const half_t* p = base + (size_t)(kv0 + srow) * kHeadDim + schunk * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i) reg[i] = load16(p + 16 * i * kHeadDim);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int pr = kv0 + 16 * i + srow;
        pr = pr < kv_len ? pr : kv_len - 1;  // rows past kv_len are masked or unused
        reg[i] = load16(base + (size_t)pr * kHeadDim + schunk * 8);
      }
    }
  };
  auto store_rows = [&](unsigned char* slot, int row_bytes, const u32x4 (&reg)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4*>(slot + (16 * i + srow) * row_bytes + schunk * 16) = reg[i];
  };
  // Per-lane LDS bases of the fragment reads (all other terms are immediates):
  //  K fragment (pb, c): row 16pb + col, 16-byte chunk 4c + kb;
  //  V^T fragment (cc, db, half h): lane j of its 16-lane group addresses row
  //  32cc + 16h + 4kb + j/4 at d = 16db + 4(j%4).
  const int kfrag_base = col * kKRow + kb * 16;
  const int vfrag_base = (4 * kb + (col >> 2)) * kVRow + 8 * (col & 3);

  auto qk = [&](const unsigned char* kslot, floatx4 (&sc)[2][4]) {
    const unsigned char* kst = kslot + kfrag_base;
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      half8 kf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kf[c] = as_half8(*reinterpret_cast<const u32x4*>(kst + 16 * pb * kKRow + 64 * c));
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        floatx4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) a = mfma16x16x32(kf[c], qf[mb][c], a);
        sc[mb][pb] = a;
      }
    }
  };
  // Row maxima of a score tile (masked first when it crosses the diagonal).
  // Returns whether any row of the wave must move its running max.
  auto tile_max = [&](floatx4 (&sc)[2][4], int tile, float (&tmax)[2]) -> bool {
    const int kv0 = tile * kBN;
    bool need = false;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      if (kv0 + kBN - 1 > first_masked_kv) {
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int pos = kv0 + 16 * pb + 4 * kb + i;
            if (pos > qpos[mb]) sc[mb][pb][i] = -1.0e30f;
          }
      }
      float t = -1.0e30f;
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int i = 0; i < 4; ++i) t = fmaxf(t, sc[mb][pb][i]);
      t = fmaxf(t, shfl_xor(t, 16));
      t = fmaxf(t, shfl_xor(t, 32));
      tmax[mb] = t * scale_log2;
      need |= tmax[mb] > m[mb] + kRescaleThreshold;
    }
    return __any(need);
  };
  auto probs = [&](const floatx4 (&sc)[2][4], half8 (&pf)[2][2]) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          pf[mb][pb >> 1][(pb & 1) * 4 + i] =
              (half_t)fast_exp2(sc[mb][pb][i] * scale_log2 - m[mb]);
  };
  auto pv = [&](const unsigned char* vslot, const half8 (&pf)[2][2]) {
    const unsigned char* vst = vslot + vfrag_base;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        // V^T fragment rows d = 16db + col, slots (kb, 0..7) = positions
        // 32cc + {4kb..4kb+3, 16+4kb..16+4kb+3}.
        const half4 lo = lds_read_tr16(vst + 32 * cc * kVRow + 32 * db);
        const half4 hi = lds_read_tr16(vst + (32 * cc + 16) * kVRow + 32 * db);
        const half8 vf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) acc[mb][db] = mfma16x16x32(vf, pf[mb][cc], acc[mb][db]);
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) lacc[mb] = mfma16x16x32(ones, pf[mb][cc], lacc[mb]);
    }
  };
  auto rescale = [&](const float (&tmax)[2]) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const float mnew = fmaxf(m[mb], tmax[mb]);
      const float alpha = fast_exp2(m[mb] - mnew);
      m[mb] = mnew;
      lacc[mb] *= alpha;
#pragma unroll
      for (int db = 0; db < 8; ++db) acc[mb][db] *= alpha;
    }
  };

  // ---- prologue: K0, V0 -> slot 0, K1 -> K slot 1; S(0) and P(0) ----
  u32x4 kreg[4], vreg[4];
  gload_rows(kh, 0, kreg);
  gload_rows(vh, 0, vreg);
  store_rows(kslot0, kKRow, kreg);
  store_rows(vslot0, kVRow, vreg);
  if (ntiles > 1) {
    gload_rows(kh, 1, kreg);
    store_rows(kslot0 + kKBytes, kKRow, kreg);
  }
  __syncthreads();

  half8 pf[2][2];
  {
    floatx4 sc[2][4];
    float tmax[2];
    qk(kslot0, sc);
    if (tile_max(sc, 0, tmax)) rescale(tmax);
    probs(sc, pf);
  }
  __syncthreads();  // K slot 0 is restaged in iteration 0

  // Iteration t: phase A computes S(t+1) from K slot (t+1)&1 while V(t+1) is
  // in flight to registers, then stages it into V slot (t+1)&1; phase B
  // accumulates P(t).V(t) from V slot t&1 and turns S(t+1) into P(t+1) while
  // K(t+2) is in flight, then stages it into K slot t&1.  Each staged slot
  // was last read in iteration t-1, so one barrier per iteration suffices.
  for (int t = 0; t < ntiles; ++t) {
    if (t + 1 < ntiles) {
      gload_rows(vh, t + 1, vreg);
      floatx4 sc[2][4];
      float tmax[2];
      qk(kslot0 + ((t + 1) & 1) * kKBytes, sc);
      const bool need = tile_max(sc, t + 1, tmax);
      store_rows(vslot0 + ((t + 1) & 1) * kVBytes, kVRow, vreg);
      if (t + 2 < ntiles) gload_rows(kh, t + 2, kreg);
      // P(t).V(t) and the softmax of tile t+1 do not depend on each other:
      // the exponentials overlap the MFMAs.
      pv(vslot0 + (t & 1) * kVBytes, pf);
      if (need) rescale(tmax);
      probs(sc, pf);
      if (t + 2 < ntiles) store_rows(kslot0 + (t & 1) * kKBytes, kKRow, kreg);
    } else {
      pv(vslot0 + (t & 1) * kVBytes, pf);
    }
    __syncthreads();
  }

#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    if (!rvalid[mb]) continue;
    const float inv = 1.0f / lacc[mb][0];
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
