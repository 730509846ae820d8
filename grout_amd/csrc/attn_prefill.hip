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
constexpr int kRowBytes = kHeadDim * 2;        // 256 B: one K or V row
constexpr int kTileBytes = kBN * kRowBytes;     // 16 KiB: one K or V tile

// LDS swizzle of a 256-byte row: 16-byte chunk j of row r is stored at chunk
// j ^ swz(r).  swz is a bijection on r % 16 (16 K rows reading one chunk hit 16
// different chunks) and swz(r) >> 1 = r % 8 (8 consecutive V rows reading one
// chunk pair hit 8 different pairs), so both fragment reads are conflict free.
__device__ __forceinline__ int swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;
typedef __attribute__((address_space(3))) void lds_void;

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

// Schedule of the P(t).V(t) + softmax(t+1) block: 36 MFMAs (32 P.V, 4 row
// sums), 32 transposing LDS reads and about 80 VALU instructions (32 fma, 32
// exp2, 16 packs).  Four reads go first; then each MFMA is followed by one
// read and two VALU instructions, so one wave keeps both units busy.
__device__ __forceinline__ void interleave_pv_softmax() {
#ifndef GROUT_PREFILL_NO_INTERLEAVE
  __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
  for (int i = 0; i < 28; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
  }
#endif
}

template <int HG>
__global__ __launch_bounds__(256, 2) void fmha_prefill_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k_cache,
    const half_t* __restrict__ v_cache, half_t* __restrict__ out, int S, int pos0, int Hq,
    int Hkv, long head_stride, float scale_log2, int nqb) {
  constexpr int BQ = kRowsPerWG / HG;
  // Two K slots and two V slots, each its own LDS object: the compiler then
  // knows that the direct-to-LDS loads filling one slot do not alias the
  // fragment reads of another and lets them stay in flight.
  __shared__ __attribute__((aligned(1024))) unsigned char s_k0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_k1[kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_v0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_v1[kTileBytes];

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
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, kb = lane >> 4;

  const unsigned char* kh = reinterpret_cast<const unsigned char*>(k_cache + (size_t)kvh * head_stride);
  const unsigned char* vh = reinterpret_cast<const unsigned char*>(v_cache + (size_t)kvh * head_stride);
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

  // Staging with global_load_lds: wave instruction i of wave w writes the
  // 1 KiB of LDS holding tile rows 16w + 4i .. +3, lane l at byte 16*l, i.e.
  // row 16w + 4i + l/16, stored chunk l%16, which holds logical chunk
  // (l%16) ^ swz(row).  Each 16-lane group reads one whole 256-byte row.
  int dma_row[4], dma_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    dma_row[i] = 16 * w + 4 * i + kb;
    dma_off[i] = dma_row[i] * kRowBytes + ((col ^ swz(dma_row[i])) << 4);
  }
  auto dma_tile = [&](const unsigned char* base, int tile, unsigned char* slot) {
    const int kv0 = tile * kBN;
    if (kv0 + kBN <= kv_len) {
      const unsigned char* p = base + (size_t)kv0 * kRowBytes;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // Opaque to the optimizer, so the per-lane 64-bit sum is not hoisted
        // out of the loop: a scalar base plus a 32-bit lane offset instead.
        unsigned o = (unsigned)dma_off[i];
        asm volatile("" : "+v"(o));
        __builtin_amdgcn_global_load_lds(p + o, (lds_void*)(slot + (4 * w + i) * 1024), 16, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // rows past kv_len repeat the last row: masked for K, zero weight for V
        unsigned o = (unsigned)dma_off[i];
        asm volatile("" : "+v"(o));
        const int pr = min(kv0 + dma_row[i], kv_len - 1);
        const unsigned char* p = base + (size_t)pr * kRowBytes + (o & 255u);
        __builtin_amdgcn_global_load_lds(p, (lds_void*)(slot + (4 * w + i) * 1024), 16, 0, 0);
      }
    }
  };
  // Per-lane LDS offsets of the fragment reads; row offsets are immediates.
  //  K fragment (pb, c): row 16pb + col, logical chunk 4c + kb;
  //  V^T fragment (cc, db, half h): lane j of its 16-lane group addresses row
  //  32cc + 16h + 4kb + j/4 at d = 16db + 4(j%4), i.e. logical chunk
  //  2db + (j%4)/2, byte 8*(j%2) inside it.
  int kfrag[4], vfrag[8];
#pragma unroll
  for (int c = 0; c < 4; ++c) kfrag[c] = col * kRowBytes + (((4 * c + kb) ^ swz(col)) << 4);
  {
    const int vr = 4 * kb + (col >> 2), e = col & 3;
#pragma unroll
    for (int db = 0; db < 8; ++db)
      vfrag[db] = vr * kRowBytes + (((2 * db + (e >> 1)) ^ swz(vr)) << 4) + ((e & 1) << 3);
  }

  auto qk = [&](const unsigned char* kslot, floatx4 (&sc)[2][4]) {
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      half8 kf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kf[c] = as_half8(*reinterpret_cast<const u32x4*>(kslot + kfrag[c] + 16 * pb * kRowBytes));
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
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        // V^T fragment rows d = 16db + col, slots (kb, 0..7) = positions
        // 32cc + {4kb..4kb+3, 16+4kb..16+4kb+3}.
        const half4 lo = lds_read_tr16(vslot + vfrag[db] + 32 * cc * kRowBytes);
        const half4 hi = lds_read_tr16(vslot + vfrag[db] + (32 * cc + 16) * kRowBytes);
        const half8 vf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) acc[mb][db] = mfma16x16x32(vf, pf[mb][cc], acc[mb][db]);
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) lacc[mb] = mfma16x16x32(ones, pf[mb][cc], lacc[mb]);
    }
  };
  // Moves the running max to max(m, tmax); what was accumulated against the
  // old max (acc, lacc and the not yet applied P(t)) is scaled by alpha.
  auto rescale = [&](const float (&tmax)[2], half8 (&pf)[2][2]) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const float mnew = fmaxf(m[mb], tmax[mb]);
      const float alpha = fast_exp2(m[mb] - mnew);
      m[mb] = mnew;
      lacc[mb] *= alpha;
#pragma unroll
      for (int db = 0; db < 8; ++db) acc[mb][db] *= alpha;
      const half_t ah = (half_t)alpha;
      pf[mb][0] *= ah;
      pf[mb][1] *= ah;
    }
  };
  // ---- prologue: K0 -> s_k0, V0 -> s_v0, K1 -> s_k1; S(0) and P(0) ----
  dma_tile(kh, 0, s_k0);
  dma_tile(vh, 0, s_v0);
  if (ntiles > 1) dma_tile(kh, 1, s_k1);
  __syncthreads();

  half8 pf[2][2];
  {
    floatx4 sc[2][4];
    float tmax[2];
    qk(s_k0, sc);
    if (tile_max(sc, 0, tmax)) rescale(tmax, pf);  // acc and pf are still zero
    probs(sc, pf);
  }
  __syncthreads();  // s_k0 is refilled in iteration 0

  // Iteration t reads K(t+1) and V(t) and, from its start, has V(t+1) and
  // K(t+2) in flight into the two slots last read in iteration t-1; the
  // barrier that ends the iteration waits for them.  S(t+1) comes first, so
  // P(t).V(t) and the softmax of tile t+1 are independent work.
  auto step = [&](int t, const unsigned char* kread, const unsigned char* vread,
                  unsigned char* vfill, unsigned char* kfill) {
    if (t + 1 < ntiles) dma_tile(vh, t + 1, vfill);
    if (t + 2 < ntiles) dma_tile(kh, t + 2, kfill);
    if (t + 1 < ntiles) {
      floatx4 sc[2][4];
      float tmax[2];
      qk(kread, sc);
      if (tile_max(sc, t + 1, tmax)) rescale(tmax, pf);
      // P(t).V(t) and the softmax of tile t+1 are independent: one basic
      // block whose schedule puts the exponentials under the MFMAs.
      half8 pn[2][2];
      pv(vread, pf);
      probs(sc, pn);
      interleave_pv_softmax();
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        pf[mb][0] = pn[mb][0];
        pf[mb][1] = pn[mb][1];
      }
    } else {
      pv(vread, pf);
    }
    __syncthreads();
  };
  for (int t = 0; t < ntiles; t += 2) {
    step(t, s_k1, s_v0, s_v1, s_k0);
    if (t + 1 < ntiles) step(t + 1, s_k0, s_v1, s_v0, s_k1);
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
