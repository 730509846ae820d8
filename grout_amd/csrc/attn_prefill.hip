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

#include <cstdlib>

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

// Schedule of the S(t+1) block: 16 K-fragment reads, 32 MFMAs and the 8
// direct-to-LDS loads of the next tiles, one load after every two MFMAs.
__device__ __forceinline__ void interleave_qk_dma() {
  __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
}

// One kernel, two work splits.
//  TEAMS = 1: a 4-wave workgroup owns one q block (128 rows) and walks its
//    causal kv tiles.
//  TEAMS = 2: an 8-wave workgroup owns the complementary pair of q blocks
//    h = nqb-1-r and l = r; team A (waves 0-3) takes tiles [0, a) of h, team
//    B (waves 4-7) all tiles of l and then tiles [a, T_h) of h, with
//    a = ceil((T_h + T_l) / 2), so the two teams do the same number of tiles
//    and every workgroup the same work.  B's partial (m, l, acc) of h is merged
//    into A's through LDS at the end.  The teams iterate in lockstep, one
//    shared barrier per tile.
template <int HG, int TEAMS>
__global__ __launch_bounds__(256 * TEAMS, 2 / TEAMS) void fmha_prefill_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k_cache,
    const half_t* __restrict__ v_cache, half_t* __restrict__ out, int S, int pos0, int Hq,
    int Hkv, long head_stride, float scale_log2, int nqb) {
  constexpr int BQ = kRowsPerWG / HG;
  // Per team: two K slots and two V slots, each slot its own LDS object, so
  // the compiler knows that the direct-to-LDS loads filling one slot do not
  // alias the fragment reads of another and lets them stay in flight.
  __shared__ __attribute__((aligned(1024))) unsigned char s_k0[TEAMS][kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_k1[TEAMS][kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_v0[TEAMS][kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_v1[TEAMS][kTileBytes];

  const int G = Hq / Hkv;
  const int nsub = G / HG;
  const int bid = blockIdx.x;
  const int kvh = bid % Hkv;
  const int rest = bid / Hkv;
  const int hsub = rest % nsub;
  const int r = rest / nsub;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int team = TEAMS == 2 ? wave >> 2 : 0;
  const int w = wave & 3;
  const int col = lane & 15, kb = lane >> 4;

  auto tiles_of = [&](int qb) __attribute__((always_inline)) {
    const int q_last = min(qb * BQ + BQ, S) - 1;
    return (pos0 + q_last + 1 + kBN - 1) / kBN;
  };
  // This team's kv tile sequence: n0 tiles of q block qb0 from tile tb0, then
  // n1 tiles of q block qb1 from tile tb1.
  int qb0, tb0 = 0, n0, qb1, tb1 = 0, n1 = 0, nloop, a_split = 0;
  bool merge_h = false;    // team B holds part of block h (workgroup-uniform)
  bool has_switch = false;  // team B moves from block l to block h (workgroup-uniform)
  int switch_after = 0;     // ... after this many iterations (workgroup-uniform)
  if (TEAMS == 1) {
    // Blocks r and r + ceil(nqb/2) of a kv head take complementary q blocks;
    // the heavy half is dispatched first.
    const int half_q = (nqb + 1) / 2;
    qb0 = r < half_q ? nqb - 1 - r : r - half_q;
    qb1 = qb0;
    n0 = tiles_of(qb0);
    nloop = n0;
  } else {
    const int h = nqb - 1 - r, l = r;
    const int th = tiles_of(h), tl = h != l ? tiles_of(l) : 0;
    a_split = (th + tl + 1) / 2;
    merge_h = a_split < th;
    has_switch = tl > 0 && merge_h;
    switch_after = tl;
    if (team == 0) {
      qb0 = h; n0 = a_split; qb1 = h;
    } else {
      qb0 = l; n0 = tl; qb1 = h; tb1 = a_split; n1 = th - a_split;
    }
    nloop = a_split;  // team B has th + tl - a_split <= a_split tiles
  }
  const int n = n0 + n1;
  auto tile_at = [&](int j) __attribute__((always_inline)) { return j < n0 ? tb0 + j : tb1 + (j - n0); };

  const unsigned char* kh = reinterpret_cast<const unsigned char*>(k_cache + (size_t)kvh * head_stride);
  const unsigned char* vh = reinterpret_cast<const unsigned char*>(v_cache + (size_t)kvh * head_stride);
  const int kv_len = pos0 + S;

  // Team t's slots sit t * kTileBytes above team 0's in every slot array;
  // that offset is folded into the per-lane addresses below, so the slot
  // arrays themselves stay compile-time constants (immediate offsets).
  const int team_off = team * kTileBytes;
  unsigned char* const k0 = s_k0[0];
  unsigned char* const k1 = s_k1[0];
  unsigned char* const v0 = s_v0[0];
  unsigned char* const v1 = s_v1[0];

  // Row rr = 32w + 16mb + col of a q block is query position qb*BQ + rr/HG of
  // head kvh*G + hsub*HG + rr%HG.
  auto row_pos = [&](int qb, int mb) __attribute__((always_inline)) { return qb * BQ + (32 * w + 16 * mb + col) / HG; };
  auto row_head = [&](int mb) __attribute__((always_inline)) { return kvh * G + hsub * HG + (32 * w + 16 * mb + col) % HG; };
  auto row_valid = [&](int qb, int mb) __attribute__((always_inline)) {
    return 32 * w + 16 * mb + col < BQ * HG && row_pos(qb, mb) < S;
  };
  int qpos[2];
  int first_masked_kv;  // a tile needs masking if it reaches past this
  half8 qf[2][4];
  auto load_q = [&](int qb) __attribute__((always_inline)) {
    first_masked_kv = pos0 + qb * BQ;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      qpos[mb] = pos0 + row_pos(qb, mb);
      const bool valid = row_valid(qb, mb);
      const half_t* qr = q + ((size_t)row_pos(qb, mb) * Hq + row_head(mb)) * kHeadDim + kb * 8;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        qf[mb][c] = valid ? as_half8(load16(qr + c * 32)) : as_half8(u32x4{0u, 0u, 0u, 0u});
    }
  };

  // m: running max (log2 units) of row `col` of each block; lacc: its sum of
  // p (every element of the C fragment holds it); acc: O^T fragments.  m
  // starts finite and masked scores are -inf, so a row whose tiles so far are
  // all masked keeps p = 0 (exp2(-inf)) instead of exp2(0).
  float m[2];
  floatx4 lacc[2], acc[2][8];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    m[mb] = -1.0e30f;
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
  // Row 16w + 4i + kb has swizzle swz(4i + kb).
  const int dma_row0 = 16 * w + kb;
  int dma_chunk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) dma_chunk[i] = (col ^ swz(4 * i + kb)) << 4;
  // Rows are clamped to kv_len - 1 (past the end they are masked for K and
  // get zero weight for V); the code has no branch, so it can share a basic
  // block, and hence an instruction schedule, with the MFMAs.
  auto dma_tile = [&](const unsigned char* base, int tile, unsigned char* slot) __attribute__((always_inline)) {
    const int kv0 = tile * kBN;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // Opaque to the optimizer, so no per-lane 64-bit address is hoisted
      // out of the loop: a scalar base plus a 32-bit lane offset instead.
      unsigned o = (unsigned)dma_chunk[i];
      asm volatile("" : "+v"(o));
      const int pr = min(kv0 + dma_row0 + 4 * i, kv_len - 1);
      const unsigned char* p = base + ((unsigned)pr * kRowBytes + o);  // < 2^32: rows*256 B
      __builtin_amdgcn_global_load_lds(p, (lds_void*)(slot + team_off + (4 * w + i) * 1024),
                                       16, 0, 0);
    }
  };
  // Per-lane LDS offsets of the fragment reads; row offsets are immediates.
  //  K fragment (pb, c): row 16pb + col, logical chunk 4c + kb;
  //  V^T fragment (cc, db, half h): lane j of its 16-lane group addresses row
  //  32cc + 16h + 4kb + j/4 at d = 16db + 4(j%4), i.e. logical chunk
  //  2db + (j%4)/2, byte 8*(j%2) inside it.
  int kfrag[4], vfrag[8];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    kfrag[c] = team_off + col * kRowBytes + (((4 * c + kb) ^ swz(col)) << 4);
  {
    const int vr = 4 * kb + (col >> 2), e = col & 3;
#pragma unroll
    for (int db = 0; db < 8; ++db)
      vfrag[db] = team_off + vr * kRowBytes + (((2 * db + (e >> 1)) ^ swz(vr)) << 4) +
                  ((e & 1) << 3);
  }

  auto qk = [&](const unsigned char* kslot, floatx4 (&sc)[2][4]) __attribute__((always_inline)) {
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
  auto tile_max = [&](floatx4 (&sc)[2][4], int tile, float (&tmax)[2]) __attribute__((always_inline)) -> bool {
    const int kv0 = tile * kBN;
    bool need = false;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      if (kv0 + kBN - 1 > first_masked_kv) {
        // element (pb, i) is kv position kv0 + 4kb + 16pb + i: compare the
        // immediate 16pb + i against one per-lane limit
        const int lim = qpos[mb] - kv0 - 4 * kb;
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (16 * pb + i > lim) sc[mb][pb][i] = -__builtin_inff();
      }
      float t = -__builtin_inff();
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
  auto probs = [&](const floatx4 (&sc)[2][4], half8 (&pf)[2][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          pf[mb][pb >> 1][(pb & 1) * 4 + i] =
              (half_t)fast_exp2(sc[mb][pb][i] * scale_log2 - m[mb]);
  };
  auto pv = [&](const unsigned char* vslot, const half8 (&pf)[2][2]) __attribute__((always_inline)) {
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
  // Moves the running max to max(m, tmax) for rows that saw a finite score;
  // what was accumulated against the old max (acc, lacc and the not yet
  // applied P(t)) is scaled by alpha.
  auto rescale = [&](const float (&tmax)[2], half8 (&pf)[2][2]) __attribute__((always_inline)) {
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
  auto write_out = [&](int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      if (!row_valid(qb, mb)) continue;
      const float inv = 1.0f / lacc[mb][0];
      half_t* orow = out + ((size_t)row_pos(qb, mb) * Hq + row_head(mb)) * kHeadDim;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        half4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (half_t)(acc[mb][db][i] * inv);
        *reinterpret_cast<u32x2*>(orow + 16 * db + 4 * kb) = __builtin_bit_cast(u32x2, o);
      }
    }
  };

  // ---- prologue: K(0) -> k0, V(0) -> v0, K(1) -> k1; S(0) and P(0) ----
  // (for team B with a block-l segment, its first segment only)
  // Both teams must run the same barriers, so the switch point is a property
  // of the workgroup, not of the team.
  const int n_first = team == 1 && has_switch ? switch_after : n;  // tiles before the switch
  half8 pf[2][2];
  if (n > 0) {
    dma_tile(kh, tile_at(0), k0);
    dma_tile(vh, tile_at(0), v0);
    if (n_first > 1) dma_tile(kh, tile_at(1), k1);
    load_q(n0 > 0 ? qb0 : qb1);
  }
  __syncthreads();
  if (n > 0) {
    floatx4 sc[2][4];
    float tmax[2];
    qk(k0, sc);
    if (tile_max(sc, tile_at(0), tmax)) rescale(tmax, pf);  // acc is zero, pf not yet set
    probs(sc, pf);
  }
  __syncthreads();  // k0 is refilled in iteration 0

  // Iteration j reads K(j+1) and V(j) and, from its start, has V(j+1) and
  // K(j+2) in flight into the two slots last read in iteration j-1; the
  // barrier that ends the iteration waits for them.  S(j+1) comes first, so
  // P(j).V(j) and the softmax of tile j+1 are independent work.  nn is the
  // length of the team's current tile run.
  auto step = [&](int j, int nn, const unsigned char* kread, const unsigned char* vread,
                  unsigned char* vfill, unsigned char* kfill) __attribute__((always_inline)) {
    if (j + 1 < nn) {
      floatx4 sc[2][4];
      float tmax[2];
      // The eight loads spread over the S MFMAs instead of queueing behind
      // one another at the top of the iteration.  Past the last tile the K
      // load repeats it into a slot that is not read again.
      dma_tile(kh, tile_at(min(j + 2, nn - 1)), kfill);
      dma_tile(vh, tile_at(j + 1), vfill);
      qk(kread, sc);
      interleave_qk_dma();
      if (tile_max(sc, tile_at(j + 1), tmax)) rescale(tmax, pf);
      // P(j).V(j) and the softmax of tile j+1 are independent: one basic
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
    } else if (j + 1 == nn) {
      pv(vread, pf);
    }
    __syncthreads();
  };
  // Team B's move from block l to the tail of block h, run between
  // iterations js = switch_after - 1 and js + 1 (both teams take part in its
  // two barriers).  After iteration js the slots K (js+1)&1, K js&1 and
  // V (js+1)&1 are free; iteration js+1 reads K(js+2) from K slot js&1 and
  // V(js+1) from V slot (js+1)&1, and refills K slot (js+1)&1.
  auto team_switch = [&](int js, unsigned char* kcur, unsigned char* knext,
                         unsigned char* vcur) __attribute__((always_inline)) {
    if (team == 1) {
      write_out(qb0);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        m[mb] = -1.0e30f;
        lacc[mb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[mb][db] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
      dma_tile(kh, tile_at(js + 1), kcur);
      dma_tile(vh, tile_at(js + 1), vcur);
      if (n1 > 1) dma_tile(kh, tile_at(js + 2), knext);
      load_q(qb1);
    }
    __syncthreads();
    if (team == 1) {
      floatx4 sc[2][4];
      float tmax[2];
      qk(kcur, sc);
      if (tile_max(sc, tile_at(js + 1), tmax)) rescale(tmax, pf);
      probs(sc, pf);
    }
    __syncthreads();  // K slot (js+1)&1 is refilled in iteration js+1
  };
  // Slots by parity: even j reads K slot 1 / V slot 0, odd j the others;
  // two sequential calls per trip (an if/else would be merged into one copy
  // with runtime slot pointers).  Team B's run before the switch is
  // switch_after tiles long.
  const int js = has_switch ? switch_after - 1 : -2;
  for (int j = 0; j < nloop; j += 2) {
    if (j == js + 1) team_switch(js, k0, k1, v0);  // js odd: (js+1)&1 = 0
    step(j, team == 1 && j <= js ? n_first : n, k1, v0, v1, k0);
    if (j + 1 < nloop) {
      if (j + 1 == js + 1) team_switch(js, k1, k0, v1);  // js even
      step(j + 1, team == 1 && j + 1 <= js ? n_first : n, k0, v1, v0, k1);
    }
  }

  if (TEAMS == 1 || !merge_h) {
    // every team finished whole q blocks
    if (n > 0) write_out(n1 > 0 ? qb1 : qb0);
    return;
  }
  // Team B holds tiles [a, T_h) of block h: its (m, l, acc) go through LDS
  // (its own K/V slots take acc, team A's first K slot takes m and l) and
  // team A combines them with its own tiles [0, a).  Same wave index, same
  // lane: same rows and columns.
  unsigned char* const accbuf = w == 0 ? s_k0[TEAMS - 1] : w == 1 ? s_k1[TEAMS - 1]
                              : w == 2 ? s_v0[TEAMS - 1] : s_v1[TEAMS - 1];
  float* const mlbuf = reinterpret_cast<float*>(s_k0[0] + w * 1024) + lane * 4;
  if (team == 1) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int db = 0; db < 8; ++db)
        *reinterpret_cast<floatx4*>(accbuf + ((mb * 8 + db) * 64 + lane) * 16) = acc[mb][db];
    *reinterpret_cast<floatx4*>(mlbuf) = floatx4{m[0], m[1], lacc[0][0], lacc[1][0]};
  }
  __syncthreads();
  if (team == 0) {
    const floatx4 mlb = *reinterpret_cast<const floatx4*>(mlbuf);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const float mn = fmaxf(m[mb], mlb[mb]);
      const float sa = fast_exp2(m[mb] - mn), sb = fast_exp2(mlb[mb] - mn);
      lacc[mb] = lacc[mb] * sa + mlb[2 + mb] * sb;
#pragma unroll
      for (int db = 0; db < 8; ++db)
        acc[mb][db] = acc[mb][db] * sa +
                      *reinterpret_cast<const floatx4*>(accbuf + ((mb * 8 + db) * 64 + lane) * 16) * sb;
    }
    write_out(qb0);
  }
}

static int prefill_teams_override() {
  const char* e = std::getenv("GROUT_FMHA_PREFILL_TEAMS");
  return e ? std::atoi(e) : 0;
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
  // Balanced pairs (TEAMS = 2) pay off when they make one to two rounds of
  // 8-wave workgroups on the 256 CUs: fewer pairs leave CUs idle, more
  // rounds let the dispatcher balance single q blocks by itself.  With
  // 16-row head groups (HG = 8) the single-block split measured faster.
  const unsigned pair_blocks = (unsigned)(((nqb + 1) / 2) * Hkv * (G / HG));
  int teams = pair_blocks >= 256 && pair_blocks <= 512 && HG <= 4 ? 2 : 1;
  if (const int o = prefill_teams_override(); o == 1 || o == 2) teams = o;
  const unsigned blocks = teams == 2 ? pair_blocks : (unsigned)(nqb * Hkv * (G / HG));
#define GROUT_PREFILL_CASE(hg)                                                              \
  case hg:                                                                                  \
    if (teams == 2)                                                                         \
      fmha_prefill_kernel<hg, 2><<<blocks, 512, 0, stream>>>(                              \
          (const half_t*)q, (const half_t*)k_cache, (const half_t*)v_cache, (half_t*)out,   \
          seq_len, pos0, Hq, Hkv, head_stride, scale_log2, nqb);                            \
    else                                                                                    \
      fmha_prefill_kernel<hg, 1><<<blocks, 256, 0, stream>>>(                              \
          (const half_t*)q, (const half_t*)k_cache, (const half_t*)v_cache, (half_t*)out,   \
          seq_len, pos0, Hq, Hkv, head_stride, scale_log2, nqb);                            \
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
