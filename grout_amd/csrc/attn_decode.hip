// Split-K GQA decode attention and its log-sum-exp merge.
//
// Reference: fmha_decode_gqa_split (src/kernels.rs:3996-4185) and
// splitk_reduce_merge (src/kernels.rs:4187-4304), recorded per layer in the
// decode graph (src/model.rs:3713-3771).  Same math: for each kv head, the
// G = Hq/Hkv query heads share every K/V read; the live context
// s_kv = position+1 is read from device memory; each split runs an fp32
// online softmax in exp2 units and the merge weights splits by 2^(m - max).
//
// gfx950 design (one workgroup = 4 waves per (split, kv head)):
//  * a wave consumes 16-position tiles (tile index t = t0 + wave + 4i, so the
//    four waves of a workgroup stream adjacent tiles).  K and V rows are read
//    with lane-contiguous 16-byte non-temporal loads (each wave instruction
//    covers 1 KiB = 4 whole rows, 8 KiB per tile), the next tile is in flight
//    in registers while the current one is stored and computed, and each wave re-lays
//    its tile out through a private LDS buffer (no workgroup barrier in the
//    loop), rows XOR-swizzled in 16-byte chunks so that both fragment reads
//    below are bank-conflict free.  Small tiles measured faster than larger
//    or deeper-buffered ones (32-position tiles, two tiles in flight, or a
//    4-slot ring filled by direct-to-LDS loads; two tiles in flight again
//    with the current loop: 23.9 against 22.7 us at 32k, also slower at 8k
//    and 16k): the memory system streams best with ~8 KiB per wave
//    outstanding;
//  * S^T = K.Q^T on v_mfma_f32_16x16x32_f16: A = the tile's 16 K rows, B = Q^T
//    with the group's query heads as the 16 columns (G <= 16, zero padded);
//  * O^T = V^T.P^T on v_mfma_f32_16x16x16_f16 (16 positions = its k): the
//    V^T fragments come straight from the row-major tile with
//    ds_read_b64_tr_b16 (gfx950's transposing LDS read), and P^T is the S^T
//    accumulator layout as is, so each query head stays in one lane column
//    and its online-softmax statistics live in the lanes that own its
//    accumulator; the accumulator rescale is skipped unless some head's max
//    grows by more than 2^8 (lazy rescale; p = 2^(s - m) against m = the max
//    minus kPHeadroom then stays below 2^15, inside fp16);
//  * the 4 waves merge through LDS at the end (float4 per (d block, lane),
//    conflict-free, one barrier) and write one fp32 partial (unnormalized
//    acc, reference point m, sum of 2^(s - m)) per (kv head, split, query
//    head); a small second kernel
//    merges the splits.  (Merging in the last workgroup of each
//    kv head behind an atomic ticket measured slower on MI355X, also with
//    every split of a kv head on one XCD so that the partials are L2 hits and
//    no L2 write-back is needed: 27.05 against 24.92 us per Qwen3-32B step at
//    32k context, 32 splits.  One workgroup reading 133 KB of partials after
//    the ticket round trip costs more than the second launch.  Interleaving
//    the splits' tiles, so that a kv head's splits stream one contiguous span
//    at a time, also measured slower: 26.3 against 25.2 us.)
#include "common.hpp"
#include "kernels.hpp"
#include "qk_norm_rope.hpp"

namespace grout {

constexpr int kTile = 16;    // kv positions per wave step
constexpr int kDecWaves = 4;  // waves per workgroup of the split pass
constexpr int kDirectWaves = 8;  // waves per workgroup of the one-split pass
constexpr int kSlotBytes = 2 * kTile * kHeadDim * 2;  // 8 KiB per wave: K rows then V rows
constexpr float kDecRescaleThreshold = 8.0f;

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;

__device__ __forceinline__ floatx4 mfma16x16x16(half4 a, half4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Swizzle of a 256-byte row: 16-byte chunk j of row r is stored at chunk
// j ^ dswz(r); a bijection on r % 16 whose upper three bits are r % 8.
__device__ __forceinline__ int dswz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

// Inputs of the fused variant: the raw QKV projection of the new token
// instead of rotated q rows, and what the norm/RoPE/KV write needs.
struct DecodeFused {
  const half_t* qkv;      // [Q (Hq*128) | K (Hkv*128) | V (Hkv*128)]
  const half_t* gamma_q;  // [128]
  const half_t* gamma_k;  // [128]
  const float* rope_cos;  // [max_ctx][64]
  const float* rope_sin;
  half_t* k_cache;        // writable views of the caches (row pos is written)
  half_t* v_cache;
  float eps;
  int Hq;
};

// WAVES waves per workgroup (split, kv head).  FUSED: the workgroup first
// computes its G rotated q rows (into LDS) and, if its split holds position
// pos, the new K row and V row of its kv head: it writes them to the cache
// and patches them into its own LDS copy of the last tile (rows pos .. end of
// that tile, which the loads clamp to row pos), so no other kernel and no
// memory ordering is involved.  DIRECT (one split): the normalized f16
// output goes straight to out [Hq][128] instead of the fp32 partials.
template <int WAVES, bool FUSED, bool DIRECT>
__global__ __launch_bounds__(WAVES * 64, (WAVES <= 4 ? 2 : 1)) void attn_decode_split_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k_cache,
    const half_t* __restrict__ v_cache, long head_stride, const uint32_t* __restrict__ d_pos,
    int max_ctx, int G, int nsplit, uint32_t split_magic, float scale_log2,
    float* __restrict__ part_acc, float* __restrict__ part_ml, DecodeFused fz,
    half_t* __restrict__ out) {
  // Wave w's tile buffer is s_buf[w].
  __shared__ __attribute__((aligned(1024))) unsigned char s_buf[WAVES][kSlotBytes];
  __shared__ float s_ml[WAVES][16][2];
  // The waves' O^T accumulators for the cross-wave merge ([d block][lane],
  // 8 KiB) go into each wave's own tile buffer once its loop is done, so the
  // workgroup needs 33 KiB (one-split variant: 71 KiB) instead of 66 (137).
  // Measured the same as a separate array at 66 KiB; the footprint matters
  // above that: the split pass padded to 99 KiB ran 0.5 us slower per 32k
  // step, although one workgroup per CU runs either way.
  static_assert(8 * 64 * sizeof(floatx4) == kSlotBytes, "accumulators fill one tile buffer");
  // FUSED: rotated q rows of the group, then the new K and V rows.
  __shared__ __attribute__((aligned(16))) half_t s_qkv[FUSED ? 18 : 1][kHeadDim];

  // Grid (Hkv, nsplit): workgroup (kvh, split) has the linear id
  // split * Hkv + kvh, and workgroups are dealt to the 8 XCDs round robin in
  // that order, so with Hkv = 8 every split of a kv head runs on one XCD and
  // its partials stay in that XCD's L2 for the merge (which uses the same
  // map).  Two grid dimensions instead of one id spare the divisions that
  // would split it.
  const int Hkv = (int)gridDim.x;
  const int kvh = (int)blockIdx.x, split = (int)blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, kb = lane >> 4;
  const int wave_off = w * kSlotBytes;  // folded into the per-lane offsets below

  // Everything up to the first tile's loads waits for the position, so the
  // chain after it has no integer division (a runtime one is ~20 dependent
  // instructions), and the q rows (independent of it) are requested first.
  const uint32_t pos = d_pos[0];
  half8 qf[4];
  if constexpr (!FUSED) {
    // Columns past the group hold a copy of head G-1 (same cache lines, no
    // branch in front of the tile loads, and no select that would wait for
    // these loads before the loop).  Every column's softmax is its own and
    // a copy rescales exactly when head G-1 does, so the wave-wide rescale
    // decision and the group's outputs are those of the G heads; the copies'
    // columns are never written.
    const int qc = col < G ? col : G - 1;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      qf[c] = as_half8(load16(q + ((size_t)kvh * G + qc) * kHeadDim + c * 32 + kb * 8));
  }
  const int s_kv = pos >= (uint32_t)max_ctx ? max_ctx : (int)pos + 1;  // always in [1, max_ctx]
  const int ntiles = (s_kv + kTile - 1) / kTile;
  // per = ceil(ntiles / nsplit): split_magic = ceil(2^31 / nsplit) = (2^31 + e)
  // / nsplit with 0 <= e < nsplit, so x * split_magic / 2^31 = x / nsplit +
  // x e / (nsplit 2^31), whose floor is floor(x / nsplit) while x e < 2^31:
  // here x < 2^18 + 2^12 (ntiles <= GROUT_MAX_CTX / 16, nsplit <= 4096).
  const int per = (int)__umulhi(2u * (uint32_t)(ntiles + nsplit - 1), split_magic);
  const int t0 = split * per;
  const int t1 = min(t0 + per, ntiles);
  // this wave's tiles: t0 + w + WAVES k, k = 0 .. nmine-1
  const int nmine = t0 + w < t1 ? (t1 - t0 - w + WAVES - 1) / WAVES : 0;

  // Wave w takes the split's tiles j = w + WAVES k, visited from j = rot on
  // (cyclically; rot is a multiple of WAVES, so the tile sets stay disjoint).
  // Splits start 256 KiB apart at 32k; staggering where each one starts
  // spreads the concurrent reads over more HBM channels (measured a few
  // percent at 4k context, within noise at 32k).  rot = (x mod P) * WAVES,
  // P = len / WAVES, x = split * 7 + kvh * 3 (kept below 2^22): the quotient
  // through the hardware reciprocal is off by at most one for these
  // magnitudes, and one correction makes the remainder exact.
  const int len = t1 - t0;
  int rot = 0;
  {
    const int P = len / WAVES;
    const int x = (split * 7 + kvh * 3) & 0x3fffff;
    const int qe = (int)((float)x * __builtin_amdgcn_rcpf((float)max(P, 1)));
    int rm = x - qe * P;
    rm = rm < 0 ? rm + P : (rm >= P ? rm - P : rm);
    rot = len > 0 && len % WAVES == 0 ? rm * WAVES : 0;
  }
  auto tile_of = [&](int k) __attribute__((always_inline)) {
    const int x = w + WAVES * k + rot;
    return t0 + (x >= len ? x - len : x);
  };

  const unsigned char* kh = reinterpret_cast<const unsigned char*>(k_cache + (size_t)kvh * head_stride);
  const unsigned char* vh = reinterpret_cast<const unsigned char*>(v_cache + (size_t)kvh * head_stride);

  // Tile as loaded: instruction i (0..3) of lane l holds row 4i + l/16,
  // logical chunk l%16, of K (rk[i]) and of V (rv[i]); it is stored at chunk
  // (l%16) ^ dswz(row) of the wave's LDS tile.
  u32x4 rk[4], rv[4];
  // The tile's four K loads go out before its four V loads (and K is stored
  // to LDS first): each wave streams one tensor at a time, which HBM serves
  // faster than alternating K and V requests, and the K stores need not wait
  // for V.  Qwen3-32B split + merge step, same box: 24.29 -> 23.89 us at 32k,
  // 14.78 -> 14.42 at 16k, 10.52 -> 9.97 at 8k (bit-identical output).
  auto load_kv = [&](int t, u32x4 (&tk)[4], u32x4 (&tv)[4]) __attribute__((always_inline)) {
    unsigned off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // rows past the context are masked; read a live row instead
      const int row = min(t * kTile + 4 * i + kb, s_kv - 1);
      off[i] = (unsigned)row * 256u + (unsigned)col * 16u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) tk[i] = load_stream16(kh + off[i]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) tv[i] = load_stream16(vh + off[i]);
  };
  auto load_tile = [&](int k) __attribute__((always_inline)) { load_kv(tile_of(k), rk, rv); };
  // FUSED prologue: 32-lane group gi of the workgroup normalizes and rotates
  // rows gi, gi + 2 WAVES, ...: rows 0..G-1 are the group's q heads, row G
  // (owner only) the new K row; the owner also stages the V row.  The reads
  // of each group's first row are issued before the wave's first K/V tile
  // loads (no branch between them, groups past the last row redo row 0), so
  // the norm waits only for its own inputs while the tile streams in, and the
  // barrier that publishes the rows orders LDS only (the tile loads stay in
  // flight across it).  Measured 0.1-0.4 us per layer at 1k-4k positions.
  const int t_new = s_kv - 1 - (s_kv - 1) % kTile;  // first position of the last tile
  const bool owner = FUSED && pos < (uint32_t)max_ctx && t_new / kTile >= t0 &&
                     t_new / kTile < t1;
  if constexpr (FUSED) {
    const int gi = threadIdx.x >> 5, j = threadIdx.x & 31;
    const int nrows = G + (owner ? 1 : 0);
    // a position past the cache writes nothing; its q rows use the last
    // table row so every read stays in bounds
    const uint32_t rpos = pos < (uint32_t)max_ctx ? pos : (uint32_t)max_ctx - 1;
    const size_t trow = (size_t)rpos * (kHeadDim / 2) + 4 * (j & 15);
    struct RowIn {
      u32x2 x, gamma, v;
      floatx4 c, s;
    };
    // Both gamma pointers in scalar registers first: selected per lane from
    // the argument block, the compiler would fetch the pointer with a vector
    // load and put that round trip in front of the tile loads.
    const half_t* gamma_q = fz.gamma_q;
    const half_t* gamma_k = fz.gamma_k;
    asm volatile("" : "+s"(gamma_q), "+s"(gamma_k));
    auto read_row = [&](int r) __attribute__((always_inline)) {
      const bool is_k = r == G;
      RowIn in;
      in.x = *reinterpret_cast<const u32x2*>(
          fz.qkv + (size_t)(is_k ? fz.Hq + kvh : kvh * G + r) * kHeadDim + 4 * j);
      typedef const __attribute__((address_space(1))) u32x2 global_u32x2;
      in.gamma = *(global_u32x2*)((is_k ? gamma_k : gamma_q) + 4 * j);  // global, not flat
      in.c = *reinterpret_cast<const floatx4*>(fz.rope_cos + trow);
      in.s = *reinterpret_cast<const floatx4*>(fz.rope_sin + trow);
      in.v = *reinterpret_cast<const u32x2*>(fz.qkv + (size_t)(fz.Hq + Hkv + kvh) * kHeadDim +
                                             4 * j);
      return in;
    };
    auto finish_row = [&](int r, const RowIn& in) __attribute__((always_inline)) {
      const u32x2 yr = norm_rope_row(in.x, __builtin_bit_cast(half4, in.gamma), in.c, in.s, j,
                                     fz.eps);
      *reinterpret_cast<u32x2*>(&s_qkv[r][4 * j]) = yr;
      if (r == G) {
        *reinterpret_cast<u32x2*>(&s_qkv[G + 1][4 * j]) = in.v;
        const size_t coff = (size_t)kvh * head_stride + (size_t)pos * kHeadDim + 4 * j;
        *reinterpret_cast<u32x2*>(fz.k_cache + coff) = yr;
        *reinterpret_cast<u32x2*>(fz.v_cache + coff) = in.v;
      }
    };
    const int r0 = gi < nrows ? gi : 0;
    const RowIn first = read_row(r0);
    __builtin_amdgcn_sched_barrier(0);
    load_tile(0);  // rows clamped to the context: in bounds for every wave
    __builtin_amdgcn_sched_barrier(0);
    finish_row(r0, first);  // same values into row 0 for the spare groups
    for (int r = gi + 2 * WAVES; r < nrows; r += 2 * WAVES)  // uniform per 32-lane group
      finish_row(r, read_row(r));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }

  if constexpr (FUSED) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      qf[c] = col < G ? as_half8(*reinterpret_cast<const u32x4*>(&s_qkv[col][c * 32 + kb * 8]))
                      : as_half8(u32x4{0u, 0u, 0u, 0u});
  }

  int st_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) st_off[i] = wave_off + (4 * i + kb) * 256 + ((col ^ dswz(4 * i + kb)) << 4);
  auto store_tile = [&](const u32x4 (&tk)[4], const u32x4 (&tv)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(&s_buf[0][0] + st_off[i]) = tk[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(&s_buf[0][0] + st_off[i] + 4096) = tv[i];
  };
  // Fragment offsets (this wave's slot base included):
  //  K (A of S^T): row col, logical chunk 4c + kb;
  //  V^T (A of O^T, via ds_read_b64_tr_b16): lane j of group kb addresses
  //  row 4kb + j/4 at d = 16db + 4(j%4), i.e. logical chunk 2db + (j%4)/2,
  //  byte 8*(j%2) inside it; lane i then holds V[4kb + k][16db + i], k < 4.
  int kfrag[4], vfrag[8];
#pragma unroll
  for (int c = 0; c < 4; ++c) kfrag[c] = wave_off + col * 256 + (((4 * c + kb) ^ dswz(col)) << 4);
  {
    const int vr = 4 * kb + (col >> 2), e = col & 3;
#pragma unroll
    for (int db = 0; db < 8; ++db)
      vfrag[db] = wave_off + 4096 + vr * 256 + (((2 * db + (e >> 1)) ^ dswz(vr)) << 4) +
                  ((e & 1) << 3);
  }

  float m = -1.0e30f;  // reference point (log2 units) of head `col`: its running max - kPHeadroom
  float l = 0.f;       // this lane's part of its sum of p (4 positions per tile)
  floatx4 acc[8];      // O^T: d = 16db + 4kb + i, head col
#pragma unroll
  for (int db = 0; db < 8; ++db) acc[db] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int k, const unsigned char* slot) __attribute__((always_inline)) {
    const int t = tile_of(k);
    floatx4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      sc = mfma16x16x32(as_half8(*reinterpret_cast<const u32x4*>(slot + kfrag[c])), qf[c], sc);
    // positions t*16 + 4kb + i; the ones past the context are masked
    const int lim = s_kv - t * kTile - 4 * kb;
    float tmax = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = i < lim ? sc[i] * scale_log2 : -__builtin_inff();
      tmax = fmaxf(tmax, sc[i]);
    }
    tmax = col_max(tmax);  // over the 4 lane groups of the column
    if (__any(tmax > m + (kDecRescaleThreshold + kPHeadroom))) {
      const float mn = fmaxf(m, tmax - kPHeadroom);
      const float alpha = fast_exp2(m - mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 8; ++db) acc[db] *= alpha;
    }
    half4 pf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = fast_exp2(sc[i] - m);
      l += p;
      pf[i] = (half_t)p;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_short4*)(__attribute__((address_space(3))) unsigned char*)(slot + vfrag[db]));
      acc[db] = mfma16x16x16(__builtin_bit_cast(half4, v), pf, acc[db]);
    }
  };

  auto patch_new_row = [&](int k) __attribute__((always_inline)) {
    if (FUSED && owner && tile_of(k) * kTile == t_new) {
      // rows pos .. t_new+15 of the slot get the new K / V row (the loads
      // read the cache's old row pos for all of them)
      const int r0 = (int)pos - t_new;
      const int chunk = lane & 15, kv = (lane >> 4) & 1;  // lanes 0..31: 16 K + 16 V chunks
      if (lane < 32) {
        const u32x4 v16 = *reinterpret_cast<const u32x4*>(&s_qkv[G + kv][chunk * 8]);
        for (int r = r0; r < kTile; ++r)
          *reinterpret_cast<u32x4*>(&s_buf[0][0] + wave_off + kv * 4096 + r * 256 +
                                    ((chunk ^ dswz(r)) << 4)) = v16;
      }
    }
  };
  if (!FUSED && nmine > 0) load_tile(0);  // FUSED: issued in the prologue
  if (nmine == 2) {
    // A wave with two tiles (4k positions over 32 splits) has both in flight
    // at once: no extra loads, 0.3-0.5 us less per launch than the loop.
    u32x4 k1[4], v1[4];
    load_kv(tile_of(1), k1, v1);
    store_tile(rk, rv);
    patch_new_row(0);
    compute(0, &s_buf[0][0]);
    store_tile(k1, v1);  // after this wave's reads of tile 0 (LDS is in order)
    patch_new_row(1);
    compute(1, &s_buf[0][0]);
  } else {
    // The loads of tile k+1 are issued before tile k is stored (two register
    // copies), so they overlap the store as well as the compute.
    for (int k = 0; k < nmine; ++k) {
      u32x4 ck[4], cv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ck[i] = rk[i];
        cv[i] = rv[i];
      }
      if (k + 1 < nmine) load_tile(k + 1);
      store_tile(ck, cv);  // after this wave's reads of the previous tile (LDS is in order)
      patch_new_row(k);
      compute(k, &s_buf[0][0]);
    }
  }
  // Per-wave statistics of head `col`; each wave's O^T accumulators go to
  // LDS as one float4 per (d block, lane) in a region of their own
  // (conflict-free, and no wait for the other waves' tile buffers); after
  // one barrier wave w merges d blocks w, w + WAVES, ... of every head for its
  // own lanes (4 exp2 per lane, float4 stores).  The first version wrote the
  // accumulators as single floats with the 16 head lanes on one LDS bank and
  // recomputed the weights per element: 1.2 + 0.75 us per wave against
  // 0.45 + 0.4 us here (Qwen3-32B, 32k context: split 22.6 -> 21.5 us).
  l = col_sum(l);
  if (kb == 0) {
    s_ml[w][col][0] = m;
    s_ml[w][col][1] = l;
  }
#pragma unroll
  for (int db = 0; db < 8; ++db) reinterpret_cast<floatx4*>(s_buf[w])[db * 64 + lane] = acc[db];
  __syncthreads();

  float M = s_ml[0][col][0];
#pragma unroll
  for (int ww = 1; ww < WAVES; ++ww) M = fmaxf(M, s_ml[ww][col][0]);
  float wgt[WAVES];
  float L = 0.f;
#pragma unroll
  for (int ww = 0; ww < WAVES; ++ww) {
    wgt[ww] = fast_exp2(s_ml[ww][col][0] - M);
    L += wgt[ww] * s_ml[ww][col][1];
  }
  const size_t base = ((size_t)kvh * nsplit + split) * G;
#pragma unroll
  for (int db = w; db < 8; db += WAVES) {
    floatx4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) {
      const floatx4 a4 = reinterpret_cast<const floatx4*>(s_buf[ww])[db * 64 + lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) O[i] += wgt[ww] * a4[i];
    }
    if (col < G) {
      const int d = 16 * db + 4 * kb;  // this lane's 4 outputs: d .. d+3 of head col
      if constexpr (DIRECT) {
        half4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (half_t)(O[i] / L);
        *reinterpret_cast<u32x2*>(out + ((size_t)kvh * G + col) * kHeadDim + d) =
            __builtin_bit_cast(u32x2, o);
      } else {
        *reinterpret_cast<floatx4*>(part_acc + (base + col) * kHeadDim + d) = O;
      }
    }
  }
  if (!DIRECT && w == 0 && kb == 0 && col < G) {
    part_ml[(base + col) * 2 + 0] = M;
    part_ml[(base + col) * 2 + 1] = L;
  }
}

// Merge: one 128-thread workgroup per (query head h = kvh*G + g, half of D),
// grid (Hkv, 2G), linear id (2g + half) * Hkv + kvh (the split pass's XCD
// map).  The split weights 2^(m_s - M) use the hardware exp2 (v_exp_f32): it
// differs from the library exp2f only below 2^-126, i.e. for splits whose max
// trails the overall max by more than 126 (log2 units), whose weight is nil either way;
// without the library's denormal path the Qwen3-32B step is ~0.2 us shorter
// (23.91 -> 23.68 us at 32k, bit-identical output).
// Thread t owns 4 consecutive d (one float4) and every 8th split, keeps its
// own running (max, sum, acc) so all its loads are independent, then the 8
// split groups combine through LDS.
constexpr int kMergeGroups = 8;

__global__ __launch_bounds__(128) void attn_decode_merge_kernel(
    const float* __restrict__ part_acc, const float* __restrict__ part_ml,
    half_t* __restrict__ out, int G, int nsplit, uint32_t* __restrict__ advance_pos) {
  __shared__ float s_m[kMergeGroups][16];
  __shared__ float s_l[kMergeGroups][16];
  __shared__ floatx4 s_o[kMergeGroups][16];
  const int kvh = (int)blockIdx.x, rest = (int)blockIdx.y;
  const int half = rest & 1, g = rest >> 1, h = kvh * G + g;
  const int dq = threadIdx.x & 15, sg = threadIdx.x >> 4;
  const int d0 = half * 64 + dq * 4;
  const size_t row0 = (size_t)kvh * nsplit * G + g;  // row of split s: row0 + s*G
  float M = -1.0e30f, L = 0.f;
  floatx4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int s = sg; s < nsplit; s += kMergeGroups) {
    const size_t r = row0 + (size_t)s * G;
    const float2 ml = *reinterpret_cast<const float2*>(part_ml + r * 2);
    const floatx4 a = *reinterpret_cast<const floatx4*>(part_acc + r * kHeadDim + d0);
    const float Mn = fmaxf(M, ml.x);
    const float so = fast_exp2(M - Mn), sn = fast_exp2(ml.x - Mn);
    L = L * so + ml.y * sn;
    O = O * so + a * sn;
    M = Mn;
  }
  s_m[sg][dq] = M;
  s_l[sg][dq] = L;
  s_o[sg][dq] = O;
  __syncthreads();
  if (sg == 0) {
    float Mt = s_m[0][dq];
#pragma unroll
    for (int i = 1; i < kMergeGroups; ++i) Mt = fmaxf(Mt, s_m[i][dq]);
    float Lt = 0.f;
    floatx4 Ot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kMergeGroups; ++i) {
      const float wgt = fast_exp2(s_m[i][dq] - Mt);
      Lt += s_l[i][dq] * wgt;
      Ot += s_o[i][dq] * wgt;
    }
    const float inv = 1.0f / Lt;
    half4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (half_t)(Ot[i] * inv);
    *reinterpret_cast<u32x2*>(out + (size_t)h * kHeadDim + d0) = __builtin_bit_cast(u32x2, o);
  }
  // The split pass that precedes this launch has read the position: this
  // kernel never does, so it may move the word on to the next step's (last,
  // so that the partials' loads go out first).
  if (advance_pos != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
    advance_pos[0] += 1u;
}

// ceil(2^31 / nsplit), the multiplier of the split kernel's division-free
// ceil(ntiles / nsplit) (nsplit in [1, GROUT_MAX_SPLITS]).
static uint32_t split_magic(int nsplit) {
  return (uint32_t)(((1ull << 31) + (unsigned long long)nsplit - 1) / (unsigned long long)nsplit);
}

hipError_t launch_attn_decode_split(const void* q, const void* k_cache, const void* v_cache,
                                    long head_stride, const uint32_t* d_pos, int max_ctx,
                                    int Hq, int Hkv, int nsplit, float qk_scale,
                                    float* part_acc, float* part_ml, hipStream_t stream) {
  const float scale_log2 = qk_scale * 1.4426950408889634f;
  attn_decode_split_kernel<kDecWaves, false, false>
      <<<dim3((unsigned)Hkv, (unsigned)nsplit), kDecWaves * 64, 0, stream>>>(
          (const half_t*)q, (const half_t*)k_cache, (const half_t*)v_cache, head_stride, d_pos,
          max_ctx, Hq / Hkv, nsplit, split_magic(nsplit), scale_log2, part_acc, part_ml,
          DecodeFused{}, nullptr);
  return hipGetLastError();
}

hipError_t launch_attn_decode_fused(const void* qkv, const void* gamma_q, const void* gamma_k,
                                    const float* rope_cos, const float* rope_sin, void* k_cache,
                                    void* v_cache, long head_stride, const uint32_t* d_pos,
                                    int max_ctx, int Hq, int Hkv, int nsplit, float eps,
                                    float qk_scale, float* part_acc, float* part_ml, void* out,
                                    hipStream_t stream, uint32_t* advance_pos) {
  const float scale_log2 = qk_scale * 1.4426950408889634f;
  const DecodeFused fz{(const half_t*)qkv, (const half_t*)gamma_q, (const half_t*)gamma_k,
                       rope_cos, rope_sin, (half_t*)k_cache, (half_t*)v_cache, eps, Hq};
  if (Hq / Hkv > 16) return hipErrorInvalidValue;
  if (nsplit == 1) {
    attn_decode_split_kernel<kDirectWaves, true, true>
        <<<dim3((unsigned)Hkv, 1u), kDirectWaves * 64, 0, stream>>>(
            nullptr, (const half_t*)k_cache, (const half_t*)v_cache, head_stride, d_pos, max_ctx,
            Hq / Hkv, 1, split_magic(1), scale_log2, nullptr, nullptr, fz, (half_t*)out);
    return hipGetLastError();
  }
  attn_decode_split_kernel<kDecWaves, true, false>
      <<<dim3((unsigned)Hkv, (unsigned)nsplit), kDecWaves * 64, 0, stream>>>(
          nullptr, (const half_t*)k_cache, (const half_t*)v_cache, head_stride, d_pos, max_ctx,
          Hq / Hkv, nsplit, split_magic(nsplit), scale_log2, part_acc, part_ml, fz, nullptr);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attn_decode_merge(part_acc, part_ml, out, Hq, Hkv, nsplit, stream, advance_pos);
}

hipError_t launch_attn_decode_merge(const float* part_acc, const float* part_ml, void* out,
                                    int Hq, int Hkv, int nsplit, hipStream_t stream,
                                    uint32_t* advance_pos) {
  attn_decode_merge_kernel<<<dim3((unsigned)Hkv, (unsigned)(2 * (Hq / Hkv))), 128, 0, stream>>>(
      part_acc, part_ml, (half_t*)out, Hq / Hkv, nsplit, advance_pos);
  return hipGetLastError();
}

// ---------------------------------------------------------------- layout probe

__global__ __launch_bounds__(64) void mfma_layout_probe_kernel(float* out) {
  const int l = threadIdx.x;
  half8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (half_t)(float)(l * 8 + i);
    b[i] = (half_t)((8 * (l >> 4) + i == (l & 15)) ? 1.0f : 0.0f);
  }
  const floatx4 c = mfma16x16x32(a, b, floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
  for (int j = 0; j < 4; ++j) out[l * 4 + j] = c[j];
}

hipError_t launch_mfma_layout_probe(float* out64x4, hipStream_t stream) {
  mfma_layout_probe_kernel<<<1, 64, 0, stream>>>(out64x4);
  return hipGetLastError();
}

}  // namespace grout
