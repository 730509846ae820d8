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
// gfx950 design (v_mfma_f32_16x16x32_f16, one 512-thread workgroup per CU):
//  * a team of 4 waves owns a q block of 128 query rows = BQ query positions
//    x HG heads of one kv group (HG = the largest divisor of G that is <= 8,
//    BQ = floor(128/HG)), so every K/V tile staged in LDS serves HG heads;
//    each wave owns 32 rows (two 16-column MFMA blocks).  Short prompts,
//    whose 128-row blocks cannot give every CU a workgroup, use 64-row
//    blocks instead (16 rows per wave: twice the workgroups, each with half
//    the MFMA work per tile);
//  * the workgroup holds two teams, A = waves 0-3 and B = waves 4-7, one wave
//    of each per SIMD.  Per kv tile a team runs two phases: G (the MFMA work:
//    P(j).V(j) and S(j+1) = Q.K(j+1)^T) and S (the VALU work: mask, row max,
//    exp2, P(j+1) and its row sums).  Team B runs one phase behind team A and
//    every phase ends in a workgroup barrier, so on every SIMD one wave feeds
//    the matrix core while the other runs the softmax ("ping-pong");
//  * causal balance: workgroup r owns the complementary q blocks h = nqb-1-r
//    and l = r (their tile counts add up to a constant).  Team A takes tiles
//    [0, a) of h, team B all tiles of l and then tiles [a, T_h) of h, with
//    a = ceil((T_h + T_l) / 2); the two partials (m, l, acc) of h meet in
//    LDS at the end and each team finishes half of h's d range.  Or each
//    workgroup takes a single q block (T_l = 0), heaviest first (the work
//    split is chosen per launch, see launch_fmha_prefill);
//  * K and V tiles (64 positions, 16 KiB each) go straight from the cache into
//    double-buffered, XOR-swizzled LDS slots with buffer_load ... lds.  A
//    per-tile buffer resource bounds the read at kv_len, so rows past the end
//    arrive as zeros with no per-lane address arithmetic or clamping.  Loads
//    for tiles j+2 (K) and j+1 (V) are issued in the S phase of tile j and
//    have three phases to land: the barriers order LDS only and each wave
//    waits for its own older loads (vmcnt) before the barrier that publishes
//    them;
//  * S^T = K.Q^T (A = K rows from LDS, B = Q held in VGPRs) and
//    O^T = V^T.P^T (the V^T fragments come straight from the row-major tile
//    with ds_read_b64_tr_b16, P from the S^T accumulators without a shuffle),
//    so each query row is one lane column and its softmax statistics live in
//    the lanes that own its accumulator; row reductions across the four lane
//    groups use v_permlane16/32_swap, row sums v_dot2 on the f16 P values;
//  * speculative softmax: P is computed against the reference point as it
//    stands (the running max minus kPHeadroom) and checked through its own
//    row sums; only a tile whose scores rise ~8 (log2 units) above the
//    running max (and the first tile of a block) pays for the exact row max,
//    the rescale and a second pass, so p stays below 2^15 (inside f16) and
//    most tiles cost 2 VALU ops per score plus the exp2;
//  * scheduling: block id -> (kv head = id mod Hkv, q block pair), so with
//    Hkv = 8 each XCD's L2 holds one kv head's K/V.
#include "common.hpp"
#include "kernels.hpp"

#include <cstdlib>
#include <type_traits>

namespace grout {

constexpr int kBN = 64;  // kv positions per tile
// A lane's share of a tile row sum at or above this, 2^(8 + kPHeadroom),
// sends the tile down the exact-max path of the speculative softmax (see
// s_phase).
constexpr float kSpecLimit = 32768.0f;
constexpr int kRowsPerTeam = 128;
constexpr int kRowBytes = kHeadDim * 2;     // 256 B: one K or V row
constexpr int kTileBytes = kBN * kRowBytes;  // 16 KiB: one K or V tile
// Buffer resource word 3 for raw (unswizzled, stride 0) 32-bit buffer access.
constexpr int kBufferWord3 = 0x00020000;

// LDS swizzles of a 256-byte row: 16-byte chunk j of row r is stored at
// chunk j ^ swz(r).  K tiles use swz(r) = r % 16 (the 16 rows of a K fragment
// read, one chunk each, spread over the banks at full ds_read_b128 rate; the
// bijection ((r&7)<<1)|((r>>3)&1) measured at ~55% of it on gfx950).  V tiles
// use swz_v(r) = ((r&7)<<1)|((r>>3)&1): swz_v(r) >> 1 = r % 8, so the 8
// consecutive rows of a transposing read address 8 different chunk pairs.
__device__ __forceinline__ int swz_v(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;
typedef __attribute__((address_space(3))) void lds_void;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// ds_read_b64_tr_b16: inside each 16-lane group, lane i receives element
// (i % 4) of the 8-byte chunks addressed by lanes i/4, i/4+4, i/4+8, i/4+12.
__device__ __forceinline__ half4 lds_read_tr16(const unsigned char* p) {
  const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)(__attribute__((address_space(3))) unsigned char*)(p));
  return __builtin_bit_cast(half4, v);
}

// Workgroup barrier that orders LDS accesses only: this wave's LDS reads and
// writes complete (lgkmcnt), direct-to-LDS loads in flight stay in flight.
// A C++ release fence would also wait for every one of those loads (they
// count as LDS writes), which would serialize the staging with the compute.
// The "memory" clobber keeps the compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// This wave's vector-memory operations except the 8 most recent (resp. all)
// are complete.
__device__ __forceinline__ void wait_vm_keep8() { asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); }
__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// s_waitcnt immediate for vmcnt(0) alone (gfx9 fields: vmcnt bits 3:0 and
// 15:14 = 0, expcnt bits 6:4 = 7, lgkmcnt bits 11:8 = 15, i.e. no wait).
constexpr int kVmcnt0 = 0x0F70;

// The per-team kernel splits its workgroup id with host-computed multipliers
// (DivBy), so its first loads wait for no integer division (Qwen3-4B S=2048
// 40.62 -> 40.16 us, S=512 9.83 -> 9.73 us, bit-identical).
// Workgroup id = (r * nsub + hsub) * Hkv + kvh, with G = Hq / Hkv query heads
// per kv head in nsub = G / HG sub-groups.
struct BlockMap {
  int G;
  DivBy hkv, nsub;
};

// MB: 16-row MFMA blocks per wave (2: 32 rows per wave, 128 per team; 1: 16
// and 64, for short prompts, where the 128-row form leaves CUs idle).
template <int HG, int MB>
__global__ __launch_bounds__(512, 1) void fmha_prefill_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k_cache,
    const half_t* __restrict__ v_cache, half_t* __restrict__ out, int S, int pos0, int Hq,
    int Hkv, long head_stride, float scale_log2, int nqb, int paired, BlockMap bm) {
  constexpr int RT = 64 * MB;  // rows per team
  constexpr int BQ = RT / HG;
  // Per team: two K slots and two V slots, each slot its own LDS object, so
  // the compiler knows that the loads filling one slot do not alias the
  // fragment reads of another and keeps them in flight.
  __shared__ __attribute__((aligned(1024))) unsigned char s_k0[2][kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_k1[2][kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_v0[2][kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_v1[2][kTileBytes];

  const int G = bm.G;
  const int nsub = G / HG;
  const int bid = blockIdx.x;
  const int rest = (int)div_by((uint32_t)bid, bm.hkv);
  const int kvh = bid - rest * Hkv;
  const int r = (int)div_by((uint32_t)rest, bm.nsub);
  const int hsub = rest - r * nsub;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int team = wave >> 2;
  const int w = wave & 3;
  const int col = lane & 15, kb = lane >> 4;
  const int kv_len = pos0 + S;

  auto tiles_of = [&](int qb) __attribute__((always_inline)) {
    const int q_last = min(qb * BQ + BQ, S) - 1;
    return (pos0 + q_last + 1 + kBN - 1) / kBN;
  };
  // Work split (workgroup-uniform): blocks h >= l, team A tiles [0, a) of h,
  // team B tiles [0, tl) of l then [a, th) of h.  Heaviest blocks first in
  // both forms; unpaired, l = h means no light block.
  const int h = nqb - 1 - r;
  const int l = paired ? r : h;
  const int th = tiles_of(h), tl = h != l ? tiles_of(l) : 0;
  const int a = (th + tl + 1) / 2;
  const int nB = tl + th - a;
  const bool merge_h = th > a;
  // This team's tile sequence: n0 tiles of q block qb0 from tile tb0, then n1
  // tiles of q block qb1 from tile tb1 (wave-uniform).
  int qb0, tb0, n0, qb1, tb1, n1;
  if (team == 0) {
    qb0 = h; tb0 = 0; n0 = a; qb1 = h; tb1 = 0; n1 = 0;
  } else if (tl > 0) {
    qb0 = l; tb0 = 0; n0 = tl; qb1 = h; tb1 = a; n1 = th - a;
  } else {
    qb0 = h; tb0 = a; n0 = th - a; qb1 = h; tb1 = 0; n1 = 0;
  }
  const int n = n0 + n1;
  auto tile_at = [&](int j) __attribute__((always_inline)) { return j < n0 ? tb0 + j : tb1 + (j - n0); };
  auto qb_at = [&](int j) __attribute__((always_inline)) { return j < n0 ? qb0 : qb1; };

  const unsigned char* kh = reinterpret_cast<const unsigned char*>(k_cache + (size_t)kvh * head_stride);
  const unsigned char* vh = reinterpret_cast<const unsigned char*>(v_cache + (size_t)kvh * head_stride);

  // Team t's slots sit t * kTileBytes above team 0's in every slot array;
  // the offset is folded into the per-lane addresses, so the slot arrays
  // stay compile-time constants (immediate offsets).
  const int team_off = team * kTileBytes;
  unsigned char* const k0 = s_k0[0];
  unsigned char* const k1 = s_k1[0];
  unsigned char* const v0 = s_v0[0];
  unsigned char* const v1 = s_v1[0];

  // Row rr = 32w + 16mb + col of a q block is query position qb*BQ + rr/HG of
  // head kvh*G + hsub*HG + rr%HG.
  auto rpos = [&](int mb) __attribute__((always_inline)) { return (16 * MB * w + 16 * mb + col) / HG; };
  auto rhead = [&](int mb) __attribute__((always_inline)) {
    return kvh * G + hsub * HG + (16 * MB * w + 16 * mb + col) % HG;
  };
  auto row_valid = [&](int qb, int mb) __attribute__((always_inline)) {
    return 16 * MB * w + 16 * mb + col < BQ * HG && qb * BQ + rpos(mb) < S;
  };

  half8 qf[MB][4];
  auto load_q = [&](int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const bool valid = row_valid(qb, mb);
      const half_t* qr = q + ((size_t)(qb * BQ + rpos(mb)) * Hq + rhead(mb)) * kHeadDim + kb * 8;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        qf[mb][c] = valid ? as_half8(load16(qr + c * 32)) : as_half8(u32x4{0u, 0u, 0u, 0u});
    }
  };

  // m: reference point (log2 units) of row `col`, its running max minus
  // kPHeadroom; lsum: this lane's share of its sum of p = 2^(s - m) (the lane
  // group kb covers 16 of every 64 positions); acc: O^T fragments.  m starts
  // finite and masked scores are -inf, so a row whose tiles so far are all
  // masked keeps p = 0 (exp2(-inf)) instead of exp2(0).
  float m[MB], lsum[MB];
  floatx4 acc[MB][8];
  auto reset_state = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      m[mb] = -1.0e30f;
      lsum[mb] = 0.f;
#pragma unroll
      for (int db = 0; db < 8; ++db) acc[mb][db] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  };
  reset_state();

  // Direct-to-LDS staging: wave instruction i of team wave w writes the 1 KiB
  // of LDS holding tile rows 16w + 4i .. +3, lane l at byte 16*l, i.e. row
  // 16w + 4i + l/16, stored chunk l%16, which holds logical chunk
  // (l%16) ^ swz(row).  Each 16-lane group reads one whole 256-byte row.
  // For these rows (r % 16 = 4i + kb) the K swizzle is 4i ^ kb and the V
  // swizzle 2kb | 8(i&1) | (i>>1) (disjoint bits), so the source offset of
  // instruction i is (dma0 ^ 16*c_i) + 1024i with c_i = 4i (K) or
  // 8(i&1) | (i>>1) (V); the 1024i is the instruction's immediate offset,
  // which moves the global and the LDS address alike.
  const int dma0_k = (16 * w + kb) * kRowBytes + ((col ^ kb) << 4);
  const int dma0_v = (16 * w + kb) * kRowBytes + ((col ^ (2 * kb)) << 4);
  auto dma_tile = [&](auto is_v, const unsigned char* base, int tile, unsigned char* slot)
                      __attribute__((always_inline)) {
    constexpr bool V = decltype(is_v)::value;
    const int valid_rows = kv_len - tile * kBN;  // >= 1 for every tile issued
    __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(base) + (size_t)tile * kTileBytes, (short)0,
        valid_rows * kRowBytes, kBufferWord3);
    int o = V ? dma0_v : dma0_k;
    asm volatile("" : "+v"(o));  // rebuilt per call, not held live across the loop
    lds_void* const dst = (lds_void*)(slot + team_off + 4 * w * 1024);
    constexpr int c1 = V ? 8 : 4, c2 = V ? 1 : 8, c3 = V ? 9 : 12;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, o, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, o ^ (c1 << 4), 0, 1024, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, o ^ (c2 << 4), 0, 2048, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, o ^ (c3 << 4), 0, 3072, 0);
  };
  const std::true_type is_v;
  const std::false_type is_k;

  // Per-lane LDS offsets of the fragment reads; row offsets are immediates.
  //  K fragment (pb, c): row 16pb + col, logical chunk 4c + kb;
  //  V^T fragment (cc, db, half h): lane j of its 16-lane group addresses row
  //  32cc + 16h + 4kb + j/4 at d = 16db + 4(j%4), i.e. logical chunk
  //  2db + (j%4)/2, byte 8*(j%2) inside it.
  // (4c + kb) ^ col = 4(c ^ (col>>2)) + (kb ^ (col&3)): the K offset of chunk
  // group c is kfrag0 ^ 64c.  Likewise (2db + e/2) ^ swz_v(vr) =
  // 2(db ^ (vr&7)) + (e/2 ^ (swz_v&1)): the V^T offset of block db is
  // vfrag0 ^ 32db.  Bits 6-7 (K) and 5-7 (V) of the bases are free for the
  // XOR constants.
  int kfrag0, vfrag0;
  {
    kfrag0 = team_off + col * kRowBytes + ((col >> 2) << 6) + ((kb ^ (col & 3)) << 4);
    const int vr = 4 * kb + (col >> 2), e = col & 3, sv = swz_v(vr);
    vfrag0 = team_off + vr * kRowBytes + ((vr & 7) << 5) + (((e >> 1) ^ (sv & 1)) << 4) +
             ((e & 1) << 3);
  }

  floatx4 sc[MB][4];   // S^T(j+1): element (pb, i) is kv position kv0 + 16pb + 4kb + i
  half8 pf[MB][2];     // P(j) as the B operand of P.V (positions 32cc + {4kb.., 16+4kb..})

  // S(j+1) = K(j+1).Q^T (each K fragment serves both 16-row blocks).
  auto qk = [&](const unsigned char* kread, int kbase) __attribute__((always_inline)) {
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      half8 kf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kf[c] = as_half8(*reinterpret_cast<const u32x4*>(kread + (kbase ^ (c << 6)) + 16 * pb * kRowBytes));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) s = mfma16x16x32(kf[c], qf[mb][c], s);
        sc[mb][pb] = s;
      }
    }
  };
  // G phase: P(j).V(j) into acc, then (unless j is the last tile) S(j+1), so
  // P and the new scores are never live together.  The instruction order is
  // fixed by hand (sched_barrier between groups):
  //  * MFMAs that accumulate into the same registers run back to back (a
  //    single wave feeding the matrix core runs at half rate when
  //    consecutive MFMAs all read their accumulator from the register file,
  //    and the scheduler would otherwise interleave independent chains);
  //  * LDS under load answers in hundreds of cycles, so fragment reads run
  //    four V blocks ahead, the K reads of pb 0-1 go under the last four V
  //    blocks and those of pb 2-3 under the chains of pb 0-1.
  auto g_phase = [&](auto with_qk, const unsigned char* kread, const unsigned char* vread)
                     __attribute__((always_inline)) {
    constexpr bool QK = decltype(with_qk)::value;
    __builtin_amdgcn_s_setprio(1);
    int vbase = vfrag0, kbase = kfrag0;
    asm volatile("" : "+v"(vbase), "+v"(kbase));  // per-phase XORs, not 12 live registers
    half8 vf[8][2];
    half8 kf[4][4];
    auto read_v = [&](int db) __attribute__((always_inline)) {
      const int vo = vbase ^ (db << 5);
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const half4 lo = lds_read_tr16(vread + vo + 32 * cc * kRowBytes);
        const half4 hi = lds_read_tr16(vread + vo + (32 * cc + 16) * kRowBytes);
        vf[db][cc] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    };
    auto read_k = [&](int pb, int c) __attribute__((always_inline)) {
      kf[pb][c] = as_half8(*reinterpret_cast<const u32x4*>(kread + (kbase ^ (c << 6)) + 16 * pb * kRowBytes));
    };
#pragma unroll
    for (int db = 0; db < 4; ++db) read_v(db);
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        acc[mb][db] = mfma16x16x32(vf[db][0], pf[mb][0], acc[mb][db]);
        acc[mb][db] = mfma16x16x32(vf[db][1], pf[mb][1], acc[mb][db]);
      }
      if (db + 4 < 8) {
        read_v(db + 4);
      } else if constexpr (QK) {
        const int i = db - 4;  // K reads of pb 0-1: two per V block
        read_k(i >> 1, 2 * (i & 1));
        read_k(i >> 1, 2 * (i & 1) + 1);
      }
    }
    if constexpr (QK) {
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          __builtin_amdgcn_sched_barrier(0);
          floatx4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < 4; ++c) a = mfma16x16x32(kf[pb][c], qf[mb][c], a);
          sc[mb][pb] = a;
          if (pb < 2) {
            if constexpr (MB == 2) {
              read_k(pb + 2, 2 * mb);
              read_k(pb + 2, 2 * mb + 1);
            } else {
#pragma unroll
              for (int c = 0; c < 4; ++c) read_k(pb + 2, c);
            }
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
  };
  // QK only (the first tile of the team's sequence).
  auto qk_only = [&](const unsigned char* kread) __attribute__((always_inline)) {
    int kbase = kfrag0;
    asm volatile("" : "+v"(kbase));
    qk(kread, kbase);
  };

  // S phase of tile j: staging of K(j+2) and V(j+1) (repeats of the last tile
  // past the end go to slots that are not read again, so every S phase issues
  // exactly 8 loads per wave), the next segment's Q when tile j+1 starts one,
  // then mask, row max, lazy rescale, P(j) and its row sums.  Ends with each
  // wave's loads of the previous S phase complete.
  auto s_phase = [&](int j, unsigned char* kfill, unsigned char* vfill) __attribute__((always_inline)) {
    // Once per workgroup (team B, before the first tile of its second
    // block): that block's Q, issued ahead of this phase's 8 tile loads.  The
    // phase's closing vmcnt(8) then covers it, so its latency hides under the
    // softmax, and the wait the compiler puts before the next S.K^T is the
    // same vmcnt(8) (8 tile loads issued after it), already satisfied.
    if (j + 1 == n0 && n1 > 0) load_q(qb1);
    dma_tile(is_k, kh, tile_at(min(j + 2, n - 1)), kfill);
    dma_tile(is_v, vh, tile_at(min(j + 1, n - 1)), vfill);
    const int kv0 = tile_at(j) * kBN;
    const int qrow0 = pos0 + qb_at(j) * BQ;  // first query position of the block
    if (kv0 + kBN - 1 > qrow0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        // element (pb, i) is kv position kv0 + 4kb + 16pb + i: compare the
        // immediate 16pb + i against one per-lane limit
        const int lim = qrow0 + rpos(mb) - kv0 - 4 * kb;
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (16 * pb + i > lim) sc[mb][pb][i] = -__builtin_inff();
      }
    }
    // Speculative softmax: P against the reference point m as it stands, and
    // this lane's share of each row sum (16 scores).  A share of kSpecLimit
    // or more (a score ~8 or more above the running max, an overflow to inf,
    // or m still at its initial -1e30) sends the wave to the exact path: tile
    // row max, rescale of what was accumulated, P again.  Accepted tiles keep
    // p < 2^15.
    float ts[MB];
    auto probs = [&]() __attribute__((always_inline)) {
      const half2v ones = {(half_t)1.f, (half_t)1.f};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        float s = 0.f;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          half8 p;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              p[hh * 4 + i] = (half_t)fast_exp2(sc[mb][2 * cc + hh][i] * scale_log2 - m[mb]);
          pf[mb][cc] = p;
          s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 0, 1), ones, s, false);
          s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 2, 3), ones, s, false);
          s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 4, 5), ones, s, false);
          s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 6, 7), ones, s, false);
        }
        ts[mb] = s;
      }
    };
    probs();
    bool over = false;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) over = over || ts[mb] >= kSpecLimit;
    if (__any(over)) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        float t = fmaxf(sc[mb][0][0], sc[mb][0][1]);
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
#pragma unroll
          for (int i = (pb == 0 ? 2 : 0); i < 4; ++i) t = fmaxf(t, sc[mb][pb][i]);
        // (m + kPHeadroom is the running max; this form needs no register
        // for the constant)
        const float mnew = fmaxf(m[mb] + kPHeadroom, col_max(t) * scale_log2) - kPHeadroom;
        const float alpha = fast_exp2(m[mb] - mnew);
        m[mb] = mnew;
        lsum[mb] *= alpha;
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[mb][db] *= alpha;
      }
      probs();
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) lsum[mb] += ts[mb];
    wait_vm_keep8();
  };

  const std::integral_constant<int, 0> c0;
  const std::integral_constant<int, 4> c4;
  const std::integral_constant<int, 8> c8;
  // Output rows of block qb, d blocks [DB0, DB0 + NDB).
  auto write_rows = [&](auto db0_c, auto ndb_c, int qb, const float (&lrow)[MB])
                        __attribute__((always_inline)) {
    constexpr int DB0 = decltype(db0_c)::value, NDB = decltype(ndb_c)::value;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      if (!row_valid(qb, mb)) continue;
      const float inv = 1.0f / lrow[mb];
      half_t* orow = out + ((size_t)(qb * BQ + rpos(mb)) * Hq + rhead(mb)) * kHeadDim;
#pragma unroll
      for (int db = DB0; db < DB0 + NDB; ++db) {
        half4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (half_t)(acc[mb][db][i] * inv);
        *reinterpret_cast<u32x2*>(orow + 16 * db + 4 * kb) = __builtin_bit_cast(u32x2, o);
      }
    }
  };
  auto row_sums = [&](float (&lrow)[MB]) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) lrow[mb] = col_sum(lsum[mb]);
  };

  // G phase of tile j plus, after the last tile of the first segment when a
  // second one follows, that block's output and a fresh state.
  auto g_step = [&](int j, const unsigned char* kread, const unsigned char* vread) __attribute__((always_inline)) {
    if (j + 1 < n)
      g_phase(std::true_type{}, kread, vread);
    else
      g_phase(std::false_type{}, kread, vread);
    if (j + 1 == n0 && n1 > 0) {
      float lrow[MB];
      row_sums(lrow);
      write_rows(c0, c8, qb0, lrow);
      reset_state();
    }
  };

  // ---- prologue: K(0) -> k0, V(0) -> v0, K(1) -> k1, Q of the first block ----
  // Team B loads its Q only after the first barrier (it idles one phase
  // anyway), so team A's Q is not slowed by the other half of the burst of Q
  // reads that opens the kernel on every CU at once.
  // K(0) and team A's Q go out first and are all that the first barrier
  // waits for: V(0) and K(1) (the 8 most recent loads of each wave) land
  // under S(0) = K(0).Q^T and team A's first softmax.  The closing wait of
  // each team's first S phase (vmcnt(8): everything but that phase's own 8
  // loads) covers them before the barrier ahead of their first reader, the
  // G phase of tile 0.
  if (n > 0) {
    dma_tile(is_k, kh, tile_at(0), k0);
    if (team == 0) load_q(qb0);
    __builtin_amdgcn_sched_barrier(0);
    dma_tile(is_v, vh, tile_at(0), v0);
    dma_tile(is_k, kh, tile_at(min(1, n - 1)), k1);
  }
  wait_vm_keep8();
  lds_barrier();
  // Phase count after this point: A runs 1 + 2*nA phases, B one idle phase
  // plus 1 + 2*nB; the shorter team pads with empty phases.
  const int total = max(1 + 2 * a, 2 + 2 * nB);
  int mine = 0;
  if (team == 1) {
    if (n > 0) load_q(qb0);
    lds_barrier();
    // Its Q (and V(0), K(1) before it) complete, in a wait the compiler
    // sees: on the code both teams share from here, team A's path then
    // needs only vmcnt(8) (its V(0) and K(1) stay in flight), where a wait
    // for team B's Q, the most recent loads, would be vmcnt(0) for both.
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    mine = 1;
  }
  if (n > 0) qk_only(k0);
  lds_barrier();
  mine += 1 + 2 * n;
  // Tile j reads K slot (j+1)&1 and V slot j&1 in its G phase and refills K
  // slot j&1 and V slot (j+1)&1 in its S phase.  Two tiles per trip, so the
  // slot of every access is a compile-time constant.
  for (int j = 0; j < n; j += 2) {
    s_phase(j, k0, v1);
    lds_barrier();
    g_step(j, k1, v0);
    lds_barrier();
    if (j + 1 < n) {
      s_phase(j + 1, k1, v0);
      lds_barrier();
      g_step(j + 1, k0, v1);
      lds_barrier();
    }
  }
  for (; mine < total; ++mine) lds_barrier();
  // The last S phases' loads may still be landing in slots that the merge
  // below reuses: every wave drains its own before one more barrier.
  wait_vm_all();
  lds_barrier();

  float lrow[MB];
  row_sums(lrow);
  if (!merge_h) {
    if (n > 0) write_rows(c0, c8, n1 > 0 ? qb1 : qb0, lrow);
    return;
  }
  // Team B holds tiles [a, T_h) of block h, team A tiles [0, a): same wave
  // index, same lane, same rows and columns.  Each team finishes half of the
  // d blocks (A 0-3, B 4-7): it publishes the other half of its (acc) and its
  // (m, l) through LDS (slot arrays of the wave index: A's half in the first
  // 8 KiB, B's in the second; team t's (m, l) in team 0's first K slot at
  // t * 4 KiB), then combines its own half with the other team's, A's terms
  // first in both teams.
  unsigned char* const accbuf = w == 0 ? s_k0[1] : w == 1 ? s_k1[1] : w == 2 ? s_v0[1] : s_v1[1];
  float* const mlbuf = reinterpret_cast<float*>(s_k0[0] + w * 1024) + lane * 4;
  const int other = 1 - team;
  auto xchg = [&](auto give_c) __attribute__((always_inline)) {
    constexpr int GIVE = decltype(give_c)::value;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<floatx4*>(accbuf + team * 8192 + ((mb * 4 + i) * 64 + lane) * 16) =
            acc[mb][GIVE + i];
  };
  if (team == 0)
    xchg(c4);
  else
    xchg(c0);
  *reinterpret_cast<floatx4*>(mlbuf + team * 1024) = floatx4{m[0], m[MB - 1], lrow[0], lrow[MB - 1]};
  lds_barrier();
  const floatx4 mlo = *reinterpret_cast<const floatx4*>(mlbuf + other * 1024);
  auto finish = [&](auto keep_c) __attribute__((always_inline)) {
    constexpr int KEEP = decltype(keep_c)::value;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const float ma = team == 0 ? m[mb] : mlo[mb], mbb = team == 0 ? mlo[mb] : m[mb];
      const float la = team == 0 ? lrow[mb] : mlo[2 + mb], lb = team == 0 ? mlo[2 + mb] : lrow[mb];
      const float mn = fmaxf(ma, mbb);
      const float sa = fast_exp2(ma - mn), sb = fast_exp2(mbb - mn);
      const float ss = team == 0 ? sa : sb, so = team == 0 ? sb : sa;
      lrow[mb] = la * sa + lb * sb;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const floatx4 mine = acc[mb][KEEP + i] * ss;
        const floatx4 theirs = *reinterpret_cast<const floatx4*>(
                                   accbuf + other * 8192 + ((mb * 4 + i) * 64 + lane) * 16) * so;
        acc[mb][KEEP + i] = team == 0 ? mine + theirs : theirs + mine;
      }
    }
    write_rows(keep_c, c4, h, lrow);
  };
  if (team == 0)
    finish(c0);
  else
    finish(c4);
}

// Shared-stream variant: a segment is one 256-row q block, team A holding its
// first BQ query positions and team B the next BQ (HG heads each), so both
// teams need the same K/V tiles and consume one staged stream: team A stages
// the K tiles and team B the V tiles (4 loads per wave per S phase instead of
// 8), into three K and three V slots (96 KiB).  A workgroup runs the
// complementary blocks h = nqb2-1-r and l = r back to back (their tile counts
// add up to a constant), both teams switching from h to l at the same tile,
// or (paired = 0) the single block h, heaviest first; each team writes its
// own rows, so there is no end-of-kernel merge.  Used for long prompts, see
// plan_fmha_prefill.
//
// Slot schedule (team B one phase behind team A; phases counted from 0):
// G(j) = P(j).V(j) + S(j+1) = Q.K(j+1)^T runs at phase 2j+2 (A) / 2j+3 (B),
// so K(j) is read at phases 2j and 2j+1 and V(j) at 2j+2 and 2j+3.  Team A
// issues K(j+2) in its S phase of tile j (phase 2j+1) into the slot of
// K(j-1), last read at phase 2j-1, and waits for it at the end of its next S
// phase; team B issues V(j+2) at phase 2j+2 into the slot of V(j-1), last
// read at phase 2j+1, and waits for it at the end of its next S phase (phase
// 2j+4), four phases before its first reader.
template <int HG>
__global__ __launch_bounds__(512, 1) void fmha_prefill_shared_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k_cache,
    const half_t* __restrict__ v_cache, half_t* __restrict__ out, int S, int pos0, int Hq,
    int Hkv, long head_stride, float scale_log2, int nqb2, int paired) {
  constexpr int BQ = kRowsPerTeam / HG;  // query positions per team
  constexpr int BQ2 = 2 * BQ;           // per block
  __shared__ __attribute__((aligned(1024))) unsigned char s_k0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_k1[kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_k2[kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_v0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_v1[kTileBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char s_v2[kTileBytes];

  // (the division-free decomposition of the per-team kernel measured 0.7%
  // slower here, Qwen3-32B S=2048)
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
  const int team = wave >> 2;
  const int w = wave & 3;
  const int col = lane & 15, kb = lane >> 4;
  const int kv_len = pos0 + S;

  auto tiles_of = [&](int qb) __attribute__((always_inline)) {
    const int q_last = min(qb * BQ2 + BQ2, S) - 1;
    return (pos0 + q_last + 1 + kBN - 1) / kBN;
  };
  // paired: complementary blocks h and l back to back; else one block per
  // workgroup, heaviest first
  const int h = nqb2 - 1 - r, l = paired ? r : h;
  const int th = tiles_of(h), tl = l < h ? tiles_of(l) : 0;
  const int n = th + tl;
  auto tile_at = [&](int j) __attribute__((always_inline)) { return j < th ? j : j - th; };
  auto qb_at = [&](int j) __attribute__((always_inline)) { return j < th ? h : l; };

  const unsigned char* kh = reinterpret_cast<const unsigned char*>(k_cache + (size_t)kvh * head_stride);
  const unsigned char* vh = reinterpret_cast<const unsigned char*>(v_cache + (size_t)kvh * head_stride);

  // Row rr = 32w + 16mb + col of this team's 128 is query position
  // qb*BQ2 + team*BQ + rr/HG of head kvh*G + hsub*HG + rr%HG.
  auto rpos = [&](int mb) __attribute__((always_inline)) {
    return team * BQ + (32 * w + 16 * mb + col) / HG;
  };
  auto rhead = [&](int mb) __attribute__((always_inline)) {
    return kvh * G + hsub * HG + (32 * w + 16 * mb + col) % HG;
  };
  auto row_valid = [&](int qb, int mb) __attribute__((always_inline)) {
    return 32 * w + 16 * mb + col < BQ * HG && qb * BQ2 + rpos(mb) < S;
  };

  half8 qf[2][4];
  auto load_q = [&](int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const bool valid = row_valid(qb, mb);
      const half_t* qr = q + ((size_t)(qb * BQ2 + rpos(mb)) * Hq + rhead(mb)) * kHeadDim + kb * 8;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        qf[mb][c] = valid ? as_half8(load16(qr + c * 32)) : as_half8(u32x4{0u, 0u, 0u, 0u});
    }
  };

  float m[2], lsum[2];
  floatx4 acc[2][8];
  auto reset_state = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      m[mb] = -1.0e30f;
      lsum[mb] = 0.f;
#pragma unroll
      for (int db = 0; db < 8; ++db) acc[mb][db] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  };
  reset_state();

  // Direct-to-LDS staging of one tensor's tile by one team: wave instruction
  // i of team wave w writes tile rows 16w + 4i .. +3 (same swizzles and
  // source offsets as the per-team kernel).
  const int dma0_k = (16 * w + kb) * kRowBytes + ((col ^ kb) << 4);
  const int dma0_v = (16 * w + kb) * kRowBytes + ((col ^ (2 * kb)) << 4);
  auto dma_tile = [&](auto is_v, const unsigned char* base, int tile, unsigned char* slot)
                      __attribute__((always_inline)) {
    constexpr bool V = decltype(is_v)::value;
    const int valid_rows = kv_len - tile * kBN;  // >= 1 for every tile issued
    __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(base) + (size_t)tile * kTileBytes, (short)0,
        valid_rows * kRowBytes, kBufferWord3);
    int o = V ? dma0_v : dma0_k;
    asm volatile("" : "+v"(o));
    lds_void* const dst = (lds_void*)(slot + 4 * w * 1024);
    constexpr int c1 = V ? 8 : 4, c2 = V ? 1 : 8, c3 = V ? 9 : 12;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, o, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, o ^ (c1 << 4), 0, 1024, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, o ^ (c2 << 4), 0, 2048, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, o ^ (c3 << 4), 0, 3072, 0);
  };
  const std::true_type is_v;
  const std::false_type is_k;

  int kfrag0, vfrag0;
  {
    kfrag0 = col * kRowBytes + ((col >> 2) << 6) + ((kb ^ (col & 3)) << 4);
    const int vr = 4 * kb + (col >> 2), e = col & 3, sv = swz_v(vr);
    vfrag0 = vr * kRowBytes + ((vr & 7) << 5) + (((e >> 1) ^ (sv & 1)) << 4) + ((e & 1) << 3);
  }

  floatx4 sc[2][4];
  half8 pf[2][2];

  auto g_phase = [&](auto with_qk, const unsigned char* kread, const unsigned char* vread)
                     __attribute__((always_inline)) {
    constexpr bool QK = decltype(with_qk)::value;
    __builtin_amdgcn_s_setprio(1);
    int vbase = vfrag0, kbase = kfrag0;
    asm volatile("" : "+v"(vbase), "+v"(kbase));
    half8 vf[8][2];
    half8 kf[4][4];
    auto read_v = [&](int db) __attribute__((always_inline)) {
      const int vo = vbase ^ (db << 5);
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const half4 lo = lds_read_tr16(vread + vo + 32 * cc * kRowBytes);
        const half4 hi = lds_read_tr16(vread + vo + (32 * cc + 16) * kRowBytes);
        vf[db][cc] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    };
    auto read_k = [&](int pb, int c) __attribute__((always_inline)) {
      kf[pb][c] = as_half8(*reinterpret_cast<const u32x4*>(kread + (kbase ^ (c << 6)) + 16 * pb * kRowBytes));
    };
#pragma unroll
    for (int db = 0; db < 4; ++db) read_v(db);
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        acc[mb][db] = mfma16x16x32(vf[db][0], pf[mb][0], acc[mb][db]);
        acc[mb][db] = mfma16x16x32(vf[db][1], pf[mb][1], acc[mb][db]);
      }
      if (db + 4 < 8) {
        read_v(db + 4);
      } else if constexpr (QK) {
        const int i = db - 4;
        read_k(i >> 1, 2 * (i & 1));
        read_k(i >> 1, 2 * (i & 1) + 1);
      }
    }
    if constexpr (QK) {
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          __builtin_amdgcn_sched_barrier(0);
          floatx4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < 4; ++c) a = mfma16x16x32(kf[pb][c], qf[mb][c], a);
          sc[mb][pb] = a;
          if (pb < 2) {
            read_k(pb + 2, 2 * mb);
            read_k(pb + 2, 2 * mb + 1);
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
  };
  auto qk_only = [&](const unsigned char* kread) __attribute__((always_inline)) {
    int kbase = kfrag0;
    asm volatile("" : "+v"(kbase));
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      half8 kf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kf[c] = as_half8(*reinterpret_cast<const u32x4*>(kread + (kbase ^ (c << 6)) + 16 * pb * kRowBytes));
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        floatx4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) a = mfma16x16x32(kf[c], qf[mb][c], a);
        sc[mb][pb] = a;
      }
    }
  };

  // S phase of tile j: this team's share of the staging (team A: K(j+2),
  // team B: V(j+2); repeats of the last tile past the end go to slots that
  // are not read again, so every S phase issues exactly 4 loads per wave),
  // the second block's Q when tile j+1 starts it, then mask and softmax.
  // Ends with this wave's loads of its previous S phase complete.
  auto s_phase = [&](int j, unsigned char* kfill, unsigned char* vfill) __attribute__((always_inline)) {
    if (j + 1 == th && tl > 0) load_q(l);
    const int tnext = tile_at(min(j + 2, n - 1));
    if (team == 0)
      dma_tile(is_k, kh, tnext, kfill);
    else
      dma_tile(is_v, vh, tnext, vfill);
    const int kv0 = tile_at(j) * kBN;
    const int qrow0 = pos0 + qb_at(j) * BQ2;  // first query position of the block
    if (kv0 + kBN - 1 > qrow0 + team * BQ) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const int lim = qrow0 + rpos(mb) - kv0 - 4 * kb;
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (16 * pb + i > lim) sc[mb][pb][i] = -__builtin_inff();
      }
    }
    float ts[2];
    auto probs = [&]() __attribute__((always_inline)) {
      const half2v ones = {(half_t)1.f, (half_t)1.f};
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        float s = 0.f;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          half8 p;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              p[hh * 4 + i] = (half_t)fast_exp2(sc[mb][2 * cc + hh][i] * scale_log2 - m[mb]);
          pf[mb][cc] = p;
          s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 0, 1), ones, s, false);
          s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 2, 3), ones, s, false);
          s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 4, 5), ones, s, false);
          s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 6, 7), ones, s, false);
        }
        ts[mb] = s;
      }
    };
    probs();
    if (__any(ts[0] >= kSpecLimit || ts[1] >= kSpecLimit)) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        float t = fmaxf(sc[mb][0][0], sc[mb][0][1]);
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
#pragma unroll
          for (int i = (pb == 0 ? 2 : 0); i < 4; ++i) t = fmaxf(t, sc[mb][pb][i]);
        // (m + kPHeadroom is the running max; this form needs no register
        // for the constant)
        const float mnew = fmaxf(m[mb] + kPHeadroom, col_max(t) * scale_log2) - kPHeadroom;
        const float alpha = fast_exp2(m[mb] - mnew);
        m[mb] = mnew;
        lsum[mb] *= alpha;
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[mb][db] *= alpha;
      }
      probs();
    }
    lsum[0] += ts[0];
    lsum[1] += ts[1];
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  };

  auto write_rows = [&](int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const float lrow = col_sum(lsum[mb]);
      if (!row_valid(qb, mb)) continue;
      const float inv = 1.0f / lrow;
      half_t* orow = out + ((size_t)(qb * BQ2 + rpos(mb)) * Hq + rhead(mb)) * kHeadDim;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        half4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (half_t)(acc[mb][db][i] * inv);
        *reinterpret_cast<u32x2*>(orow + 16 * db + 4 * kb) = __builtin_bit_cast(u32x2, o);
      }
    }
  };

  auto g_step = [&](int j, const unsigned char* kread, const unsigned char* vread) __attribute__((always_inline)) {
    if (j + 1 < n)
      g_phase(std::true_type{}, kread, vread);
    else
      g_phase(std::false_type{}, kread, vread);
    if (j + 1 == th && tl > 0) {
      write_rows(h);
      reset_state();
    }
  };

  // ---- prologue: team A stages K(0) -> k0, K(1) -> k1, team B V(0) -> v0,
  // V(1) -> v1; team A loads its Q now, team B after the first barrier (it
  // idles one phase anyway) ----
  if (team == 0) {
    dma_tile(is_k, kh, tile_at(0), s_k0);
    dma_tile(is_k, kh, tile_at(min(1, n - 1)), s_k1);
    load_q(qb_at(0));
  } else {
    dma_tile(is_v, vh, tile_at(0), s_v0);
    dma_tile(is_v, vh, tile_at(min(1, n - 1)), s_v1);
  }
  wait_vm_all();
  lds_barrier();
  if (team == 1) {
    load_q(qb_at(0));
    lds_barrier();
  }
  qk_only(s_k0);
  lds_barrier();
  // Tile j: G reads K slot (j+1)%3 and V slot j%3; S stages into slot
  // (j+2)%3.  Three tiles per trip keep every slot a compile-time constant.
  for (int j = 0; j < n; j += 3) {
    s_phase(j, s_k2, s_v2);
    lds_barrier();
    g_step(j, s_k1, s_v0);
    lds_barrier();
    if (j + 1 < n) {
      s_phase(j + 1, s_k0, s_v0);
      lds_barrier();
      g_step(j + 1, s_k2, s_v1);
      lds_barrier();
      if (j + 2 < n) {
        s_phase(j + 2, s_k1, s_v1);
        lds_barrier();
        g_step(j + 2, s_k0, s_v2);
        lds_barrier();
      }
    }
  }
  if (team == 0) lds_barrier();  // team B runs one phase more
  // Loads of the last S phases may still target LDS: drain before exiting.
  wait_vm_all();
  write_rows(tl > 0 ? l : h);
}

// GROUT_FMHA_PREFILL_PAIRED=0/1 forces the single-block / paired work split
// of the per-team kernel, GROUT_FMHA_PREFILL_WAVE_ROWS=16/32 its 64-row /
// 128-row blocks, GROUT_FMHA_PREFILL_SHARED=0/1 the per-team / shared-stream
// kernel (tests exercise every form); plan_fmha_prefill picks one by default.
static int env_override(const char* name) {
  const char* e = std::getenv(name);
  return e ? std::atoi(e) : -1;
}

PrefillPlan plan_fmha_prefill(int seq_len, int Hq, int Hkv) {
  const int G = Hq / Hkv;
  int HG = 8;
  while (G % HG != 0) --HG;
  const int BQ = kRowsPerTeam / HG;
  const int per_block = Hkv * (G / HG);
  // Work splits (one 512-thread workgroup per CU at a time, 256 CUs).  Pairs
  // of complementary blocks give every workgroup the same work, so a pair
  // form is taken when its workgroups fill the CUs: 192-256 of them (one
  // round), or at least 90% of the CU rounds they take (a second round that is
  // only partly full costs a whole pair's time).  Large blocks first (less
  // staging per FLOP): the shared stream (256-row blocks), per-team 128-row
  // pairs, per-team 64-row pairs (one round only: their half-size MFMA work
  // per tile loses to 128-row blocks once the GPU is full).  Otherwise single
  // blocks, heaviest first, which the dispatcher balances like a longest-first
  // list schedule: 128-row blocks when there are at least 192 of them, else
  // 64-row blocks.  Measured over S = 256-8192 at G = 4 and 8 (Qwen3-4B and
  // -32B heads): the pick is the fastest of the six forms or within 2% of it
  // at every length.
  constexpr long kCUs = 256;
  auto fills = [&](long wgs) {
    if (wgs <= kCUs) return 4 * wgs >= 3 * kCUs;
    const long rounds = (wgs + kCUs - 1) / kCUs;
    return 10 * wgs >= 9 * kCUs * rounds;
  };
  auto blocks_of = [&](int bq) { return (long)((seq_len + bq - 1) / bq) * per_block; };
  auto pairs_of = [&](int bq) { return (long)(((seq_len + bq - 1) / bq + 1) / 2) * per_block; };
  const int BQ64 = (kRowsPerTeam / 2) / HG;  // positions per 64-row block
  PrefillPlan p;
  p.HG = HG;
  p.nqb2 = (seq_len + 2 * BQ - 1) / (2 * BQ);
  p.shared = fills(pairs_of(2 * BQ));
  if (const int o = env_override("GROUT_FMHA_PREFILL_SHARED"); o == 0 || o == 1) p.shared = o;
  auto pairs_fill = [&](int rows) {
    return rows == 32 ? fills(pairs_of(BQ)) : pairs_of(BQ64) <= kCUs && fills(pairs_of(BQ64));
  };
  p.wave_rows =
      pairs_fill(32) ? 32 : pairs_fill(16) ? 16 : blocks_of(BQ) >= 3 * kCUs / 4 ? 32 : 16;
  if (const int o = env_override("GROUT_FMHA_PREFILL_WAVE_ROWS"); o == 16 || o == 32)
    p.wave_rows = o;
  const int BQr = p.wave_rows == 32 ? BQ : BQ64;
  p.nqb = (seq_len + BQr - 1) / BQr;
  // The shared stream's pairs take the whole GPU only in full rounds; with
  // 192-255 of them (one partial round) its single blocks, heaviest first,
  // finish sooner (measured 3-10%).
  p.paired = p.shared ? (pairs_of(2 * BQ) >= kCUs ? 1 : 0) : pairs_fill(p.wave_rows);
  if (const int o = env_override("GROUT_FMHA_PREFILL_PAIRED"); o == 0 || o == 1) p.paired = o;
  if (p.shared)
    p.workgroups = p.paired ? pairs_of(2 * BQ) : blocks_of(2 * BQ);
  else
    p.workgroups = (p.paired ? (p.nqb + 1) / 2 : p.nqb) * (long)per_block;
  return p;
}

hipError_t launch_fmha_prefill(const void* q, const void* k_cache, const void* v_cache,
                               void* out, int seq_len, int pos0, int Hq, int Hkv,
                               long head_stride, float qk_scale, hipStream_t stream) {
  const float scale_log2 = qk_scale * 1.4426950408889634f;
  const PrefillPlan p = plan_fmha_prefill(seq_len, Hq, Hkv);
  const long blocks = p.workgroups;
  const int shared = p.shared, wave_rows = p.wave_rows, paired = p.paired, nqbr = p.nqb,
            nqb2 = p.nqb2;
  if (blocks <= 0 || blocks > 0x7fffffffL) return hipErrorInvalidValue;
  const BlockMap bm{Hq / Hkv, make_div(Hkv), make_div(Hq / Hkv / p.HG)};
#define GROUT_PREFILL_CASE(hg)                                                             \
  case hg:                                                                                 \
    if (shared)                                                                            \
      fmha_prefill_shared_kernel<hg><<<(unsigned)blocks, 512, 0, stream>>>(                \
          (const half_t*)q, (const half_t*)k_cache, (const half_t*)v_cache, (half_t*)out,  \
          seq_len, pos0, Hq, Hkv, head_stride, scale_log2, nqb2, paired);                  \
    else if (wave_rows == 32)                                                              \
      fmha_prefill_kernel<hg, 2><<<(unsigned)blocks, 512, 0, stream>>>(                    \
          (const half_t*)q, (const half_t*)k_cache, (const half_t*)v_cache, (half_t*)out,  \
          seq_len, pos0, Hq, Hkv, head_stride, scale_log2, nqbr, paired, bm);                  \
    else                                                                                   \
      fmha_prefill_kernel<hg, 1><<<(unsigned)blocks, 512, 0, stream>>>(                    \
          (const half_t*)q, (const half_t*)k_cache, (const half_t*)v_cache, (half_t*)out,  \
          seq_len, pos0, Hq, Hkv, head_stride, scale_log2, nqbr, paired, bm);                  \
    break;
  switch (p.HG) {
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
