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
//  * a wave consumes 32-position tiles (tile index t = t0 + wave + 4i, so the
//    four waves of a workgroup stream adjacent tiles).  K and V rows are read
//    with lane-contiguous 16-byte non-temporal loads (each wave instruction
//    covers 1 KiB = 4 whole rows), the next tile is in flight while the
//    current one is computed, and each wave re-lays its tile out through a
//    private, XOR-swizzled LDS buffer into MFMA fragments (no workgroup
//    barrier in the loop).  Reading rows directly in fragment order (16 rows
//    x 64 B per instruction) measured ~15% below the lane-contiguous stream;
//  * S^T = K.Q^T on v_mfma_f32_16x16x32_f16: A = 16 K rows (the natural
//    row-major fragment), B = Q^T with the group's query heads as the 16
//    columns (G <= 16, padded with zeros);
//  * P.V needs V with positions along the reduction axis.  The row-major V
//    fragment is turned around in registers by multiplying it with a 0/1
//    selector on the MFMA unit (exact: every product is v*1 or v*0), which
//    yields V^T fragments in the C layout, converted back to f16 losslessly;
//  * O^T = V^T.P^T keeps each query head in one lane column, so the online
//    softmax statistics (max, sum) of head g live in the lanes that own its
//    accumulator: no cross-lane traffic for the rescale;
//  * the 4 waves merge through LDS at the end and write one fp32 partial
//    (unnormalized acc, max, sum) per (kv head, split, query head); a small
//    second kernel merges the splits.  (Merging in the last workgroup of each
//    kv head behind an atomic ticket measured slower on MI355X: the ticket
//    needs either an L2 write-back per workgroup or same-address agent-scope
//    atomics, both of which serialize at ~0.3-1 us per split.)
#include "common.hpp"
#include "kernels.hpp"

namespace grout {

constexpr int kTile = 32;  // kv positions per wave step
constexpr int kDecWaves = 4;

// One tile (32 rows of K and of V) as loaded: instruction i of lane l holds
// row 4i + l/16, 16-byte chunk l%16.
struct KvRegs {
  u32x4 k[8];
  u32x4 v[8];
};

__device__ __forceinline__ void load_kv_tile(KvRegs& r, const half_t* __restrict__ kh,
                                             const half_t* __restrict__ vh, int tile, int s_kv,
                                             int lane) {
  const int sub = lane >> 4, chunk = lane & 15;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int p = tile * kTile + 4 * i + sub;
    p = p < s_kv ? p : s_kv - 1;  // rows past the context are masked; read a live row instead
    r.k[i] = load_stream16(kh + (size_t)p * kHeadDim + chunk * 8);
    r.v[i] = load_stream16(vh + (size_t)p * kHeadDim + chunk * 8);
  }
}

// Wave-private LDS tile: [K rows 0..31 | V rows 0..31], 256 B per row, the
// 16-byte chunk c of row r stored at chunk slot c ^ (r & 15) so that both the
// row-contiguous stores and the 16-rows-per-chunk fragment reads are
// conflict-free.
constexpr int kTileBytes = 2 * kTile * kHeadDim * 2;  // 16 KiB

__device__ __forceinline__ int swz(int row, int chunk) { return row * 256 + ((chunk ^ (row & 15)) << 4); }

__device__ __forceinline__ void store_kv_tile(unsigned char* buf, const KvRegs& r, int lane) {
  const int sub = lane >> 4, chunk = lane & 15;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 4 * i + sub;
    *reinterpret_cast<u32x4*>(buf + swz(row, chunk)) = r.k[i];
    *reinterpret_cast<u32x4*>(buf + kTile * 256 + swz(row, chunk)) = r.v[i];
  }
}

// MFMA A fragment of 16 rows starting at row0 for d in [32c, 32c+32): lane l
// gets row row0 + l%16, chunk 4c + l/16.
__device__ __forceinline__ half8 frag(const unsigned char* base, int row0, int c, int lane) {
  const int row = row0 + (lane & 15);
  return as_half8(*reinterpret_cast<const u32x4*>(base + swz(row, 4 * c + (lane >> 4))));
}

struct DecState {
  float m;  // running max (log2 units) of this lane's query head column
  float l;  // this lane's partial sum of exp2 (reduced over the 4 lane groups at the end)
  floatx4 acc[8];  // O^T fragments: d = 16*db + 4*(lane/16) + i, head = lane%16
};

__device__ __forceinline__ void compute_kv_tile(DecState& st, const unsigned char* buf,
                                                const half8 (&qf)[4], const half8 (&sel)[2],
                                                int tile, int s_kv, float scale_log2, int lane) {
  const int kb = lane >> 4;
  const unsigned char* vbuf = buf + kTile * 256;
  floatx4 sc[2];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    floatx4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) a = mfma16x16x32(frag(buf, 16 * pb, c, lane), qf[c], a);
    sc[pb] = a;
  }
  float s[8];
  float tmax = -1.0e30f;
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pos = tile * kTile + pb * 16 + kb * 4 + i;
      float val = sc[pb][i] * scale_log2;
      val = pos < s_kv ? val : -1.0e30f;
      s[pb * 4 + i] = val;
      tmax = fmaxf(tmax, val);
    }
  }
  tmax = fmaxf(tmax, shfl_xor(tmax, 16));
  tmax = fmaxf(tmax, shfl_xor(tmax, 32));
  const float mnew = fmaxf(st.m, tmax);
  const float alpha = fast_exp2(st.m - mnew);
  half8 pf;
  float psum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = fast_exp2(s[e] - mnew);
    psum += p;
    pf[e] = (half_t)p;
  }
  st.l = st.l * alpha + psum;
  st.m = mnew;
#pragma unroll
  for (int db = 0; db < 8; ++db) st.acc[db] *= alpha;

  const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const floatx4 t0 = mfma16x16x32(frag(vbuf, 0, c, lane), sel[h], zero);
      const floatx4 t1 = mfma16x16x32(frag(vbuf, 16, c, lane), sel[h], zero);
      half8 vt;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        vt[i] = (half_t)t0[i];
        vt[4 + i] = (half_t)t1[i];
      }
      st.acc[2 * c + h] = mfma16x16x32(vt, pf, st.acc[2 * c + h]);
    }
  }
}

__global__ __launch_bounds__(kDecWaves * 64, 2) void attn_decode_split_kernel(
    const half_t* __restrict__ q, const half_t* __restrict__ k_cache,
    const half_t* __restrict__ v_cache, long head_stride, const uint32_t* __restrict__ d_pos,
    int max_ctx, int G, int nsplit, float scale_log2, float* __restrict__ part_acc,
    float* __restrict__ part_ml) {
  // Tile buffers during the loop; reused for the cross-wave merge afterwards.
  __shared__ __attribute__((aligned(16))) unsigned char s_tiles[kDecWaves * kTileBytes];
  __shared__ float s_ml[kDecWaves][16][2];
  float(*s_acc)[16][kHeadDim] = reinterpret_cast<float(*)[16][kHeadDim]>(s_tiles);

  const int split = blockIdx.x, kvh = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int col = lane & 15, kb = lane >> 4;

  const uint32_t pos = d_pos[0];
  const int s_kv = pos >= (uint32_t)max_ctx ? max_ctx : (int)pos + 1;  // always in [1, max_ctx]
  const int ntiles = (s_kv + kTile - 1) / kTile;
  const int per = (ntiles + nsplit - 1) / nsplit;
  const int t0 = split * per;
  const int t1 = min(t0 + per, ntiles);

  const half_t* kh = k_cache + (size_t)kvh * head_stride;
  const half_t* vh = v_cache + (size_t)kvh * head_stride;

  half8 qf[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (col < G) {
      qf[c] = as_half8(load16(q + ((size_t)kvh * G + col) * kHeadDim + c * 32 + kb * 8));
    } else {
      qf[c] = as_half8(u32x4{0u, 0u, 0u, 0u});
    }
  }
  half8 sel[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) sel[h][i] = (half_t)((kb * 8 + i == h * 16 + col) ? 1.0f : 0.0f);

  DecState st;
  st.m = -1.0e30f;
  st.l = 0.f;
#pragma unroll
  for (int db = 0; db < 8; ++db) st.acc[db] = floatx4{0.f, 0.f, 0.f, 0.f};

  unsigned char* buf = s_tiles + w * kTileBytes;
  KvRegs regs;
  int t = t0 + w;
  if (t < t1) load_kv_tile(regs, kh, vh, t, s_kv, lane);
  while (t < t1) {
    store_kv_tile(buf, regs, lane);  // program order keeps this wave's LDS reads after the stores
    const int tn = t + kDecWaves;
    if (tn < t1) load_kv_tile(regs, kh, vh, tn, s_kv, lane);
    compute_kv_tile(st, buf, qf, sel, t, s_kv, scale_log2, lane);
    t = tn;
  }
  __syncthreads();  // all waves are done with their tile buffers before s_acc reuses them

  // Per-wave statistics of head `col`, then merge the 4 waves through LDS.
  float l = st.l;
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
  if (kb == 0) {
    s_ml[w][col][0] = st.m;
    s_ml[w][col][1] = l;
  }
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_acc[w][col][db * 16 + kb * 4 + i] = st.acc[db][i];
  __syncthreads();

  const size_t base = ((size_t)kvh * nsplit + split) * G;
  for (int e = threadIdx.x; e < G * kHeadDim; e += kDecWaves * 64) {
    const int g = e / kHeadDim, d = e - g * kHeadDim;
    float M = s_ml[0][g][0];
#pragma unroll
    for (int ww = 1; ww < kDecWaves; ++ww) M = fmaxf(M, s_ml[ww][g][0]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int ww = 0; ww < kDecWaves; ++ww) {
      const float wgt = fast_exp2(s_ml[ww][g][0] - M);
      L += wgt * s_ml[ww][g][1];
      O += wgt * s_acc[ww][g][d];
    }
    part_acc[(base + g) * kHeadDim + d] = O;
    if (d == 0) {
      part_ml[(base + g) * 2 + 0] = M;
      part_ml[(base + g) * 2 + 1] = L;
    }
  }
}

// Merge: one 128-thread workgroup per (query head h = kvh*G + g, half of D).
// Thread t owns 4 consecutive d (one float4) and every 8th split, keeps its
// own running (max, sum, acc) so all its loads are independent, then the 8
// split groups combine through LDS.
constexpr int kMergeGroups = 8;

__global__ __launch_bounds__(128) void attn_decode_merge_kernel(
    const float* __restrict__ part_acc, const float* __restrict__ part_ml,
    half_t* __restrict__ out, int G, int nsplit) {
  __shared__ float s_m[kMergeGroups][16];
  __shared__ float s_l[kMergeGroups][16];
  __shared__ floatx4 s_o[kMergeGroups][16];
  const int h = blockIdx.x, half = blockIdx.y;
  const int kvh = h / G, g = h - kvh * G;
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
    const float so = exp2f(M - Mn), sn = exp2f(ml.x - Mn);
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
      const float wgt = exp2f(s_m[i][dq] - Mt);
      Lt += s_l[i][dq] * wgt;
      Ot += s_o[i][dq] * wgt;
    }
    const float inv = 1.0f / Lt;
    half4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (half_t)(Ot[i] * inv);
    *reinterpret_cast<u32x2*>(out + (size_t)h * kHeadDim + d0) = __builtin_bit_cast(u32x2, o);
  }
}

hipError_t launch_attn_decode_split(const void* q, const void* k_cache, const void* v_cache,
                                    long head_stride, const uint32_t* d_pos, int max_ctx,
                                    int Hq, int Hkv, int nsplit, float qk_scale,
                                    float* part_acc, float* part_ml, hipStream_t stream) {
  const float scale_log2 = qk_scale * 1.4426950408889634f;
  dim3 grid((unsigned)nsplit, (unsigned)Hkv);
  attn_decode_split_kernel<<<grid, kDecWaves * 64, 0, stream>>>(
      (const half_t*)q, (const half_t*)k_cache, (const half_t*)v_cache, head_stride, d_pos,
      max_ctx, Hq / Hkv, nsplit, scale_log2, part_acc, part_ml);
  return hipGetLastError();
}

hipError_t launch_attn_decode_merge(const float* part_acc, const float* part_ml, void* out,
                                    int Hq, int Hkv, int nsplit, hipStream_t stream) {
  attn_decode_merge_kernel<<<dim3((unsigned)Hq, 2), 128, 0, stream>>>(part_acc, part_ml,
                                                                      (half_t*)out, Hq / Hkv, nsplit);
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
