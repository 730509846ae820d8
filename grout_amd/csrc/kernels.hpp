// Internal launch functions (C++ linkage) called by the C ABI layer in api.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace grout {

// ldq / ldkv: elements from one token's q (k, v) rows to the next; 0 = packed
// (Hq * 128, Hkv * 128), e.g. Hq*128 + 2*Hkv*128 for rows of a fused QKV output.
hipError_t launch_qk_norm_rope_kv_prefill(const void* q, const void* k, const void* v,
                                          const void* gamma_q, const void* gamma_k,
                                          const float* rope_cos, const float* rope_sin,
                                          void* q_out, void* k_cache, void* v_cache, int pos0,
                                          int seq_len, int Hq, int Hkv, long head_stride,
                                          int max_ctx, float eps, hipStream_t stream,
                                          long ldq = 0, long ldkv = 0);

hipError_t launch_qk_norm_rope_kv_decode(const void* qkv, const void* gamma_q,
                                         const void* gamma_k, const float* rope_cos,
                                         const float* rope_sin, void* q_out, void* k_cache,
                                         void* v_cache, const uint32_t* d_pos, int Hq, int Hkv,
                                         long head_stride, int max_ctx, float eps,
                                         hipStream_t stream);

// Split pass: part_acc [Hkv][nsplit][G][128] fp32 (unnormalized), part_ml
// [Hkv][nsplit][G][2] fp32 (running max in log2 units, sum of exp2).
hipError_t launch_attn_decode_split(const void* q, const void* k_cache, const void* v_cache,
                                    long head_stride, const uint32_t* d_pos, int max_ctx,
                                    int Hq, int Hkv, int nsplit, float qk_scale,
                                    float* part_acc, float* part_ml, hipStream_t stream);

// Fused decode step of one layer: QK-RMSNorm + RoPE of the new token's q
// rows and K row, K/V cache write at d_pos[0], and split-K attention; one
// split (nsplit == 1) writes out directly, more splits add the merge launch.
// advance_pos (nsplit > 1 only, else ignored; may be NULL): the merge adds
// one to *advance_pos once every split has read the position, so a captured
// step can leave the next step's position behind.
hipError_t launch_attn_decode_fused(const void* qkv, const void* gamma_q, const void* gamma_k,
                                    const float* rope_cos, const float* rope_sin, void* k_cache,
                                    void* v_cache, long head_stride, const uint32_t* d_pos,
                                    int max_ctx, int Hq, int Hkv, int nsplit, float eps,
                                    float qk_scale, float* part_acc, float* part_ml, void* out,
                                    hipStream_t stream, uint32_t* advance_pos = nullptr);
hipError_t launch_attn_decode_merge(const float* part_acc, const float* part_ml, void* out,
                                    int Hq, int Hkv, int nsplit, hipStream_t stream,
                                    uint32_t* advance_pos = nullptr);

// Work split of the causal prefill FMHA for one launch (host side, no GPU):
// shared K/V stream (256-row q blocks, pairs) or the per-team kernel with
// wave_rows = 32 (128-row blocks) or 16 (64-row blocks), single blocks or
// complementary pairs; HG heads per q block, nqb (nqb2) blocks per kv head
// group of the per-team (shared) form, workgroups = grid size.
struct PrefillPlan {
  int HG = 1, shared = 0, wave_rows = 32, paired = 0, nqb = 0, nqb2 = 0;
  long workgroups = 0;
};
PrefillPlan plan_fmha_prefill(int seq_len, int Hq, int Hkv);
hipError_t launch_fmha_prefill(const void* q, const void* k_cache, const void* v_cache,
                               void* out, int seq_len, int pos0, int Hq, int Hkv,
                               long head_stride, float qk_scale, hipStream_t stream);

// Model-step kernels (model_kernels.hip).  residual == nullptr selects plain
// RMSNorm; otherwise out = norm(residual + x), residual_out = residual + x.
hipError_t launch_embedding(const uint32_t* ids, const void* table, void* out, int rows, int H,
                            int vocab, hipStream_t stream);
hipError_t launch_rms_norm(const void* residual, const void* x, const void* w, void* out,
                           void* residual_out, int rows, int H, float eps, hipStream_t stream);
hipError_t launch_silu_mul(const void* gate_up, void* out, int rows, int I, hipStream_t stream);
hipError_t launch_gemv(const void* W, const void* x, void* y, int N, int K, hipStream_t stream);
// GEMV whose input is the RMSNorm (residual == nullptr) or add-RMSNorm of x,
// computed per wave; the first wave writes residual_out = residual + x.
// silu_pairs: W holds 2N rows [gate | up] and y[n] = silu(gate_n) * up_n.
hipError_t launch_gemv_norm(const void* W, const void* residual, const void* x, const void* gamma,
                            void* residual_out, float eps, void* y, int N, int K, bool silu_pairs,
                            hipStream_t stream);
int argmax_num_blocks(int V);
// dst[i] = f16(src[i]) for n elements of dtype 0 = f16, 1 = bf16, 2 = f32,
// 3 = f64 (through f32), round to nearest even.
hipError_t launch_convert_to_f16(const void* src, int dtype, size_t n, void* dst,
                                 hipStream_t stream);
// Greedy token of V f16 logits into out[0]; advance_pos (may be NULL) is
// incremented by the same thread, for a captured decode step that leaves the
// next step's token and position behind.
hipError_t launch_argmax(const void* logits, float* block_max, uint32_t* block_idx, int V,
                         uint32_t* out, hipStream_t stream, uint32_t* advance_pos = nullptr);

// Low-bit decode GEMVs (quant_gemv.hip); fmt is the ggml type id: 8 = Q8_0,
// 12 = Q4_K, 14 = Q6_K.  Weights in the repacked layout (qweight_bytes).
size_t qweight_bytes(int fmt, int N, int K);
hipError_t launch_qweight_repack(int fmt, const void* ggml_blocks, int N, int K, void* dst,
                                 hipStream_t stream);
// silu: W holds 2N rows [gate | up] and y[n] = silu(gate_n) * up_n.
hipError_t launch_gemv_q(int fmt, const void* W, const void* x, void* y, int N, int K, bool silu,
                         hipStream_t stream);
// As launch_gemv_q with the input RMSNorm folded in: x' = f16(x * inv *
// gamma) (residual NULL) or, for c = residual + x, x' = f16(c * inv * gamma)
// with f16(c) written to residual_out when it is not NULL.
hipError_t launch_gemv_q_norm(int fmt, const void* W, const void* residual, const void* x,
                              const void* gamma, void* residual_out, float eps, void* y, int N,
                              int K, bool silu, hipStream_t stream);
// out[t] = row ids[t] of the N x K matrix as f16 (CPU dequantization rule).
hipError_t launch_qgather(int fmt, const void* W, int N, int K, const uint32_t* ids, int rows,
                          void* out, hipStream_t stream);
hipError_t launch_qweight_dequant(int fmt, const void* W, int N, int K, void* out,
                                  hipStream_t stream);

// Writes the 16x16 C fragment of A x B for A[i][k] = i*32+k (k < 32), B = I
// padded, one float per (lane, element): used to confirm the MFMA lane layout.
hipError_t launch_mfma_layout_probe(float* out64x4, hipStream_t stream);

}  // namespace grout
