/*
 * grout_attn.h -- C ABI of the MI355X-native (gfx950) attention hot path of
 * grout (rtburger/grout).  Plain C: pointers, sizes and status codes only.
 *
 * Conventions
 *  - Every device pointer is caller-owned; head_dim must be 128 (the reference
 *    enforces it at load, src/model.rs:1446).  fp16 tensors are passed as
 *    `void*` to 16-byte-aligned device memory.
 *  - KV caches use the reference layout [num_kv_heads][max_ctx][128] fp16
 *    (src/model.rs:1587-1592).  `kv_head_stride` is the element distance
 *    between kv heads (max_ctx*128 for such a cache).
 *  - `stream` is a hipStream_t (NULL = default stream).  Every call is
 *    asynchronous on that stream, allocates nothing, never synchronizes and
 *    never reads device memory on the host, so it can be captured in a HIP
 *    graph.  Calls are re-entrant; the only global state is a thread-local
 *    error message.
 *  - Return value: 0 on success, < 0 for an invalid argument (shape, stride,
 *    alignment; the message is in grout_last_error()), > 0 a hipError_t.
 *    This mirrors the reference's `ensure!` before every launch
 *    (e.g. src/model.rs:4771-4854) and its anyhow::Result errors.
 */
#ifndef GROUT_ATTN_H
#define GROUT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GROUT_OK 0
#define GROUT_EINVAL (-1)   /* bad shape / count / range                */
#define GROUT_EALIGN (-2)   /* pointer or stride not 16-byte aligned    */
#define GROUT_ENOTSUP (-3)  /* configuration this build does not handle */

/* Largest cache length (max_ctx, or pos0 + seq_len for prefill) any entry
 * point accepts: the kernels address cache rows and rope-table rows with
 * 32-bit byte offsets. */
#define GROUT_MAX_CTX (1 << 22)

/* Largest decode split count (num_splits) any entry point accepts. */
#define GROUT_MAX_SPLITS 4096

/* Message of the last failing call on this thread ("" if none). */
const char* grout_last_error(void);

/* ABI version of this library: (major << 16) | minor. */
int grout_abi_version(void);

/* ------------------------------------------------------------------ */
/* RoPE (a9)                                                          */
/* ------------------------------------------------------------------ */

/* Host function. inv_freq[i/2] = 1 / theta^(i/head_dim), i = 0,2,..., in f32.
 * Replaces build_inv_freq (src/model.rs:7295-7306). */
int grout_rope_inv_freq(int head_dim, float theta, float* inv_freq);

/* Host function. cos/sin of the f32 angle (float)pos * inv_freq[i] for
 * pos in [0, max_ctx), layout [max_ctx][head_dim/2] f32, each evaluated in
 * double and rounded once.  The device kernels read these tables instead of
 * evaluating cos/sin (the reference evaluates them per element,
 * src/kernels.rs:5076-5082), which makes K-cache rows reproducible bit for
 * bit on the CPU.  Upload the two arrays once per model. */
int grout_rope_table_host(int max_ctx, int head_dim, float theta, float* cos_out,
                          float* sin_out);

/* ------------------------------------------------------------------ */
/* Fused QK-RMSNorm + RoPE + KV-cache write (a1, a2)                   */
/* ------------------------------------------------------------------ */

/* Prefill: q [seq_len][Hq][128], k, v [seq_len][Hkv][128] (the projection
 * outputs), gamma_q/gamma_k [128] fp16, rope tables [max_ctx][64] f32.
 * Writes q_out [seq_len][Hq][128] and cache rows pos0 .. pos0+seq_len-1 of
 * every kv head.  Requires pos0 + seq_len <= max_ctx.
 * Replaces qk_norm_rope_kv_prefill_raw_f16 (src/kernels.rs:4837-5168) as
 * launched by execute_qk_norm_rope_kv_prefill_op_ctx (src/model.rs:4753-4888),
 * i.e. GraphOp::QkNormRopeKvPrefill (src/model.rs:773-779). */
int grout_qk_norm_rope_kv_prefill(const void* q, const void* k, const void* v,
                                  const void* gamma_q, const void* gamma_k,
                                  const float* rope_cos, const float* rope_sin, void* q_out,
                                  void* k_cache, void* v_cache, int pos0, int seq_len,
                                  int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                                  long kv_head_stride, float eps, void* stream);

/* Decode: qkv = [Q (Hq*128) | K (Hkv*128) | V (Hkv*128)] contiguous (the QKV
 * GEMV output), position read from device memory d_pos[0] (u32).  Writes
 * q_out [Hq][128] and cache row d_pos[0] of every kv head; a position
 * >= max_ctx writes nothing.
 * Replaces qk_norm_rope_kv_decode_raw_f16 (src/kernels.rs:5170-5452) as
 * recorded in the decode graph (src/model.rs:3492-3519). */
int grout_qk_norm_rope_kv_decode(const void* qkv, const void* gamma_q, const void* gamma_k,
                                 const float* rope_cos, const float* rope_sin, void* q_out,
                                 void* k_cache, void* v_cache, const uint32_t* d_pos,
                                 int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                                 long kv_head_stride, float eps, void* stream);

/* ------------------------------------------------------------------ */
/* Causal GQA prefill attention (a3, a4, a7)                           */
/* ------------------------------------------------------------------ */

/* q [seq_len][Hq][128] post-RoPE, caches [Hkv][..][128] with
 * kv_head_stride, out [seq_len][Hq][128].  Row s attends to kv positions
 * 0 .. pos0+s (kv_len = pos0 + seq_len); kv head of q head h is h / (Hq/Hkv).
 * qk_scale is normally 1/sqrt(128).
 * Replaces fmha_prefill_causal / fmha_prefill_gqa / fmha_prefill_gqa_lpt
 * (src/kernels.rs:2559-3298) as dispatched for GraphOp::Attention with a host
 * position by attend_seq_arc_into_ctx_with_position (src/model.rs:6856-7134). */
int grout_fmha_prefill(const void* q, const void* k_cache, const void* v_cache, void* out,
                       int seq_len, int pos0, int num_q_heads, int num_kv_heads, int head_dim,
                       long kv_head_stride, float qk_scale, void* stream);

/* The work split grout_fmha_prefill launches for seq_len query rows (host
 * only, no GPU; the GROUT_FMHA_PREFILL_SHARED / _PAIRED / _WAVE_ROWS test
 * overrides apply): *form = 0 the shared K/V stream (256-row q blocks), 1 the
 * per-team kernel with 128-row q blocks, 2 with 64-row q blocks; *paired = 1
 * for complementary block pairs, 0 for single blocks (heaviest first); *workgroups = the grid size.  Any output pointer may be NULL;
 * 1 <= seq_len <= GROUT_MAX_CTX.
 * Stands in for the tile and kernel choice of
 * attend_seq_arc_into_ctx_with_position (src/model.rs:6905-6927, 6946-7079). */
int grout_fmha_prefill_plan(int seq_len, int num_q_heads, int num_kv_heads, int* form,
                            int* paired, long* workgroups);

/* ------------------------------------------------------------------ */
/* Split-K GQA decode attention + LSE merge (a5, a6)                   */
/* ------------------------------------------------------------------ */

/* Split count the library picks for a live context of ctx_len positions
 * (the reference's FMHA_NUM_KV_SPLITS default / per-context overrides,
 * src/model.rs:135-141): 1 up to 128 positions, else one split per 32
 * positions, at most ceil(256 / num_kv_heads) (one workgroup per CU). */
int grout_attn_decode_default_splits(int ctx_len, int num_q_heads, int num_kv_heads);

/* Bytes of fp32 scratch grout_attn_decode needs for num_splits splits:
 * partial accumulators [Hkv][splits][G][128] + (m, sum) [Hkv][splits][G][2].
 * Calls sharing one workspace must not overlap in time. */
size_t grout_attn_decode_workspace_bytes(int num_q_heads, int num_kv_heads, int head_dim,
                                         int num_splits);

/* q [Hq][128] post-RoPE (q head h = kvh*G + g, i.e. the [Hkv][G][128] grouped
 * view), caches [Hkv][..][128], out [Hq][128].  Attends to positions
 * 0 .. d_pos[0] (s_kv = d_pos[0]+1, clamped to max_ctx).  num_splits <= 0
 * picks grout_attn_decode_default_splits(max_ctx, ...); at most
 * GROUT_MAX_SPLITS, and splits past the context's tiles stay empty.  Two launches
 * (split pass, then the merge) on `stream`.
 * Replaces fmha_decode_gqa_split + splitk_reduce_merge
 * (src/kernels.rs:3996-4304) as recorded in src/model.rs:3713-3771. */
int grout_attn_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
                      void* workspace, size_t workspace_bytes, const uint32_t* d_pos,
                      int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                      long kv_head_stride, int num_splits, float qk_scale, void* stream);

/* Bytes of the static device scratch of grout_attn_decode_noalloc (per GPU). */
#define GROUT_NOALLOC_SCRATCH_BYTES (4 << 20)

/* grout_attn_decode without a workspace and without any allocation.  No
 * counterpart in the reference: this entry point is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The split partials live in a static
 * device array of GROUT_NOALLOC_SCRATCH_BYTES (4 MiB) that each GPU the
 * library runs on holds until the process ends; a call whose
 * grout_attn_decode_workspace_bytes(..., num_splits) exceeds that fails with
 * GROUT_EINVAL before launching.  The first call on a device looks the array's
 * address up (hipGetSymbolAddress); make that first call outside graph
 * capture.  Every call on one GPU shares its array: calls that overlap in
 * time on one GPU (other streams, other threads) race.  Output is
 * bit-identical to grout_attn_decode's with the same num_splits. */
int grout_attn_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, void* out,
                              const uint32_t* d_pos, int num_q_heads, int num_kv_heads,
                              int head_dim, int max_ctx, long kv_head_stride, int num_splits,
                              float qk_scale, void* stream);

/* The two halves of grout_attn_decode, for callers that schedule them
 * separately (the reference records them as two kernels).  part_acc
 * [Hkv][splits][G][128] fp32 unnormalized, part_ml [Hkv][splits][G][2] fp32
 * (reference point m in log2 units, the split's running max minus 7, and
 * the sum of 2^(s - m); the merge needs only that m and that sum agree). */
int grout_fmha_decode_gqa_split(const void* q, const void* k_cache, const void* v_cache,
                                float* part_acc, float* part_ml, const uint32_t* d_pos,
                                int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                                long kv_head_stride, int num_splits, float qk_scale,
                                void* stream);
int grout_splitk_reduce_merge(const float* part_acc, const float* part_ml, void* out,
                              int num_q_heads, int num_kv_heads, int head_dim, int num_splits,
                              void* stream);

/* One layer's attention of a decode step in one launch (two with more than
 * one split): the QK-RMSNorm + RoPE of the new token's q heads and K head and
 * the K/V cache write at d_pos[0] (grout_qk_norm_rope_kv_decode), then the
 * split-K attention over positions 0 .. d_pos[0] (grout_attn_decode), with
 * the rotated q rows kept on chip.  qkv, gammas, rope tables and caches as in
 * grout_qk_norm_rope_kv_decode; out [Hq][128].  num_splits == 1 writes out
 * directly (no workspace needed, workspace may be NULL); num_splits > 1 uses
 * grout_attn_decode_workspace_bytes(..., num_splits) of workspace and adds
 * the merge launch; num_splits <= 0 picks the default for max_ctx.  A
 * position >= max_ctx writes nothing.  K/V cache rows are bit-identical to
 * grout_qk_norm_rope_kv_decode's.
 * Replaces the decode graph's qk_norm_rope_kv_decode_raw_f16 +
 * fmha_decode_gqa_split + splitk_reduce_merge records (src/model.rs:3492-3519,
 * 3713-3771; src/kernels.rs:3996-4304, 5170-5452). */
int grout_attn_decode_fused(const void* qkv, const void* gamma_q, const void* gamma_k,
                            const float* rope_cos, const float* rope_sin, void* k_cache,
                            void* v_cache, void* out, void* workspace, size_t workspace_bytes,
                            const uint32_t* d_pos, int num_q_heads, int num_kv_heads,
                            int head_dim, int max_ctx, long kv_head_stride, int num_splits,
                            float eps, float qk_scale, void* stream);

/* ------------------------------------------------------------------ */
/* Decode-step graph (a8)                                              */
/* ------------------------------------------------------------------ */

/* Per-layer buffers of the attention part of one decode step. */
typedef struct grout_decode_layer {
  const void* qkv;      /* [(Hq+2Hkv)*128] fp16 input of the fused norm/RoPE/KV write */
  const void* gamma_q;  /* [128] fp16 */
  const void* gamma_k;  /* [128] fp16 */
  void* q_rope;         /* unused (the rotated q rows stay on chip); may be NULL */
  void* k_cache;        /* [Hkv][max_ctx][128] fp16 */
  void* v_cache;        /* [Hkv][max_ctx][128] fp16 */
  void* attn_out;       /* [Hq][128] fp16 */
} grout_decode_layer;

typedef struct grout_decode_graph grout_decode_graph;

/* Captures num_layers x grout_attn_decode_fused (the fused norm/RoPE/KV
 * write + split-K pass, then the merge: two launches per layer, one with a
 * single split) into one HIP graph.  The capture runs on `stream`, or on a
 * private stream when `stream` is NULL (the legacy stream cannot be
 * captured); nothing is executed on `stream` by this call.  Creation is not
 * a hot call: it allocates the graph's device position word (hipMalloc) and
 * zeroes it synchronously before the capture.  The graph reads the position
 * from that word, written by grout_decode_graph_launch; `workspace`
 * (grout_attn_decode_workspace_bytes(..., num_splits)) is shared by the
 * layers, which run in order.  num_splits <= 0 picks the default for max_ctx.
 * Replaces DecodeCudaGraphRunner / build_decode_graph_scope
 * (src/model.rs:408-596, 2631-4006) for the attention records
 * (src/model.rs:3492-3519, 3713-3771). */
int grout_decode_graph_create(const grout_decode_layer* layers, int num_layers,
                              const float* rope_cos, const float* rope_sin, void* workspace,
                              size_t workspace_bytes, int num_q_heads, int num_kv_heads,
                              int head_dim, int max_ctx, int num_splits, float eps,
                              float qk_scale, void* stream, grout_decode_graph** out);

/* Launches the graph for `position` (host-checked: position < max_ctx) on
 * `stream`; asynchronous.  With more than one split the last layer's merge
 * leaves position + 1 in the graph's device word, so a launch at the
 * previous launch's position + 1 is a single hipGraphLaunch; any other
 * position is first written into the word by a one-thread kernel.  Launches
 * of one graph must be ordered (one stream, or ordered by the caller), as
 * its layers share the workspace anyway.
 * Mirrors DecodeCudaGraphRunner::launch_step (src/model.rs:466-506). */
int grout_decode_graph_launch(grout_decode_graph* graph, uint32_t position, void* stream);

/* Device address of the graph's position word (u32), for callers that chain
 * their own kernels on it: it reads `position` while the graph runs and,
 * with more than one split, position + 1 after it.  The graph owns the word:
 * callers only read it. */
const uint32_t* grout_decode_graph_position_ptr(const grout_decode_graph* graph);

int grout_decode_graph_destroy(grout_decode_graph* graph);

/* ------------------------------------------------------------------ */
/* Diagnostics                                                         */
/* ------------------------------------------------------------------ */

/* Runs one v_mfma_f32_16x16x32_f16 with A[l][i] = 8l+i and a 0/1 selector B,
 * writing the 64x4 C fragment to out (device, 256 floats).  Confirms the
 * operand/accumulator lane layout every kernel here assumes. */
int grout_diag_mfma_layout(float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GROUT_ATTN_H */
