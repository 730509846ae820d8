/*
 * grout_engine.h -- C ABI of the Qwen3 decode/prefill engine built around the
 * gfx950 attention path of grout_attn.h (one GPU, fp16 weights).
 *
 * It replaces the reference's public Rust API `grout::Engine`
 * (src/api.rs:11-183) over Qwen3Engine (src/model.rs): a synchronous,
 * token-based engine.  Conventions are those of grout_attn.h (status codes,
 * grout_last_error()), with these differences:
 *  - The engine owns its KV caches, activation buffers, RoPE tables, one HIP
 *    stream, a rocBLAS handle (prefill GEMMs) and the captured decode-step
 *    HIP graph.  It borrows the weights: every weight pointer is caller-owned
 *    device memory that must stay valid until grout_engine_destroy.
 *  - Calls are blocking (they synchronize the engine's stream before
 *    returning, like Engine's block_on in src/api.rs:97-126) and must not be
 *    made concurrently on one engine.
 *  - Weight layouts are the reference's fused ones (src/model.rs weights):
 *    qkv_proj rows [Q (Hq*128) | K (Hkv*128) | V (Hkv*128)] x hidden,
 *    gate_up_proj rows [gate (inter) | up (inter)] x hidden, every matrix
 *    row-major [out_features][in_features] fp16, 16-byte aligned.
 */
#ifndef GROUT_ENGINE_H
#define GROUT_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#include "grout_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GROUT_EBLAS (-4) /* a rocBLAS call of the prefill failed (message in grout_last_error) */
#define GROUT_ENOMEM (-5) /* VRAM preflight: the engine would not fit in free device memory */

/* The Qwen3Config fields the engine reads (src/config.rs:7-33). */
typedef struct grout_qwen3_config {
  int num_layers;           /* num_hidden_layers */
  int hidden_size;          /* multiple of 8, at most 8192 */
  int intermediate_size;    /* multiple of 8 */
  int num_q_heads;          /* num_attention_heads */
  int num_kv_heads;         /* num_key_value_heads; Hq/Hkv <= 16 */
  int head_dim;             /* must be 128 */
  int vocab_size;
  float rms_norm_eps;       /* 1e-6 for Qwen3 */
  float rope_theta;         /* 1e6 for Qwen3 */
  int max_ctx;              /* allocated context (KV cache rows per layer) */
} grout_qwen3_config;

/* One decoder layer's weights (borrowed device pointers, fp16). */
typedef struct grout_qwen3_layer {
  const void* input_layernorm;           /* [hidden] */
  const void* qkv_proj;                  /* [(Hq+2Hkv)*128][hidden] */
  const void* q_norm;                    /* [128] */
  const void* k_norm;                    /* [128] */
  const void* o_proj;                    /* [hidden][Hq*128] */
  const void* post_attention_layernorm;  /* [hidden] */
  const void* gate_up_proj;              /* [2*inter][hidden] */
  const void* down_proj;                 /* [hidden][inter] */
} grout_qwen3_layer;

typedef struct grout_qwen3_weights {
  const void* embed_tokens;         /* [vocab][hidden] */
  const void* norm;                 /* [hidden], the final norm */
  const void* lm_head;              /* [vocab][hidden]; == embed_tokens when tied */
  const grout_qwen3_layer* layers;  /* num_layers entries (the array is copied) */
} grout_qwen3_weights;

/* ------------------------------------------------------------------ */
/* Step kernels around the attention path (device pointers, async on   */
/* `stream`, graph-capturable; fp16 rows of `hidden` elements)          */
/* ------------------------------------------------------------------ */

/* out[r] = table[ids[r]] for r < rows; ids is device memory (u32).  An id
 * >= vocab_size gives a zero row (the engine rejects such ids first).
 * Replaces embedding_f16 / embedding_batch_f16 (src/kernels.rs:1893-1938). */
int grout_embedding(const uint32_t* ids, const void* table, void* out, int rows, int hidden,
                    int vocab_size, void* stream);

/* out = f16(x * 1/sqrt(sum(x^2)/hidden + eps) * w) per row, fp32 math.
 * Replaces rms_norm_f16 (src/kernels.rs:1530-1569). */
int grout_rms_norm(const void* x, const void* w, void* out, int rows, int hidden, float eps,
                   void* stream);

/* c = residual + x (fp32); out = f16(c * 1/sqrt(sum(c^2)/hidden + eps) * w);
 * residual_out = f16(c).  residual_out may alias residual.
 * Replaces add_rms_norm_decode_raw_f16 (src/kernels.rs:4518-4657). */
int grout_add_rms_norm(const void* residual, const void* x, const void* w, void* out,
                       void* residual_out, int rows, int hidden, float eps, void* stream);

/* gate_up rows [gate (inter) | up (inter)] -> out rows f16(silu(gate) * up).
 * Replaces silu_mul_2d_f16 (src/kernels.rs:1493-1522). */
int grout_silu_mul(const void* gate_up, void* out, int rows, int inter, void* stream);

/* y[n] = sum_k W[n][k] x[k], W row-major [n][k] fp16, fp32 accumulation,
 * f16 out; k a multiple of 8.  Replaces the decode GEMVs (cuBLAS in the
 * reference, src/cublas.rs:434-570). */
int grout_gemv(const void* W, const void* x, void* y, int n, int k, void* stream);

/* y = W . x' where x' = rms_norm(x) * gamma (residual == NULL) or
 * x' = rms_norm(residual + x) * gamma, rounded to f16 as the separate norm
 * kernels round it; with a residual, residual_out = f16(residual + x) is
 * written too (it must not alias residual or x).  The decode step's input and
 * post-attention norms fused into the QKV / gate_up GEMVs: one launch for
 * rms_norm_f16 or add_rms_norm_decode_raw_f16 (src/kernels.rs:1530-1569,
 * 4518-4657) followed by the projection GEMV (src/model.rs:3427-3474,
 * 3819-3848).  k = hidden size, a multiple of 8 in [8, 8192]. */
int grout_gemv_rms_norm(const void* W, const void* residual, const void* x, const void* gamma,
                        void* residual_out, void* y, int n, int k, float eps, void* stream);

/* As grout_gemv_rms_norm for W = gate_up_proj [2*inter][k] (rows [gate | up]),
 * with SiLU * up applied in the epilogue: y[i] = f16(silu(g_i) * u_i) for
 * i < inter, g_i and u_i the f16 products of gate row i and up row i.  The
 * decode step's post-attention add-RMSNorm, gate_up GEMV and silu_mul_2d_f16
 * (src/kernels.rs:4518-4657, 1493-1522; src/model.rs:3819-3880) in one
 * launch. */
int grout_gemv_rms_norm_silu_mul(const void* W, const void* residual, const void* x,
                                 const void* gamma, void* residual_out, void* y, int inter, int k,
                                 float eps, void* stream);

/* ------------------------------------------------------------------ */
/* Low-bit weights (ggml block formats, as GGUF files store them)      */
/* ------------------------------------------------------------------ */

#define GROUT_WFMT_F16 0    /* plain fp16 [n][k] */
#define GROUT_WFMT_Q8_0 8   /* ggml type ids */
#define GROUT_WFMT_Q4_K 12
#define GROUT_WFMT_Q5_K 13
#define GROUT_WFMT_Q6_K 14

/* Device bytes of an [n][k] matrix of format fmt in the GEMV layout (0 when
 * the format or shape is unsupported: k a multiple of the block size, 32 for
 * Q8_0 and 256 for the K-quants, at most 32768). */
size_t grout_qweight_bytes(int fmt, int n, int k);

/* Splits n rows of ggml blocks (device memory, rows contiguous) into the GEMV
 * layout `out` (grout_qweight_bytes bytes); bytes are moved, not changed. */
int grout_qweight_repack(int fmt, const void* ggml_blocks, int n, int k, void* out,
                         void* stream);

/* y[r] = f16(sum_k dequant(W)[r][k] x[k]), fp32 dequantization and
 * accumulation.  Replaces gemv_q8_0_f16 / gemv_q4k_f16 / gemv_q5k_f16 /
 * gemv_q6k_f16 and their SoA forms (src/kernels.rs:259-804). */
int grout_gemv_q(int fmt, const void* wq, const void* x, void* y, int n, int k, void* stream);

/* wq holds 2*inter rows [gate | up]: y[i] = f16(silu(g_i) * u_i) with g_i,
 * u_i the f16 products (the gate_up GEMV with silu_mul_2d_f16 in its
 * epilogue, src/kernels.rs:1493-1522). */
int grout_gemv_q_silu_mul(int fmt, const void* wq, const void* x, void* y, int inter, int k,
                          void* stream);

/* grout_gemv_q with the input RMSNorm folded in, as grout_gemv_rms_norm:
 * x' = f16(norm(x) * gamma) (residual NULL) or, for c = residual + x (fp32),
 * x' = f16(norm(c) * gamma) with f16(c) written to residual_out unless it is
 * NULL (it must not alias residual or x).  The decode step's
 * add_rms_norm_decode_raw_f16 (src/kernels.rs:4518-4657) and the low-bit
 * projection GEMV in one launch. */
int grout_gemv_q_rms_norm(int fmt, const void* wq, const void* residual, const void* x,
                          const void* gamma, void* residual_out, void* y, int n, int k, float eps,
                          void* stream);

/* grout_gemv_q_silu_mul with the input RMSNorm folded in (as above). */
int grout_gemv_q_rms_norm_silu_mul(int fmt, const void* wq, const void* residual, const void* x,
                                   const void* gamma, void* residual_out, void* y, int inter,
                                   int k, float eps, void* stream);

/* The [n][k] matrix dequantized to f16 (out) with the decode layout's scales,
 * e.g. for prefill GEMMs: the reference's prefill dequant into its pooled
 * scratch (dequant_q4k_soa_to_f16 / dequant_q5k_to_f16 /
 * dequant_q6k_soa_to_f16 / dequant_q8_0_to_f16, src/kernels.rs:1075-1300;
 * src/quant_scratch.rs). */
int grout_qweight_dequant(int fmt, const void* wq, int n, int k, void* out, void* stream);

/* out[t][0..k) = row ids[t] of the [n][k] matrix as f16 for t < rows, by the
 * CPU dequantization rule (Q4_K with fp32 d*sc and dmin*m); ids (device
 * memory) at or past n read row n - 1.  The token-embedding gather from a
 * quantized table: embed_gather_q8_0_f16 / embed_gather_q4k_f16 /
 * embed_gather_q5k_f16 / embed_gather_q6k_f16 (src/kernels.rs:1940-2120). */
int grout_qweight_gather(int fmt, const void* wq, int n, int k, const uint32_t* ids, int rows,
                         void* out, void* stream);

/* Scratch bytes grout_argmax needs for vocab_size logits. */
size_t grout_argmax_workspace_bytes(int vocab_size);

/* out[0] = index of the largest of logits[0..vocab_size) (f16), ties to the
 * smallest index.  Two launches.  Replaces argmax_blocks_f16 +
 * argmax_reduce_blocks_to_u32 (src/kernels.rs:1571-1740). */
int grout_argmax(const void* logits, int vocab_size, void* workspace, size_t workspace_bytes,
                 uint32_t* out, void* stream);

/* ------------------------------------------------------------------ */
/* Engine                                                              */
/* ------------------------------------------------------------------ */

typedef struct grout_engine grout_engine;

/* ------------------------------------------------------------------ */
/* Checkpoint loading                                                  */
/* ------------------------------------------------------------------ */

#define GROUT_MAX_EOS 8

/* What a model directory holds (config.json, generation_config.json). */
typedef struct grout_model_info {
  grout_qwen3_config config;  /* max_ctx = max_position_embeddings */
  int tie_word_embeddings;
  int num_eos;                /* stop tokens (generation_config.json, else config.json) */
  uint32_t eos_token_ids[GROUT_MAX_EOS];
  size_t weight_bytes;        /* device bytes of the fp16 weights in the fused layouts */
} grout_model_info;

typedef struct grout_model grout_model;

/* Host only (no GPU): parses config.json, generation_config.json and the
 * safetensors headers (model.safetensors.index.json + its shards, or a single
 * model.safetensors) and checks that every tensor the engine needs is present
 * with the expected shape and a castable dtype (F16/BF16/F32/F64).  Mirrors
 * Loader::new + Qwen3Config::from_model_dir/validate (src/loader.rs:33-88,
 * src/config.rs:24-95).  A path ending in ".gguf" names a GGUF file (v2/v3)
 * instead: the qwen3.* metadata becomes the config (config_from_gguf,
 * src/loader.rs:276-330), eos = tokenizer.ggml.eos_token_id, the head is tied
 * when output.weight is absent, and every tensor must be F32/F16/BF16 (norms)
 * or F32/F16/BF16/Q8_0/Q4_K/Q5_K/Q6_K (matrices) with the config's shape; the
 * reader's bounds are the reference's (src/gguf.rs:212-445).  weight_bytes is
 * then the device bytes in the low-bit layouts. */
int grout_model_inspect(const char* model_dir, grout_model_info* info);

/* grout_model_inspect, then the weights into one device allocation on
 * `device` (GGUF: low-bit matrices in grout_qweight_repack's layout, one part
 * per same-format run of q|k|v and gate|up, every other tensor cast to f16;
 * read them with grout_model_qweights) in the fused layouts (qkv_proj = q|k|v rows, gate_up_proj =
 * gate|up rows, lm_head shared with embed_tokens when tied), bf16/f32/f64
 * cast to f16 through f32 with round-to-nearest-even on the GPU.  Replaces
 * the weight half of Qwen3Engine::load (src/model.rs:1508-1600) and
 * cast_to_f16 (src/loader.rs:702-740). */
int grout_model_load(const char* model_dir, int device, grout_model** out);
int grout_model_get_info(const grout_model* model, grout_model_info* info);
/* Device pointers of the loaded weights (valid until grout_model_free; the
 * layers array belongs to the model). */
int grout_model_weights(const grout_model* model, grout_qwen3_weights* weights);
int grout_model_free(grout_model* model);

/* Validates the configuration and every weight pointer, runs the VRAM
 * preflight (grout_engine_vram_preflight with weight_bytes = 0: the caller's
 * weights are resident already) against hipMemGetInfo, allocates the
 * engine's device state on `device` and captures the decode-step graph.
 * Mirrors Engine::load (src/api.rs:60-90) minus the file loading, with the
 * graph capture of DecodeCudaGraphRunner (src/model.rs:408-596,
 * 2631-4006).  With GROUT_HIP_GRAPH_DECODE set off in the environment (0,
 * false, off, no or empty; see grout_env_flag), or when the capture fails (a warning goes to stderr), the engine is still created and
 * decode launches the same step's kernels one by one on the engine's stream
 * (the reference's sequential fallback, src/model.rs:2130-2145, 2300-2309);
 * grout_engine_decode_graph_error says which. */
int grout_engine_create(const grout_qwen3_config* config, const grout_qwen3_weights* weights,
                        int device, grout_engine** out);

/* One weight matrix of a projection: `rows` output rows over the
 * projection's input width k, as f16 [rows][k] (fmt GROUT_WFMT_F16) or in
 * grout_qweight_repack's layout (GROUT_WFMT_Q8_0 / Q4_K / Q5_K / Q6_K).  Mirrors
 * Weight / MatrixWeight (src/weights.rs:7-56), whose parts may differ in
 * format (a Q4_K_M file stores some attn_v and ffn_down matrices as Q6_K). */
typedef struct {
  int fmt;
  int rows;
  const void* data;
} grout_wpart;

/* One decoder layer over mixed-format weights.  qkv parts cover the q | k | v
 * output rows in order (one part when q, k and v share a format and were
 * repacked together); gate_up parts cover gate | up rows in order. */
typedef struct {
  const void* input_layernorm;          /* f16 [hidden] */
  int num_qkv_parts;                    /* 1..3 */
  grout_wpart qkv[3];                   /* k = hidden */
  const void* q_norm;                   /* f16 [128] */
  const void* k_norm;                   /* f16 [128] */
  grout_wpart o_proj;                   /* [hidden] rows, k = Hq * 128 */
  const void* post_attention_layernorm; /* f16 [hidden] */
  int num_gate_up_parts;                /* 1..2 */
  grout_wpart gate_up[2];               /* k = hidden */
  grout_wpart down_proj;                /* [hidden] rows, k = intermediate */
} grout_qwen3_qlayer;

typedef struct {
  grout_wpart embed_tokens;             /* [vocab] rows, k = hidden; gathered */
  const void* norm;                     /* f16 [hidden] */
  grout_wpart lm_head;                  /* [vocab] rows; embed_tokens when tied */
  const grout_qwen3_qlayer* layers;     /* num_layers entries */
} grout_qwen3_qweights;

/* grout_engine_create over mixed-format weights.  Decode: every qkv and
 * gate_up part runs the low-bit GEMV with the input / post-attention RMSNorm
 * folded in (grout_gemv_q_rms_norm; each part recomputes the norm and writes
 * the same residual bits), gate_up as one part with SiLU(gate) * up in the
 * epilogue (grout_gemv_q_rms_norm_silu_mul), o / down / lm_head the plain
 * low-bit GEMV, f16 parts as in grout_engine_create; the embedding row is
 * gathered from the table.  Prefill and extend: each low-bit part is
 * dequantized to f16 into an engine scratch buffer and multiplied with the
 * GEMM (the reference's prefill dequant scratch, src/quant_scratch.rs:17-105).
 * Every part's format must fit its k (grout_qweight_bytes != 0). */
int grout_engine_create_q(const grout_qwen3_config* config, const grout_qwen3_qweights* weights,
                          int device, grout_engine** out);

/* Device pointers of a model loaded from a GGUF file (GROUT_EINVAL for an
 * fp16 checkpoint, whose weights grout_model_weights returns; and the other
 * way round).  Valid until grout_model_free. */
int grout_model_qweights(const grout_model* model, grout_qwen3_qweights* weights);

/* Engine::load (src/api.rs:60-90): grout_model_inspect, the VRAM preflight
 * with the model's weight bytes (before any weight is uploaded, as
 * src/model.rs:1491-1506), grout_model_load + grout_engine_create
 * (grout_engine_create_q for a .gguf path) with max_ctx
 * (0 = max_position_embeddings, which must then be <= GROUT_MAX_CTX); the
 * engine owns the model and frees it in grout_engine_destroy. */
int grout_engine_load(const char* model_dir, int max_ctx, int device, grout_engine** out);

/* Info of the model an engine was loaded from (GROUT_EINVAL for engines made
 * by grout_engine_create). */
int grout_engine_model_info(const grout_engine* engine, grout_model_info* info);

/* New-session prefill over tokens[0..n_tokens) (positions 0..n-1).  Writes
 * the last token's logits as f32 to logits_out (vocab_size floats, host
 * memory, may be NULL) and its greedy argmax to next_token (may be NULL).
 * Fails with GROUT_EINVAL for n_tokens < 1, n_tokens > max_ctx or a token
 * id >= vocab_size.  Mirrors Engine::prefill (src/api.rs:92-108). */
int grout_engine_prefill(grout_engine* engine, const uint32_t* tokens, int n_tokens,
                         float* logits_out, uint32_t* next_token);

/* Chunked prefill: runs tokens[0..n_tokens) at the session's next positions
 * (after a prefill, extends, or decodes), with the same prefill kernels at
 * pos0 = grout_engine_position(); outputs as grout_engine_prefill.  Requires
 * an active session and position + n_tokens <= max_ctx.  An invalid argument
 * leaves the session as it was; a failure while running ends it (the next
 * call must be a prefill).  The reference's kernels take
 * a prefill start position but its API only issues new sessions
 * (src/model.rs:2126); this is that path, e.g. for prompts longer than one
 * chunk or multi-turn input. */
int grout_engine_extend(grout_engine* engine, const uint32_t* tokens, int n_tokens,
                        float* logits_out, uint32_t* next_token);

/* Decodes `token` at the next position of the session (one replay of the
 * decode-step graph, or the same kernels launched one by one without it)
 * and writes next-token logits (f32, vocab_size floats).
 * Requires a preceding prefill and position < max_ctx.
 * Mirrors Engine::decode (src/api.rs:110-121). */
int grout_engine_decode(grout_engine* engine, uint32_t token, float* logits_out);

/* As grout_engine_decode, but returns only the greedy next token (device
 * argmax; 4 bytes cross to the host).  Mirrors Engine::decode_greedy
 * (src/api.rs:123-137). */
int grout_engine_decode_greedy(grout_engine* engine, uint32_t token, uint32_t* next_token);

/* Ends the session: the next call must be a prefill.  The KV caches are
 * zeroed in place (graph pointers stay valid).  A failure is also stashed
 * and reported by the next call.  Mirrors Engine::reset (src/api.rs:139-154)
 * and the in-place cache reset (src/model.rs:536-565). */
int grout_engine_reset(grout_engine* engine);

/* Host only.  Device bytes an engine for `config` needs besides what the
 * caller already holds: weight_bytes (the model's, when they are still to be
 * uploaded; 0 for caller-owned weights) + the K/V caches
 * (num_layers * 2 * Hkv * max_ctx * 128 * 2 B) + the RoPE tables
 * (max_ctx * 128 * 4 B) + scratch_bytes (decode buffers, prefill dequant
 * scratch) + 700 MiB of slack, written to *required (may be NULL).  Returns
 * GROUT_ENOMEM, with the itemized summary in grout_last_error(), when that
 * exceeds free_bytes.  Mirrors run_vram_preflight (src/model.rs:345-380). */
int grout_engine_vram_preflight(const grout_qwen3_config* config, size_t weight_bytes,
                                size_t scratch_bytes, size_t free_bytes, size_t total_bytes,
                                size_t* required);

/* 1 when decode replays the captured decode-step graph, 0 when it runs the
 * sequential fallback (or engine is NULL). */
int grout_engine_uses_decode_graph(const grout_engine* engine);

/* Why decode runs the sequential fallback: the capture error, or the
 * GROUT_HIP_GRAPH_DECODE setting (off); "" when the graph is in use.  Mirrors
 * GenerationOutput::decode_graph_error (src/model.rs:1359).  Valid until
 * grout_engine_destroy. */
const char* grout_engine_decode_graph_error(const grout_engine* engine);

/* Runs a dummy one-token step at positions 0 and 1 (a one-token prefill,
 * then one decode-graph replay) with the model's first stop token (0 for
 * an engine over caller weights), so the first request does not pay for
 * loading library kernels or the graph's first upload; then zeroes the
 * caches and ends the session as grout_engine_reset does (position 0, the
 * next call must be a prefill).  Mirrors Engine::warmup (src/api.rs:153-162,
 * api_warmup src/model.rs:2204-2212). */
int grout_engine_warmup(grout_engine* engine);

/* Position the next decode writes (number of tokens in the session). */
int grout_engine_position(const grout_engine* engine);

/* Split count of the engine's decode attention: GROUT_FMHA_NUM_KV_SPLITS
 * from the environment at creation (read as grout_env_usize does, capped at
 * GROUT_MAX_SPLITS; the reference's knob of the same name,
 * src/model.rs:2713-2714), else grout_attn_decode_default_splits(max_ctx).
 * -1 for NULL. */
int grout_engine_num_splits(const grout_engine* engine);

/* Host only.  How the engine reads a boolean switch from the environment
 * (GROUT_HIP_GRAPH_DECODE, the counterpart of the reference's
 * GROUT_CUDA_GRAPH_DECODE): `value` is the variable's text, NULL when unset.
 * Returns 1 for "1", "true", "on", "yes" and 0 for "0", "false", "off", "no"
 * or "" (whitespace trimmed, case ignored), default_value (0 or 1) for
 * anything else or NULL.  Mirrors env_bool_or (src/model.rs:212-224). */
int grout_env_flag(const char* value, int default_value);

/* Host only.  How the engine reads a positive integer setting
 * (GROUT_FMHA_NUM_KV_SPLITS): an optional '+' and decimal digits, nothing
 * else; zero, a value past 2^63 - 1 (a long; Rust's usize takes up to
 * 2^64 - 1), any other text or NULL give default_value.  Mirrors
 * env_usize_or (src/model.rs:204-210). */
long grout_env_usize(const char* value, long default_value);

/* Frees everything the engine owns (not the weights).  NULL is a no-op. */
int grout_engine_destroy(grout_engine* engine);

#ifdef __cplusplus
}
#endif

#endif /* GROUT_ENGINE_H */
