// Qwen3 engine on one gfx950 GPU: new-session prefill (rocBLAS GEMMs for the
// projections, the hand-written norm/RoPE/KV-write, prefill attention and
// elementwise kernels) and the decode step, captured once as a HIP graph and
// replayed per token.
//
// Reference: Engine (src/api.rs:11-183) over Qwen3Engine (src/model.rs); the
// decode step is build_decode_graph_scope (src/model.rs:2631-4006), replayed by
// DecodeCudaGraphRunner (src/model.rs:408-596); the prefill layer sequence is
// the StepGraph of src/model.rs:4031-4678.  Per layer, in both paths:
//   normed   = layer 0 ? rms_norm(hidden) : add_rms_norm(hidden_after_attn + ff_down)
//   q, k, v  = normed x qkv_proj^T
//   q_rope, K/V cache rows = qk_norm_rope_kv(q, k, v)
//   attn     = attention(q_rope, caches)
//   ff_normed, hidden_after_attn = add_rms_norm(hidden + attn x o_proj^T)
//   ff       = silu(gate) * up, [gate | up] = ff_normed x gate_up_proj^T
//   ff_down  = ff x down_proj^T
// and the residual add of the last layer folds into the final norm before the
// lm_head (src/model.rs:3896-3910).
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "../../include/grout_attn.h"
#include "../../include/grout_engine.h"
#include "abi_util.hpp"
#include "kernels.hpp"

using namespace grout_abi;

namespace {

constexpr size_t kAlign = 256;

size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

// Sub-allocations of one device allocation.
struct Arena {
  void* base = nullptr;
  size_t used = 0;
  size_t take(size_t bytes) {
    const size_t off = used;
    used += align_up(bytes);
    return off;
  }
  template <class T>
  T* at(size_t off) const {
    return reinterpret_cast<T*>(static_cast<char*>(base) + off);
  }
};

// Decode-step activations: one token.
struct DecodeBufs {
  size_t hidden, normed, hidden_after_attn, qkv, attn_out, attn_proj, ff, ff_down, logits,
      argmax_max, argmax_idx, token, pos, workspace;
};

// Prefill activations: cap rows.
struct PrefillBufs {
  size_t ids, hidden, normed, hidden_after_attn, q, k, v, q_rope, attn_out, attn_proj, ff_normed,
      gate_up, ff, ff_down;
};

__global__ void set_step_kernel(uint32_t* d_token, uint32_t token, uint32_t* d_pos,
                                uint32_t pos) {
  d_token[0] = token;
  d_pos[0] = pos;
}

int blas_status(rocblas_status s, const char* what) {
  if (s == rocblas_status_success) return GROUT_OK;
  return fail(GROUT_EBLAS, "%s: %s", what, rocblas_status_to_string(s));
}

}  // namespace

struct grout_engine {
  grout_qwen3_config cfg{};
  const void* embed = nullptr;
  const void* final_norm = nullptr;
  const void* lm_head = nullptr;
  std::vector<grout_qwen3_layer> layers;
  int device = 0;
  hipStream_t stream = nullptr;
  rocblas_handle blas = nullptr;

  // Derived sizes.
  int q_dim = 0, kv_dim = 0, qkv_dim = 0;
  long head_stride = 0;
  int num_splits = 0;
  size_t ws_bytes = 0;
  int argmax_blocks = 0;
  float qk_scale = 0.f;

  // Device memory.
  void* kv = nullptr;  // [layers][K|V][Hkv][max_ctx][128]
  float* rope = nullptr;  // cos [max_ctx][64] | sin [max_ctx][64]
  Arena dec;
  DecodeBufs db{};
  Arena pre;
  PrefillBufs pb{};
  int prefill_cap = 0;

  // Pinned host staging.
  uint16_t* h_logits = nullptr;
  uint32_t* h_token = nullptr;

  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;

  int next_pos = 0;
  bool session_active = false;
  std::string pending_reset_error;

  // Set by grout_engine_load: the checkpoint's weights, freed with the engine.
  grout_model* owned_model = nullptr;

  void* k_cache(int l) const {
    return static_cast<char*>(kv) + (size_t)l * 2 * cache_bytes();
  }
  void* v_cache(int l) const { return static_cast<char*>(k_cache(l)) + cache_bytes(); }
  size_t cache_bytes() const {
    return (size_t)cfg.num_kv_heads * cfg.max_ctx * 128 * sizeof(uint16_t);
  }
  const float* rope_cos() const { return rope; }
  const float* rope_sin() const { return rope + (size_t)cfg.max_ctx * 64; }
  template <class T = void>
  T* d(size_t off) const {
    return dec.at<T>(off);
  }
  template <class T = void>
  T* p(size_t off) const {
    return pre.at<T>(off);
  }
};

namespace {

// y[rows][n] = x[rows][k] . W[n][k]^T, fp16 in/out, fp32 accumulation.  In
// rocBLAS's column-major terms: C (n x rows, ldc n) = W^T(col-major k x n,
// transposed) x X (col-major k x rows).
int gemm_rows(grout_engine* e, const void* W, const void* x, void* y, int rows, int n, int k) {
  const float alpha = 1.f, beta = 0.f;
  return blas_status(
      rocblas_gemm_ex(e->blas, rocblas_operation_transpose, rocblas_operation_none, n, rows, k,
                      &alpha, W, rocblas_datatype_f16_r, k, x, rocblas_datatype_f16_r, k, &beta, y,
                      rocblas_datatype_f16_r, n, y, rocblas_datatype_f16_r, n,
                      rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0),
      "rocblas_gemm_ex");
}

// Projection of `rows` tokens.  One row uses the decode GEMV kernel.
int project(grout_engine* e, const void* W, const void* x, void* y, int rows, int n, int k) {
  if (rows == 1) return hip_status(grout::launch_gemv(W, x, y, n, k, e->stream), "gemv");
  return gemm_rows(e, W, x, y, rows, n, k);
}

int norm(grout_engine* e, const void* residual, const void* x, const void* w, void* out,
         void* residual_out, int rows) {
  return hip_status(grout::launch_rms_norm(residual, x, w, out, residual_out, rows,
                                           e->cfg.hidden_size, e->cfg.rms_norm_eps, e->stream),
                    "rms_norm");
}

// Final norm (folding the last layer's residual add), lm_head and argmax
// over one token's hidden state; leaves f16 logits and the token on device.
int head(grout_engine* e, const void* hidden_after_attn, const void* ff_down) {
  const auto& c = e->cfg;
  GROUT_CHECK(norm(e, hidden_after_attn, ff_down, e->final_norm, e->d(e->db.normed),
                   e->d(e->db.hidden), 1));
  GROUT_CHECK(hip_status(grout::launch_gemv(e->lm_head, e->d(e->db.normed), e->d(e->db.logits),
                                            c.vocab_size, c.hidden_size, e->stream),
                         "lm_head gemv"));
  return hip_status(grout::launch_argmax(e->d(e->db.logits), e->d<float>(e->db.argmax_max),
                                         e->d<uint32_t>(e->db.argmax_idx), c.vocab_size,
                                         e->d<uint32_t>(e->db.token), e->stream),
                    "argmax");
}

// The decode step, as recorded into the graph.
int record_decode_step(grout_engine* e) {
  const auto& c = e->cfg;
  const DecodeBufs& b = e->db;
  hipStream_t s = e->stream;
  GROUT_CHECK(hip_status(grout::launch_embedding(e->d<uint32_t>(b.token), e->embed,
                                                 e->d(b.hidden), 1, c.hidden_size, c.vocab_size,
                                                 s),
                         "embedding"));
  for (int l = 0; l < c.num_layers; ++l) {
    const grout_qwen3_layer& w = e->layers[l];
    // input norm fused into the QKV GEMV (layer 0: plain RMSNorm of the
    // embedding; later layers: add the previous layer's MLP output first)
    if (l == 0)
      GROUT_CHECK(hip_status(grout::launch_gemv_norm(w.qkv_proj, nullptr, e->d(b.hidden),
                                                     w.input_layernorm, nullptr, c.rms_norm_eps,
                                                     e->d(b.qkv), e->qkv_dim, c.hidden_size,
                                                     false, s),
                             "qkv gemv"));
    else
      GROUT_CHECK(hip_status(grout::launch_gemv_norm(w.qkv_proj, e->d(b.hidden_after_attn),
                                                     e->d(b.ff_down), w.input_layernorm,
                                                     e->d(b.hidden), c.rms_norm_eps, e->d(b.qkv),
                                                     e->qkv_dim, c.hidden_size, false, s),
                             "qkv gemv"));
    // QK-norm/RoPE + K/V cache write inside the split-K attention, then the merge
    GROUT_CHECK(grout_attn_decode_fused(
        e->d(b.qkv), w.q_norm, w.k_norm, e->rope_cos(), e->rope_sin(), e->k_cache(l),
        e->v_cache(l), e->d(b.attn_out), e->d(b.workspace), e->ws_bytes,
        e->d<uint32_t>(b.pos), c.num_q_heads, c.num_kv_heads, 128, c.max_ctx, e->head_stride,
        e->num_splits, c.rms_norm_eps, e->qk_scale, s));
    GROUT_CHECK(project(e, w.o_proj, e->d(b.attn_out), e->d(b.attn_proj), 1, c.hidden_size,
                        e->q_dim));
    // post-attention add + RMSNorm fused into the gate_up GEMV, whose
    // epilogue applies SiLU(gate) * up: it writes ff directly
    GROUT_CHECK(hip_status(grout::launch_gemv_norm(w.gate_up_proj, e->d(b.hidden),
                                                   e->d(b.attn_proj), w.post_attention_layernorm,
                                                   e->d(b.hidden_after_attn), c.rms_norm_eps,
                                                   e->d(b.ff), c.intermediate_size,
                                                   c.hidden_size, true, s),
                           "gate_up gemv"));
    GROUT_CHECK(project(e, w.down_proj, e->d(b.ff), e->d(b.ff_down), 1, c.hidden_size,
                        c.intermediate_size));
  }
  return head(e, e->d(b.hidden_after_attn), e->d(b.ff_down));
}

int capture_decode_graph(grout_engine* e) {
  int rc = hip_status(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal),
                      "hipStreamBeginCapture");
  if (rc != GROUT_OK) return rc;
  rc = record_decode_step(e);
  hipGraph_t g = nullptr;
  const hipError_t end = hipStreamEndCapture(e->stream, &g);
  if (rc == GROUT_OK) rc = hip_status(end, "hipStreamEndCapture");
  e->graph = g;
  if (rc != GROUT_OK) return rc;
  return hip_status(hipGraphInstantiate(&e->exec, e->graph, nullptr, nullptr, 0),
                    "hipGraphInstantiate");
}

int ensure_prefill_capacity(grout_engine* e, int rows) {
  if (rows <= e->prefill_cap) return GROUT_OK;
  const auto& c = e->cfg;
  int cap = 64;
  while (cap < rows) cap *= 2;
  if (cap > c.max_ctx) cap = c.max_ctx;
  if (e->pre.base) {
    GROUT_CHECK(hip_status(hipStreamSynchronize(e->stream), "hipStreamSynchronize"));
    (void)hipFree(e->pre.base);
    e->pre = Arena{};
    e->prefill_cap = 0;
  }
  const size_t H = c.hidden_size, I = c.intermediate_size, r = cap, h2 = sizeof(uint16_t);
  Arena a;
  PrefillBufs& b = e->pb;
  b.ids = a.take(r * sizeof(uint32_t));
  b.hidden = a.take(r * H * h2);
  b.normed = a.take(r * H * h2);
  b.hidden_after_attn = a.take(r * H * h2);
  b.q = a.take(r * e->q_dim * h2);
  b.k = a.take(r * e->kv_dim * h2);
  b.v = a.take(r * e->kv_dim * h2);
  b.q_rope = a.take(r * e->q_dim * h2);
  b.attn_out = a.take(r * e->q_dim * h2);
  b.attn_proj = a.take(r * H * h2);
  b.ff_normed = a.take(r * H * h2);
  b.gate_up = a.take(r * 2 * I * h2);
  b.ff = a.take(r * I * h2);
  b.ff_down = a.take(r * H * h2);
  GROUT_CHECK(hip_status(hipMalloc(&a.base, a.used), "hipMalloc(prefill buffers)"));
  e->pre = a;
  e->prefill_cap = cap;
  return GROUT_OK;
}

int copy_logits_out(grout_engine* e, float* logits_out, uint32_t* next_token) {
  const int V = e->cfg.vocab_size;
  if (logits_out)
    GROUT_CHECK(hip_status(hipMemcpyAsync(e->h_logits, e->d(e->db.logits), (size_t)V * 2,
                                          hipMemcpyDeviceToHost, e->stream),
                           "logits D2H"));
  if (next_token)
    GROUT_CHECK(hip_status(hipMemcpyAsync(e->h_token, e->d(e->db.token), sizeof(uint32_t),
                                          hipMemcpyDeviceToHost, e->stream),
                           "token D2H"));
  GROUT_CHECK(hip_status(hipStreamSynchronize(e->stream), "hipStreamSynchronize"));
  if (logits_out) {
    for (int i = 0; i < V; ++i) {
      _Float16 h;
      std::memcpy(&h, &e->h_logits[i], 2);
      logits_out[i] = (float)h;
    }
  }
  if (next_token) *next_token = *e->h_token;
  return GROUT_OK;
}

int take_pending(grout_engine* e) {
  if (e->pending_reset_error.empty()) return GROUT_OK;
  const std::string msg = e->pending_reset_error;
  e->pending_reset_error.clear();
  return fail(GROUT_EINVAL, "previous reset failed: %s", msg.c_str());
}

int decode_common(grout_engine* e, uint32_t token) {
  GROUT_CHECK(take_pending(e));
  GROUT_NEED(e->session_active, GROUT_EINVAL, "decode requires a preceding prefill");
  GROUT_NEED(e->next_pos < e->cfg.max_ctx, GROUT_EINVAL, "decode position %d exceeds max_ctx=%d",
             e->next_pos, e->cfg.max_ctx);
  GROUT_NEED(token < (uint32_t)e->cfg.vocab_size, GROUT_EINVAL, "token %u >= vocab_size=%d",
             token, e->cfg.vocab_size);
  GROUT_CHECK(hip_status(hipSetDevice(e->device), "hipSetDevice"));
  // Token and position travel as kernel arguments: no host staging buffer
  // that a queued replay could still be reading.
  set_step_kernel<<<1, 1, 0, e->stream>>>(e->d<uint32_t>(e->db.token), token,
                                          e->d<uint32_t>(e->db.pos), (uint32_t)e->next_pos);
  GROUT_CHECK(hip_status(hipGetLastError(), "set step"));
  GROUT_CHECK(hip_status(hipGraphLaunch(e->exec, e->stream), "hipGraphLaunch"));
  e->next_pos += 1;
  return GROUT_OK;
}

int validate(const grout_qwen3_config* c, const grout_qwen3_weights* w) {
  GROUT_NEED(c != nullptr && w != nullptr, GROUT_EINVAL, "config or weights is NULL");
  GROUT_NEED(c->num_layers >= 1, GROUT_EINVAL, "num_layers=%d", c->num_layers);
  GROUT_CHECK(check_heads(c->num_q_heads, c->num_kv_heads, c->head_dim, kMaxDecodeGroup));
  GROUT_NEED(c->hidden_size >= 8 && c->hidden_size % 8 == 0 && c->hidden_size <= 8192,
             GROUT_ENOTSUP, "hidden_size=%d must be a multiple of 8 in [8, 8192]",
             c->hidden_size);
  GROUT_NEED(c->intermediate_size >= 8 && c->intermediate_size % 8 == 0, GROUT_ENOTSUP,
             "intermediate_size=%d must be a positive multiple of 8", c->intermediate_size);
  GROUT_NEED(c->vocab_size >= 1, GROUT_EINVAL, "vocab_size=%d", c->vocab_size);
  GROUT_NEED(c->max_ctx >= 1, GROUT_EINVAL, "max_ctx=%d", c->max_ctx);
  GROUT_NEED(std::isfinite(c->rms_norm_eps) && c->rms_norm_eps > 0.f, GROUT_EINVAL,
             "rms_norm_eps=%g", (double)c->rms_norm_eps);
  GROUT_NEED(std::isfinite(c->rope_theta) && c->rope_theta > 0.f, GROUT_EINVAL, "rope_theta=%g",
             (double)c->rope_theta);
  GROUT_CHECK(check_ptrs16({{w->embed_tokens, "embed_tokens"}, {w->norm, "norm"},
                            {w->lm_head, "lm_head"}}));
  GROUT_NEED(w->layers != nullptr, GROUT_EINVAL, "layers is NULL");
  for (int l = 0; l < c->num_layers; ++l) {
    const grout_qwen3_layer& L = w->layers[l];
    const int rc = check_ptrs16({{L.input_layernorm, "input_layernorm"},
                                 {L.qkv_proj, "qkv_proj"},
                                 {L.q_norm, "q_norm"},
                                 {L.k_norm, "k_norm"},
                                 {L.o_proj, "o_proj"},
                                 {L.post_attention_layernorm, "post_attention_layernorm"},
                                 {L.gate_up_proj, "gate_up_proj"},
                                 {L.down_proj, "down_proj"}});
    if (rc != GROUT_OK) return fail(rc, "layer %d: %s", l, g_last_error.c_str());
  }
  return GROUT_OK;
}

int create_impl(grout_engine* e, const grout_qwen3_config* c, const grout_qwen3_weights* w,
                int device) {
  e->cfg = *c;
  e->device = device;
  e->embed = w->embed_tokens;
  e->final_norm = w->norm;
  e->lm_head = w->lm_head;
  e->layers.assign(w->layers, w->layers + c->num_layers);
  e->q_dim = c->num_q_heads * 128;
  e->kv_dim = c->num_kv_heads * 128;
  e->qkv_dim = e->q_dim + 2 * e->kv_dim;
  e->head_stride = (long)c->max_ctx * 128;
  e->num_splits = grout_attn_decode_default_splits(c->max_ctx, c->num_q_heads, c->num_kv_heads);
  e->ws_bytes = decode_ws_bytes(c->num_q_heads, c->num_kv_heads, e->num_splits);
  e->argmax_blocks = grout::argmax_num_blocks(c->vocab_size);
  e->qk_scale = 1.0f / std::sqrt(128.0f);  // src/model.rs:2654, 6901

  GROUT_CHECK(hip_status(hipSetDevice(device), "hipSetDevice"));
  GROUT_CHECK(hip_status(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking),
                         "hipStreamCreate"));
  GROUT_CHECK(blas_status(rocblas_create_handle(&e->blas), "rocblas_create_handle"));
  GROUT_CHECK(blas_status(rocblas_set_stream(e->blas, e->stream), "rocblas_set_stream"));

  // KV caches [layers][K|V][Hkv][max_ctx][128], zeroed (src/model.rs:1587-1599).
  const size_t kv_bytes = (size_t)c->num_layers * 2 * e->cache_bytes();
  GROUT_CHECK(hip_status(hipMalloc(&e->kv, kv_bytes), "hipMalloc(kv caches)"));
  GROUT_CHECK(hip_status(hipMemsetAsync(e->kv, 0, kv_bytes, e->stream), "hipMemset(kv caches)"));

  // RoPE tables, built on the host once (bit-reproducible angles).
  const size_t half_rows = (size_t)c->max_ctx * 64;
  std::vector<float> tab(2 * half_rows);
  GROUT_CHECK(grout_rope_table_host(c->max_ctx, 128, c->rope_theta, tab.data(),
                                    tab.data() + half_rows));
  GROUT_CHECK(hip_status(hipMalloc(&e->rope, tab.size() * sizeof(float)), "hipMalloc(rope)"));
  GROUT_CHECK(hip_status(hipMemcpy(e->rope, tab.data(), tab.size() * sizeof(float),
                                   hipMemcpyHostToDevice),
                         "rope H2D"));

  const size_t H = c->hidden_size, I = c->intermediate_size, h2 = sizeof(uint16_t);
  Arena a;
  DecodeBufs& b = e->db;
  b.hidden = a.take(H * h2);
  b.normed = a.take(H * h2);
  b.hidden_after_attn = a.take(H * h2);
  b.qkv = a.take(e->qkv_dim * h2);
  b.attn_out = a.take(e->q_dim * h2);
  b.attn_proj = a.take(H * h2);
  b.ff = a.take(I * h2);
  b.ff_down = a.take(H * h2);
  b.logits = a.take((size_t)c->vocab_size * h2);
  b.argmax_max = a.take((size_t)e->argmax_blocks * sizeof(float));
  b.argmax_idx = a.take((size_t)e->argmax_blocks * sizeof(uint32_t));
  b.token = a.take(sizeof(uint32_t));
  b.pos = a.take(sizeof(uint32_t));
  b.workspace = a.take(e->ws_bytes);
  GROUT_CHECK(hip_status(hipMalloc(&a.base, a.used), "hipMalloc(decode buffers)"));
  e->dec = a;
  GROUT_CHECK(hip_status(hipMemsetAsync(a.base, 0, a.used, e->stream), "hipMemset(decode)"));

  GROUT_CHECK(hip_status(hipHostMalloc(reinterpret_cast<void**>(&e->h_logits),
                                       (size_t)c->vocab_size * h2, hipHostMallocDefault),
                         "hipHostMalloc(logits)"));
  GROUT_CHECK(hip_status(hipHostMalloc(reinterpret_cast<void**>(&e->h_token), sizeof(uint32_t),
                                       hipHostMallocDefault),
                         "hipHostMalloc(token)"));
  GROUT_CHECK(hip_status(hipStreamSynchronize(e->stream), "hipStreamSynchronize"));
  return capture_decode_graph(e);
}

}  // namespace

extern "C" {

int grout_embedding(const uint32_t* ids, const void* table, void* out, int rows, int hidden,
                    int vocab_size, void* stream) {
  GROUT_NEED(rows >= 1 && vocab_size >= 1, GROUT_EINVAL, "rows=%d vocab_size=%d", rows,
             vocab_size);
  GROUT_NEED(hidden >= 8 && hidden % 8 == 0, GROUT_EINVAL, "hidden=%d must be a multiple of 8",
             hidden);
  GROUT_NEED(ids != nullptr, GROUT_EINVAL, "ids is NULL");
  GROUT_CHECK(check_ptrs16({{table, "table"}, {out, "out"}}));
  return hip_status(grout::launch_embedding(ids, table, out, rows, hidden, vocab_size,
                                            as_stream(stream)),
                    "embedding launch");
}

static int check_norm(int rows, int hidden, float eps) {
  GROUT_NEED(rows >= 1, GROUT_EINVAL, "rows=%d", rows);
  GROUT_NEED(hidden >= 8 && hidden % 8 == 0 && hidden <= 8192, GROUT_ENOTSUP,
             "hidden=%d must be a multiple of 8 in [8, 8192]", hidden);
  GROUT_NEED(std::isfinite(eps) && eps > 0.f, GROUT_EINVAL, "eps=%g", (double)eps);
  return GROUT_OK;
}

int grout_rms_norm(const void* x, const void* w, void* out, int rows, int hidden, float eps,
                   void* stream) {
  GROUT_CHECK(check_norm(rows, hidden, eps));
  GROUT_CHECK(check_ptrs16({{x, "x"}, {w, "w"}, {out, "out"}}));
  return hip_status(grout::launch_rms_norm(nullptr, x, w, out, nullptr, rows, hidden, eps,
                                           as_stream(stream)),
                    "rms_norm launch");
}

int grout_add_rms_norm(const void* residual, const void* x, const void* w, void* out,
                       void* residual_out, int rows, int hidden, float eps, void* stream) {
  GROUT_CHECK(check_norm(rows, hidden, eps));
  GROUT_CHECK(check_ptrs16({{residual, "residual"}, {x, "x"}, {w, "w"}, {out, "out"},
                            {residual_out, "residual_out"}}));
  return hip_status(grout::launch_rms_norm(residual, x, w, out, residual_out, rows, hidden, eps,
                                           as_stream(stream)),
                    "add_rms_norm launch");
}

int grout_silu_mul(const void* gate_up, void* out, int rows, int inter, void* stream) {
  GROUT_NEED(rows >= 1, GROUT_EINVAL, "rows=%d", rows);
  GROUT_NEED(inter >= 8 && inter % 8 == 0, GROUT_EINVAL, "inter=%d must be a multiple of 8",
             inter);
  GROUT_CHECK(check_ptrs16({{gate_up, "gate_up"}, {out, "out"}}));
  return hip_status(grout::launch_silu_mul(gate_up, out, rows, inter, as_stream(stream)),
                    "silu_mul launch");
}

int grout_gemv(const void* W, const void* x, void* y, int n, int k, void* stream) {
  GROUT_NEED(n >= 1, GROUT_EINVAL, "n=%d", n);
  GROUT_NEED(k >= 8 && k % 8 == 0, GROUT_EINVAL, "k=%d must be a multiple of 8", k);
  GROUT_CHECK(check_ptrs16({{W, "W"}, {x, "x"}}));
  GROUT_NEED(y != nullptr && (reinterpret_cast<uintptr_t>(y) & 1u) == 0, GROUT_EALIGN,
             "y is NULL or not 2-byte aligned");
  return hip_status(grout::launch_gemv(W, x, y, n, k, as_stream(stream)), "gemv launch");
}

static int check_gemv_norm(const void* W, const void* residual, const void* x,
                           const void* gamma, void* residual_out, void* y, int n, int k,
                           float eps) {
  GROUT_NEED(n >= 1, GROUT_EINVAL, "n=%d", n);
  GROUT_CHECK(check_norm(1, k, eps));
  GROUT_CHECK(check_ptrs16({{W, "W"}, {x, "x"}, {gamma, "gamma"}}));
  if (residual) GROUT_CHECK(check_ptrs16({{residual, "residual"}, {residual_out, "residual_out"}}));
  GROUT_NEED(y != nullptr && (reinterpret_cast<uintptr_t>(y) & 1u) == 0, GROUT_EALIGN,
             "y is NULL or not 2-byte aligned");
  return GROUT_OK;
}

int grout_gemv_rms_norm(const void* W, const void* residual, const void* x, const void* gamma,
                        void* residual_out, void* y, int n, int k, float eps, void* stream) {
  GROUT_CHECK(check_gemv_norm(W, residual, x, gamma, residual_out, y, n, k, eps));
  return hip_status(grout::launch_gemv_norm(W, residual, x, gamma, residual_out, eps, y, n, k,
                                            false, as_stream(stream)),
                    "gemv_rms_norm launch");
}

int grout_gemv_rms_norm_silu_mul(const void* W, const void* residual, const void* x,
                                 const void* gamma, void* residual_out, void* y, int inter, int k,
                                 float eps, void* stream) {
  GROUT_CHECK(check_gemv_norm(W, residual, x, gamma, residual_out, y, inter, k, eps));
  return hip_status(grout::launch_gemv_norm(W, residual, x, gamma, residual_out, eps, y, inter,
                                            k, true, as_stream(stream)),
                    "gemv_rms_norm_silu_mul launch");
}

size_t grout_qweight_bytes(int fmt, int n, int k) { return grout::qweight_bytes(fmt, n, k); }

static int check_q(int fmt, int n, int k) {
  GROUT_NEED(fmt == GROUT_WFMT_Q8_0 || fmt == GROUT_WFMT_Q4_K || fmt == GROUT_WFMT_Q6_K,
             GROUT_ENOTSUP, "weight format %d: Q8_0 (8), Q4_K (12) or Q6_K (14) expected", fmt);
  GROUT_NEED(grout::qweight_bytes(fmt, n, k) != 0, GROUT_EINVAL,
             "[%d][%d] of format %d: k must be a multiple of the block size and <= 16384", n, k,
             fmt);
  return GROUT_OK;
}

int grout_qweight_repack(int fmt, const void* ggml_blocks, int n, int k, void* out,
                         void* stream) {
  GROUT_CHECK(check_q(fmt, n, k));
  GROUT_NEED(ggml_blocks != nullptr, GROUT_EINVAL, "ggml_blocks is NULL");
  GROUT_CHECK(check_ptrs16({{out, "out"}}));
  return hip_status(grout::launch_qweight_repack(fmt, ggml_blocks, n, k, out, as_stream(stream)),
                    "qweight_repack launch");
}

int grout_gemv_q(int fmt, const void* wq, const void* x, void* y, int n, int k, void* stream) {
  GROUT_CHECK(check_q(fmt, n, k));
  GROUT_CHECK(check_ptrs16({{wq, "wq"}, {x, "x"}}));
  GROUT_NEED(y != nullptr && (reinterpret_cast<uintptr_t>(y) & 1u) == 0, GROUT_EALIGN,
             "y is NULL or not 2-byte aligned");
  return hip_status(grout::launch_gemv_q(fmt, wq, x, y, n, k, false, as_stream(stream)),
                    "gemv_q launch");
}

int grout_gemv_q_silu_mul(int fmt, const void* wq, const void* x, void* y, int inter, int k,
                          void* stream) {
  GROUT_CHECK(check_q(fmt, 2 * inter, k));
  GROUT_CHECK(check_ptrs16({{wq, "wq"}, {x, "x"}}));
  GROUT_NEED(y != nullptr && (reinterpret_cast<uintptr_t>(y) & 1u) == 0, GROUT_EALIGN,
             "y is NULL or not 2-byte aligned");
  return hip_status(grout::launch_gemv_q(fmt, wq, x, y, inter, k, true, as_stream(stream)),
                    "gemv_q_silu_mul launch");
}

int grout_qweight_dequant(int fmt, const void* wq, int n, int k, void* out, void* stream) {
  GROUT_CHECK(check_q(fmt, n, k));
  GROUT_CHECK(check_ptrs16({{wq, "wq"}, {out, "out"}}));
  return hip_status(grout::launch_qweight_dequant(fmt, wq, n, k, out, as_stream(stream)),
                    "qweight_dequant launch");
}

size_t grout_argmax_workspace_bytes(int vocab_size) {
  if (vocab_size < 1) return 0;
  return (size_t)grout::argmax_num_blocks(vocab_size) * (sizeof(float) + sizeof(uint32_t));
}

int grout_argmax(const void* logits, int vocab_size, void* workspace, size_t workspace_bytes,
                 uint32_t* out, void* stream) {
  GROUT_NEED(vocab_size >= 1, GROUT_EINVAL, "vocab_size=%d", vocab_size);
  const size_t need = grout_argmax_workspace_bytes(vocab_size);
  GROUT_NEED(workspace != nullptr && workspace_bytes >= need, GROUT_EINVAL,
             "workspace of %zu bytes < %zu needed", workspace_bytes, need);
  GROUT_CHECK(check_ptrs16({{logits, "logits"}, {workspace, "workspace"}}));
  GROUT_NEED(out != nullptr, GROUT_EINVAL, "out is NULL");
  const int nb = grout::argmax_num_blocks(vocab_size);
  float* bmax = static_cast<float*>(workspace);
  uint32_t* bidx = reinterpret_cast<uint32_t*>(bmax + nb);
  return hip_status(grout::launch_argmax(logits, bmax, bidx, vocab_size, out, as_stream(stream)),
                    "argmax launch");
}

int grout_engine_create(const grout_qwen3_config* config, const grout_qwen3_weights* weights,
                        int device, grout_engine** out) {
  GROUT_NEED(out != nullptr, GROUT_EINVAL, "out is NULL");
  *out = nullptr;
  GROUT_CHECK(validate(config, weights));
  int ndev = 0;
  GROUT_CHECK(hip_status(hipGetDeviceCount(&ndev), "hipGetDeviceCount"));
  GROUT_NEED(device >= 0 && device < ndev, GROUT_EINVAL, "device %d of %d", device, ndev);
  grout_engine* e = new (std::nothrow) grout_engine();
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "out of host memory");
  const int rc = create_impl(e, config, weights, device);
  if (rc != GROUT_OK) {
    const std::string msg = g_last_error;
    grout_engine_destroy(e);
    g_last_error = msg;
    return rc;
  }
  *out = e;
  return GROUT_OK;
}

}  // extern "C"

namespace {

// Runs tokens[0..n) at positions pos0 .. pos0+n-1 through every layer (their
// K/V rows land in the caches; rows < pos0 must already hold the session's
// earlier tokens), then the head over the last one.
int run_chunk(grout_engine* e, const uint32_t* tokens, int n, int pos0, float* logits_out,
              uint32_t* next_token) {
  const auto& c = e->cfg;
  GROUT_NEED(tokens != nullptr && n >= 1, GROUT_EINVAL, "prefill requires at least one token");
  GROUT_NEED((long)pos0 + n <= c.max_ctx, GROUT_EINVAL,
             "prefill of %d tokens at position %d exceeds max_ctx=%d", n, pos0, c.max_ctx);
  for (int i = 0; i < n; ++i)
    GROUT_NEED(tokens[i] < (uint32_t)c.vocab_size, GROUT_EINVAL,
               "token %u at %d >= vocab_size=%d", tokens[i], i, c.vocab_size);
  GROUT_CHECK(hip_status(hipSetDevice(e->device), "hipSetDevice"));
  e->session_active = false;
  GROUT_CHECK(ensure_prefill_capacity(e, n));
  const PrefillBufs& b = e->pb;
  hipStream_t s = e->stream;
  GROUT_CHECK(hip_status(hipMemcpyAsync(e->p(b.ids), tokens, (size_t)n * sizeof(uint32_t),
                                        hipMemcpyHostToDevice, s),
                         "tokens H2D"));
  GROUT_CHECK(hip_status(grout::launch_embedding(e->p<uint32_t>(b.ids), e->embed, e->p(b.hidden),
                                                 n, c.hidden_size, c.vocab_size, s),
                         "embedding"));
  const int H = c.hidden_size, I = c.intermediate_size;
  const size_t kv_rows_off = (size_t)e->q_dim * H;  // element offset of K rows in qkv_proj
  for (int l = 0; l < c.num_layers; ++l) {
    const grout_qwen3_layer& w = e->layers[l];
    if (l == 0)
      GROUT_CHECK(norm(e, nullptr, e->p(b.hidden), w.input_layernorm, e->p(b.normed), nullptr, n));
    else
      GROUT_CHECK(norm(e, e->p(b.hidden_after_attn), e->p(b.ff_down), w.input_layernorm,
                       e->p(b.normed), e->p(b.hidden), n));
    const uint16_t* wqkv = static_cast<const uint16_t*>(w.qkv_proj);
    GROUT_CHECK(project(e, wqkv, e->p(b.normed), e->p(b.q), n, e->q_dim, H));
    GROUT_CHECK(project(e, wqkv + kv_rows_off, e->p(b.normed), e->p(b.k), n, e->kv_dim, H));
    GROUT_CHECK(project(e, wqkv + kv_rows_off + (size_t)e->kv_dim * H, e->p(b.normed), e->p(b.v),
                        n, e->kv_dim, H));
    GROUT_CHECK(grout_qk_norm_rope_kv_prefill(
        e->p(b.q), e->p(b.k), e->p(b.v), w.q_norm, w.k_norm, e->rope_cos(), e->rope_sin(),
        e->p(b.q_rope), e->k_cache(l), e->v_cache(l), pos0, n, c.num_q_heads, c.num_kv_heads,
        128, c.max_ctx, e->head_stride, c.rms_norm_eps, s));
    GROUT_CHECK(grout_fmha_prefill(e->p(b.q_rope), e->k_cache(l), e->v_cache(l),
                                   e->p(b.attn_out), n, pos0, c.num_q_heads, c.num_kv_heads, 128,
                                   e->head_stride, e->qk_scale, s));
    GROUT_CHECK(project(e, w.o_proj, e->p(b.attn_out), e->p(b.attn_proj), n, H, e->q_dim));
    GROUT_CHECK(norm(e, e->p(b.hidden), e->p(b.attn_proj), w.post_attention_layernorm,
                     e->p(b.ff_normed), e->p(b.hidden_after_attn), n));
    GROUT_CHECK(project(e, w.gate_up_proj, e->p(b.ff_normed), e->p(b.gate_up), n, 2 * I, H));
    GROUT_CHECK(hip_status(grout::launch_silu_mul(e->p(b.gate_up), e->p(b.ff), n, I, s),
                           "silu_mul"));
    GROUT_CHECK(project(e, w.down_proj, e->p(b.ff), e->p(b.ff_down), n, H, I));
  }
  // Only the last token's logits are needed (src/model.rs api_prefill_logits).
  const size_t last = (size_t)(n - 1) * H;
  GROUT_CHECK(head(e, e->p<uint16_t>(b.hidden_after_attn) + last, e->p<uint16_t>(b.ff_down) + last));
  GROUT_CHECK(copy_logits_out(e, logits_out, next_token));
  e->next_pos = pos0 + n;
  e->session_active = true;
  return GROUT_OK;
}

}  // namespace

extern "C" {

int grout_engine_prefill(grout_engine* e, const uint32_t* tokens, int n, float* logits_out,
                         uint32_t* next_token) {
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "engine is NULL");
  GROUT_CHECK(take_pending(e));
  return run_chunk(e, tokens, n, 0, logits_out, next_token);
}

int grout_engine_extend(grout_engine* e, const uint32_t* tokens, int n, float* logits_out,
                        uint32_t* next_token) {
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "engine is NULL");
  GROUT_CHECK(take_pending(e));
  GROUT_NEED(e->session_active, GROUT_EINVAL, "extend requires a preceding prefill");
  return run_chunk(e, tokens, n, e->next_pos, logits_out, next_token);
}

int grout_engine_decode(grout_engine* e, uint32_t token, float* logits_out) {
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "engine is NULL");
  GROUT_CHECK(decode_common(e, token));
  return copy_logits_out(e, logits_out, nullptr);
}

int grout_engine_decode_greedy(grout_engine* e, uint32_t token, uint32_t* next_token) {
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "engine is NULL");
  GROUT_NEED(next_token != nullptr, GROUT_EINVAL, "next_token is NULL");
  GROUT_CHECK(decode_common(e, token));
  return copy_logits_out(e, nullptr, next_token);
}

int grout_engine_reset(grout_engine* e) {
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "engine is NULL");
  e->next_pos = 0;
  e->session_active = false;
  int rc = hip_status(hipSetDevice(e->device), "hipSetDevice");
  if (rc == GROUT_OK)
    rc = hip_status(
        hipMemsetAsync(e->kv, 0, (size_t)e->cfg.num_layers * 2 * e->cache_bytes(), e->stream),
        "hipMemset(kv caches)");
  if (rc == GROUT_OK) rc = hip_status(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
  if (rc != GROUT_OK) {
    e->pending_reset_error = g_last_error;
    return fail(rc, "reset failed: %s", e->pending_reset_error.c_str());
  }
  return GROUT_OK;
}

int grout_engine_position(const grout_engine* e) { return e ? e->next_pos : -1; }

int grout_engine_destroy(grout_engine* e) {
  if (!e) return GROUT_OK;
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  if (e->exec) (void)hipGraphExecDestroy(e->exec);
  if (e->graph) (void)hipGraphDestroy(e->graph);
  if (e->blas) (void)rocblas_destroy_handle(e->blas);
  if (e->pre.base) (void)hipFree(e->pre.base);
  if (e->dec.base) (void)hipFree(e->dec.base);
  if (e->rope) (void)hipFree(e->rope);
  if (e->kv) (void)hipFree(e->kv);
  if (e->h_logits) (void)hipHostFree(e->h_logits);
  if (e->h_token) (void)hipHostFree(e->h_token);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  grout_model* m = e->owned_model;
  delete e;
  return grout_model_free(m);
}

int grout_engine_load(const char* model_dir, int max_ctx, int device, grout_engine** out) {
  GROUT_NEED(out != nullptr, GROUT_EINVAL, "out is NULL");
  *out = nullptr;
  GROUT_NEED(max_ctx >= 0, GROUT_EINVAL, "max_ctx=%d", max_ctx);
  grout_model* m = nullptr;
  GROUT_CHECK(grout_model_load(model_dir, device, &m));
  grout_model_info info;
  grout_qwen3_weights w;
  (void)grout_model_get_info(m, &info);
  (void)grout_model_weights(m, &w);
  grout_qwen3_config cfg = info.config;
  if (max_ctx > 0) cfg.max_ctx = max_ctx;
  grout_engine* e = nullptr;
  const int rc = grout_engine_create(&cfg, &w, device, &e);
  if (rc != GROUT_OK) {
    const std::string msg = g_last_error;
    grout_model_free(m);
    g_last_error = msg;
    return rc;
  }
  e->owned_model = m;
  *out = e;
  return GROUT_OK;
}

int grout_engine_model_info(const grout_engine* e, grout_model_info* info) {
  GROUT_NEED(e != nullptr && info != nullptr, GROUT_EINVAL, "engine or info is NULL");
  GROUT_NEED(e->owned_model != nullptr, GROUT_EINVAL,
             "engine was created from caller weights, not loaded from a model directory");
  GROUT_CHECK(grout_model_get_info(e->owned_model, info));
  info->config.max_ctx = e->cfg.max_ctx;
  return GROUT_OK;
}

}  // extern "C"
