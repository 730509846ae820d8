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

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
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

// One weight matrix (a part of a projection): f16 [rows][k] or a low-bit
// layout (grout_qweight_repack).
struct Mat {
  int fmt = GROUT_WFMT_F16;
  int rows = 0;
  const void* data = nullptr;
};

struct LayerW {
  const void* input_norm = nullptr;
  const void* q_norm = nullptr;
  const void* k_norm = nullptr;
  const void* post_norm = nullptr;
  int nqkv = 0;
  Mat qkv[3];  // q | k | v rows
  Mat o;
  int ngu = 0;
  Mat gu[2];  // gate | up rows
  Mat down;
};

// A projection held as one f16 matrix: the fused-norm f16 GEMV paths apply.
bool single_f16(const Mat* parts, int n) { return n == 1 && parts[0].fmt == GROUT_WFMT_F16; }

// Decode-step activations: one token.
struct DecodeBufs {
  size_t hidden, normed, hidden_after_attn, qkv, attn_out, attn_proj, gate_up, ff, ff_down,
      logits, argmax_max, argmax_idx, token, pos, workspace;
};

// Prefill activations: cap rows.
struct PrefillBufs {
  size_t ids, hidden, normed, hidden_after_attn, qkv, q_rope, attn_out, attn_proj, ff_normed,
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
  Mat embed;
  const void* final_norm = nullptr;
  Mat lm_head;
  std::vector<LayerW> layers;
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
  // f16 copy of one low-bit matrix at a time for the prefill GEMMs
  void* deq = nullptr;
  size_t deq_bytes = 0;

  // Pinned host staging.
  uint16_t* h_logits = nullptr;
  uint32_t* h_token = nullptr;

  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  // Why decode runs without the graph ("" while the graph is in use).
  std::string graph_error;

  int next_pos = 0;
  bool session_active = false;
  // What the device's decode token / position words hold, as far as the host
  // knows (-1: unknown).  Each decode step leaves its argmax and position + 1
  // there; a step whose token and position match needs no write.
  long dev_token = -1, dev_pos = -1;
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

// y[rows][0..n) = x[rows][k] . W[n][k]^T with y's rows ldy apart, fp16
// in/out, fp32 accumulation.  In rocBLAS's column-major terms: C (n x rows,
// ldc ldy) = W^T (col-major k x n, transposed) x X (col-major k x rows).
int gemm_rows(grout_engine* e, const void* W, const void* x, void* y, int rows, int n, int k,
              int ldy) {
  const float alpha = 1.f, beta = 0.f;
  return blas_status(
      rocblas_gemm_ex(e->blas, rocblas_operation_transpose, rocblas_operation_none, n, rows, k,
                      &alpha, W, rocblas_datatype_f16_r, k, x, rocblas_datatype_f16_r, k, &beta, y,
                      rocblas_datatype_f16_r, ldy, y, rocblas_datatype_f16_r, ldy,
                      rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0),
      "rocblas_gemm_ex");
}

// Projection of `rows` tokens by an f16 matrix.  One row uses the decode
// GEMV kernel.
int project(grout_engine* e, const void* W, const void* x, void* y, int rows, int n, int k) {
  if (rows == 1) return hip_status(grout::launch_gemv(W, x, y, n, k, e->stream), "gemv");
  return gemm_rows(e, W, x, y, rows, n, k, n);
}

// One token through one weight part with the decode GEMV of its format.
int mat_gemv(grout_engine* e, const Mat& m, const void* x, void* y, int k) {
  if (m.fmt == GROUT_WFMT_F16)
    return hip_status(grout::launch_gemv(m.data, x, y, m.rows, k, e->stream), "gemv");
  return hip_status(grout::launch_gemv_q(m.fmt, m.data, x, y, m.rows, k, false, e->stream),
                    "gemv_q");
}

// f16 [rows][k] form of a part for the prefill GEMM: an f16 part as it is, a
// low-bit part dequantized into the engine's scratch (the scratch holds one
// matrix at a time; stream order keeps its reuse safe).
int mat_f16(grout_engine* e, const Mat& m, int k, const void** w) {
  if (m.fmt == GROUT_WFMT_F16) {
    *w = m.data;
    return GROUT_OK;
  }
  GROUT_CHECK(hip_status(grout::launch_qweight_dequant(m.fmt, m.data, m.rows, k, e->deq, e->stream),
                         "qweight dequant"));
  *w = e->deq;
  return GROUT_OK;
}

// Projection of `rows` tokens by one part into columns [0, m.rows) of y
// (rows ldy apart).
int mat_project(grout_engine* e, const Mat& m, const void* x, void* y, int rows, int k, int ldy) {
  if (m.fmt == GROUT_WFMT_F16 && ldy == m.rows) return project(e, m.data, x, y, rows, m.rows, k);
  const void* w = nullptr;
  GROUT_CHECK(mat_f16(e, m, k, &w));
  return gemm_rows(e, w, x, y, rows, m.rows, k, ldy);
}

// Token-embedding rows for ids (device memory).
int embed_rows(grout_engine* e, const uint32_t* ids, void* out, int rows) {
  const auto& c = e->cfg;
  if (e->embed.fmt == GROUT_WFMT_F16)
    return hip_status(grout::launch_embedding(ids, e->embed.data, out, rows, c.hidden_size,
                                              c.vocab_size, e->stream),
                      "embedding");
  return hip_status(grout::launch_qgather(e->embed.fmt, e->embed.data, c.vocab_size, c.hidden_size,
                                          ids, rows, out, e->stream),
                    "embedding gather");
}

int norm(grout_engine* e, const void* residual, const void* x, const void* w, void* out,
         void* residual_out, int rows) {
  return hip_status(grout::launch_rms_norm(residual, x, w, out, residual_out, rows,
                                           e->cfg.hidden_size, e->cfg.rms_norm_eps, e->stream),
                    "rms_norm");
}

// Final norm (folding the last layer's residual add), lm_head and argmax
// over one token's hidden state; leaves f16 logits and the token on device
// (and, when advance_pos is set, moves that position word on by one).
int head(grout_engine* e, const void* hidden_after_attn, const void* ff_down,
         uint32_t* advance_pos = nullptr) {
  const auto& c = e->cfg;
  GROUT_CHECK(norm(e, hidden_after_attn, ff_down, e->final_norm, e->d(e->db.normed),
                   e->d(e->db.hidden), 1));
  GROUT_CHECK(mat_gemv(e, e->lm_head, e->d(e->db.normed), e->d(e->db.logits), c.hidden_size));
  return hip_status(grout::launch_argmax(e->d(e->db.logits), e->d<float>(e->db.argmax_max),
                                         e->d<uint32_t>(e->db.argmax_idx), c.vocab_size,
                                         e->d<uint32_t>(e->db.token), e->stream, advance_pos),
                    "argmax");
}

// One token through one weight part with the input RMSNorm folded into the
// GEMV (x' = norm(residual + x) * gamma, or norm(x) * gamma without a
// residual); f16(residual + x) goes to residual_out.  Every part of a
// projection recomputes x' and writes the same residual_out bits.
int mat_gemv_norm(grout_engine* e, const Mat& m, const void* residual, const void* x,
                  const void* gamma, void* residual_out, void* y, int k, bool silu_rows) {
  const float eps = e->cfg.rms_norm_eps;
  if (m.fmt == GROUT_WFMT_F16)
    return hip_status(grout::launch_gemv_norm(m.data, residual, x, gamma, residual_out, eps, y,
                                              silu_rows ? m.rows / 2 : m.rows, k, silu_rows,
                                              e->stream),
                      "gemv_norm");
  return hip_status(grout::launch_gemv_q_norm(m.fmt, m.data, residual, x, gamma, residual_out, eps,
                                              y, silu_rows ? m.rows / 2 : m.rows, k, silu_rows,
                                              e->stream),
                    "gemv_q_norm");
}

// The decode step, as recorded into the graph.  The input and
// post-attention norms fold into the first GEMV of their projection (every
// part of a multi-part projection recomputes them).
int record_decode_step(grout_engine* e) {
  const auto& c = e->cfg;
  const DecodeBufs& b = e->db;
  hipStream_t s = e->stream;
  const int H = c.hidden_size, I = c.intermediate_size;
  GROUT_CHECK(embed_rows(e, e->d<uint32_t>(b.token), e->d(b.hidden), 1));
  for (int l = 0; l < c.num_layers; ++l) {
    const LayerW& w = e->layers[l];
    // input norm (layer 0: plain RMSNorm of the embedding; later layers: add
    // the previous layer's MLP output first), then the QKV projection
    const void* res = l == 0 ? nullptr : e->d(b.hidden_after_attn);
    const void* xin = l == 0 ? e->d(b.hidden) : e->d(b.ff_down);
    void* res_out = l == 0 ? nullptr : e->d(b.hidden);
    size_t row = 0;
    for (int i = 0; i < w.nqkv; ++i) {
      GROUT_CHECK(mat_gemv_norm(e, w.qkv[i], res, xin, w.input_norm, res_out,
                                e->d<uint16_t>(b.qkv) + row, H, false));
      row += (size_t)w.qkv[i].rows;
    }
    // QK-norm/RoPE + K/V cache write inside the split-K attention, then the merge
    GROUT_CHECK(grout_attn_decode_fused(
        e->d(b.qkv), w.q_norm, w.k_norm, e->rope_cos(), e->rope_sin(), e->k_cache(l),
        e->v_cache(l), e->d(b.attn_out), e->d(b.workspace), e->ws_bytes,
        e->d<uint32_t>(b.pos), c.num_q_heads, c.num_kv_heads, 128, c.max_ctx, e->head_stride,
        e->num_splits, c.rms_norm_eps, e->qk_scale, s));
    GROUT_CHECK(mat_gemv(e, w.o, e->d(b.attn_out), e->d(b.attn_proj), e->q_dim));
    // post-attention add + RMSNorm, gate_up and SiLU(gate) * up into ff
    if (w.ngu == 1) {  // SiLU(gate) * up in the GEMV epilogue
      GROUT_CHECK(mat_gemv_norm(e, w.gu[0], e->d(b.hidden), e->d(b.attn_proj), w.post_norm,
                                e->d(b.hidden_after_attn), e->d(b.ff), H, true));
    } else {
      GROUT_CHECK(mat_gemv_norm(e, w.gu[0], e->d(b.hidden), e->d(b.attn_proj), w.post_norm,
                                e->d(b.hidden_after_attn), e->d(b.gate_up), H, false));
      GROUT_CHECK(mat_gemv_norm(e, w.gu[1], e->d(b.hidden), e->d(b.attn_proj), w.post_norm,
                                e->d(b.hidden_after_attn), e->d<uint16_t>(b.gate_up) + w.gu[0].rows,
                                H, false));
      GROUT_CHECK(hip_status(grout::launch_silu_mul(e->d(b.gate_up), e->d(b.ff), 1, I, s),
                             "silu_mul"));
    }
    GROUT_CHECK(mat_gemv(e, w.down, e->d(b.ff), e->d(b.ff_down), I));
  }
  // The step leaves the next step's token (the greedy argmax) and position
  // behind, so a greedy decode loop needs no write of its own per token.
  return head(e, e->d(b.hidden_after_attn), e->d(b.ff_down), e->d<uint32_t>(b.pos));
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

// The decode-step graph, or the sequential fallback: GROUT_HIP_GRAPH_DECODE
// set off (read like the reference's GROUT_CUDA_GRAPH_DECODE, default on)
// skips the capture, and a failed capture is reported on stderr and recorded
// (src/model.rs:1700-1701, 2130-2145, 2300-2309).  Either way decode then
// launches record_decode_step's kernels directly, in the same order.
int setup_decode_graph(grout_engine* e) {
  const char* env = std::getenv("GROUT_HIP_GRAPH_DECODE");
  if (!parse_bool_or(env, true)) {
    e->graph_error = std::string("decode graph disabled by GROUT_HIP_GRAPH_DECODE=") + env;
    return GROUT_OK;
  }
  if (capture_decode_graph(e) == GROUT_OK) return GROUT_OK;
  e->graph_error = "decode graph capture failed: " + g_last_error;
  std::fprintf(stderr, "grout: warning: %s; falling back to sequential decode\n",
               e->graph_error.c_str());
  (void)hipGetLastError();
  if (e->exec) (void)hipGraphExecDestroy(e->exec);
  if (e->graph) (void)hipGraphDestroy(e->graph);
  e->exec = nullptr;
  e->graph = nullptr;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(e->stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(e->stream, &g);
    if (g) (void)hipGraphDestroy(g);
  }
  // the stream must still work for the sequential path
  return hip_status(hipStreamSynchronize(e->stream), "hipStreamSynchronize");
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
  b.qkv = a.take(r * e->qkv_dim * h2);  // rows [Q | K | V], qkv_dim apart
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
  // The previous step left its greedy token and this position on the device
  // (the usual decode_greedy loop): one graph launch.  Otherwise token and
  // position travel as kernel arguments of a one-thread kernel first: no host
  // staging buffer that a queued replay could still be reading.
  const bool ready = e->dev_token == (long)token && e->dev_pos == (long)e->next_pos;
  e->dev_token = -1;
  e->dev_pos = -1;
  if (!ready) {
    set_step_kernel<<<1, 1, 0, e->stream>>>(e->d<uint32_t>(e->db.token), token,
                                            e->d<uint32_t>(e->db.pos), (uint32_t)e->next_pos);
    GROUT_CHECK(hip_status(hipGetLastError(), "set step"));
  }
  if (e->exec)
    GROUT_CHECK(hip_status(hipGraphLaunch(e->exec, e->stream), "hipGraphLaunch"));
  else
    GROUT_CHECK(record_decode_step(e));
  e->next_pos += 1;
  e->dev_pos = e->next_pos;
  return GROUT_OK;
}

int validate_config(const grout_qwen3_config* c) {
  GROUT_NEED(c != nullptr, GROUT_EINVAL, "config is NULL");
  GROUT_NEED(c->num_layers >= 1, GROUT_EINVAL, "num_layers=%d", c->num_layers);
  GROUT_CHECK(check_heads(c->num_q_heads, c->num_kv_heads, c->head_dim, kMaxDecodeGroup));
  GROUT_NEED(c->hidden_size >= 8 && c->hidden_size % 8 == 0 && c->hidden_size <= 8192,
             GROUT_ENOTSUP, "hidden_size=%d must be a multiple of 8 in [8, 8192]",
             c->hidden_size);
  GROUT_NEED(c->intermediate_size >= 8 && c->intermediate_size % 8 == 0, GROUT_ENOTSUP,
             "intermediate_size=%d must be a positive multiple of 8", c->intermediate_size);
  GROUT_NEED(c->vocab_size >= 1, GROUT_EINVAL, "vocab_size=%d", c->vocab_size);
  GROUT_NEED(c->max_ctx >= 1 && c->max_ctx <= GROUT_MAX_CTX, GROUT_ENOTSUP,
             "max_ctx=%d outside [1, %d]", c->max_ctx, GROUT_MAX_CTX);
  GROUT_NEED(std::isfinite(c->rms_norm_eps) && c->rms_norm_eps > 0.f, GROUT_EINVAL,
             "rms_norm_eps=%g", (double)c->rms_norm_eps);
  GROUT_NEED(std::isfinite(c->rope_theta) && c->rope_theta > 0.f, GROUT_EINVAL, "rope_theta=%g",
             (double)c->rope_theta);
  return GROUT_OK;
}

// The f16 API's weights as single-part projections.
int convert_f16(const grout_qwen3_config* c, const grout_qwen3_weights* w, Mat& embed,
                Mat& lm_head, std::vector<LayerW>& layers) {
  GROUT_NEED(w != nullptr, GROUT_EINVAL, "weights is NULL");
  GROUT_CHECK(check_ptrs16({{w->embed_tokens, "embed_tokens"}, {w->norm, "norm"},
                            {w->lm_head, "lm_head"}}));
  GROUT_NEED(w->layers != nullptr, GROUT_EINVAL, "layers is NULL");
  const int qd = c->num_q_heads * 128, qkv = qd + 2 * c->num_kv_heads * 128;
  embed = Mat{GROUT_WFMT_F16, c->vocab_size, w->embed_tokens};
  lm_head = Mat{GROUT_WFMT_F16, c->vocab_size, w->lm_head};
  layers.assign(c->num_layers, LayerW{});
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
    LayerW& o = layers[l];
    o.input_norm = L.input_layernorm;
    o.q_norm = L.q_norm;
    o.k_norm = L.k_norm;
    o.post_norm = L.post_attention_layernorm;
    o.nqkv = 1;
    o.qkv[0] = Mat{GROUT_WFMT_F16, qkv, L.qkv_proj};
    o.o = Mat{GROUT_WFMT_F16, c->hidden_size, L.o_proj};
    o.ngu = 1;
    o.gu[0] = Mat{GROUT_WFMT_F16, 2 * c->intermediate_size, L.gate_up_proj};
    o.down = Mat{GROUT_WFMT_F16, c->hidden_size, L.down_proj};
  }
  return GROUT_OK;
}

int check_part(const grout_wpart& p, int k, const char* what, int layer) {
  const char* lname = layer < 0 ? "" : " of layer ";
  GROUT_NEED(p.fmt == GROUT_WFMT_F16 || p.fmt == GROUT_WFMT_Q8_0 || p.fmt == GROUT_WFMT_Q4_K ||
                 p.fmt == GROUT_WFMT_Q5_K || p.fmt == GROUT_WFMT_Q6_K,
             GROUT_ENOTSUP, "%s%s%d: format %d is not f16, Q8_0, Q4_K, Q5_K or Q6_K", what, lname,
             layer, p.fmt);
  GROUT_NEED(p.rows >= 1, GROUT_EINVAL, "%s%s%d: rows=%d", what, lname, layer, p.rows);
  GROUT_NEED(p.data != nullptr && aligned16(p.data), GROUT_EINVAL,
             "%s%s%d: data is NULL or not 16-byte aligned", what, lname, layer);
  if (p.fmt == GROUT_WFMT_F16)
    GROUT_NEED(k % 8 == 0, GROUT_ENOTSUP, "%s%s%d: f16 needs k %% 8 == 0 (k=%d)", what, lname,
               layer, k);
  else
    GROUT_NEED(grout::qweight_bytes(p.fmt, p.rows, k) != 0, GROUT_ENOTSUP,
               "%s%s%d: format %d does not fit k=%d (a multiple of the block size, at most "
               "32768)",
               what, lname, layer, p.fmt, k);
  return GROUT_OK;
}

Mat to_mat(const grout_wpart& p) { return Mat{p.fmt, p.rows, p.data}; }

// The mixed-format API's weights, checked part by part.
int convert_q(const grout_qwen3_config* c, const grout_qwen3_qweights* w, Mat& embed,
              Mat& lm_head, std::vector<LayerW>& layers) {
  GROUT_NEED(w != nullptr, GROUT_EINVAL, "weights is NULL");
  const int H = c->hidden_size, I = c->intermediate_size, V = c->vocab_size;
  const int qd = c->num_q_heads * 128, qkv = qd + 2 * c->num_kv_heads * 128;
  GROUT_CHECK(check_part(w->embed_tokens, H, "embed_tokens", -1));
  GROUT_CHECK(check_part(w->lm_head, H, "lm_head", -1));
  GROUT_NEED(w->embed_tokens.rows == V && w->lm_head.rows == V, GROUT_EINVAL,
             "embed_tokens / lm_head rows %d / %d != vocab_size=%d", w->embed_tokens.rows,
             w->lm_head.rows, V);
  GROUT_CHECK(check_ptrs16({{w->norm, "norm"}}));
  GROUT_NEED(w->layers != nullptr, GROUT_EINVAL, "layers is NULL");
  embed = to_mat(w->embed_tokens);
  lm_head = to_mat(w->lm_head);
  layers.assign(c->num_layers, LayerW{});
  for (int l = 0; l < c->num_layers; ++l) {
    const grout_qwen3_qlayer& L = w->layers[l];
    const int rc = check_ptrs16({{L.input_layernorm, "input_layernorm"},
                                 {L.q_norm, "q_norm"},
                                 {L.k_norm, "k_norm"},
                                 {L.post_attention_layernorm, "post_attention_layernorm"}});
    if (rc != GROUT_OK) return fail(rc, "layer %d: %s", l, g_last_error.c_str());
    GROUT_NEED(L.num_qkv_parts >= 1 && L.num_qkv_parts <= 3, GROUT_EINVAL,
               "layer %d: num_qkv_parts=%d", l, L.num_qkv_parts);
    GROUT_NEED(L.num_gate_up_parts >= 1 && L.num_gate_up_parts <= 2, GROUT_EINVAL,
               "layer %d: num_gate_up_parts=%d", l, L.num_gate_up_parts);
    LayerW& o = layers[l];
    o.input_norm = L.input_layernorm;
    o.q_norm = L.q_norm;
    o.k_norm = L.k_norm;
    o.post_norm = L.post_attention_layernorm;
    long sum = 0;
    o.nqkv = L.num_qkv_parts;
    for (int i = 0; i < o.nqkv; ++i) {
      GROUT_CHECK(check_part(L.qkv[i], H, "qkv part", l));
      o.qkv[i] = to_mat(L.qkv[i]);
      sum += L.qkv[i].rows;
    }
    GROUT_NEED(sum == qkv, GROUT_EINVAL, "layer %d: qkv parts cover %ld rows, expected %d", l,
               sum, qkv);
    sum = 0;
    o.ngu = L.num_gate_up_parts;
    for (int i = 0; i < o.ngu; ++i) {
      GROUT_CHECK(check_part(L.gate_up[i], H, "gate_up part", l));
      o.gu[i] = to_mat(L.gate_up[i]);
      sum += L.gate_up[i].rows;
    }
    GROUT_NEED(sum == 2L * I, GROUT_EINVAL, "layer %d: gate_up parts cover %ld rows, expected %d",
               l, sum, 2 * I);
    // two parts must split at the gate | up boundary (silu pairs row i with i + I)
    GROUT_NEED(o.ngu == 1 || o.gu[0].rows == I, GROUT_EINVAL,
               "layer %d: the first gate_up part has %d rows, expected %d (gate)", l,
               o.gu[0].rows, I);
    GROUT_CHECK(check_part(L.o_proj, qd, "o_proj", l));
    GROUT_CHECK(check_part(L.down_proj, I, "down_proj", l));
    GROUT_NEED(L.o_proj.rows == H && L.down_proj.rows == H, GROUT_EINVAL,
               "layer %d: o_proj / down_proj rows %d / %d != hidden_size=%d", l, L.o_proj.rows,
               L.down_proj.rows, H);
    o.o = to_mat(L.o_proj);
    o.down = to_mat(L.down_proj);
  }
  return GROUT_OK;
}

// Largest low-bit matrix the prefill dequantizes (bytes of its f16 form).
size_t dequant_scratch_bytes(const grout_engine* e) {
  const auto& c = e->cfg;
  size_t mx = 0;
  auto see = [&](const Mat& m, int k) {
    if (m.fmt != GROUT_WFMT_F16) mx = std::max(mx, (size_t)m.rows * k * sizeof(uint16_t));
  };
  for (const LayerW& w : e->layers) {
    for (int i = 0; i < w.nqkv; ++i) see(w.qkv[i], c.hidden_size);
    for (int i = 0; i < w.ngu; ++i) see(w.gu[i], c.hidden_size);
    see(w.o, e->q_dim);
    see(w.down, c.intermediate_size);
  }
  return mx;
}

// Takes the converted weights (embed, lm_head, layers moved in).
int create_impl(grout_engine* e, const grout_qwen3_config* c, const void* final_norm, Mat embed,
                Mat lm_head, std::vector<LayerW>&& layers, int device) {
  e->cfg = *c;
  e->device = device;
  e->embed = embed;
  e->final_norm = final_norm;
  e->lm_head = lm_head;
  e->layers = std::move(layers);
  e->q_dim = c->num_q_heads * 128;
  e->kv_dim = c->num_kv_heads * 128;
  e->qkv_dim = e->q_dim + 2 * e->kv_dim;
  e->head_stride = (long)c->max_ctx * 128;
  // GROUT_FMHA_NUM_KV_SPLITS overrides the decode split count, as the
  // reference's does (src/model.rs:2713-2714), capped at GROUT_MAX_SPLITS.
  {
    const long dflt =
        grout_attn_decode_default_splits(c->max_ctx, c->num_q_heads, c->num_kv_heads);
    const long ns = parse_usize_or(std::getenv("GROUT_FMHA_NUM_KV_SPLITS"), dflt);
    e->num_splits = (int)(ns < GROUT_MAX_SPLITS ? ns : GROUT_MAX_SPLITS);
  }
  e->ws_bytes = decode_ws_bytes(c->num_q_heads, c->num_kv_heads, e->num_splits);
  e->argmax_blocks = grout::argmax_num_blocks(c->vocab_size);
  e->qk_scale = 1.0f / std::sqrt(128.0f);  // src/model.rs:2654, 6901

  // Decode buffers (offsets only until the preflight has passed).
  const size_t H = c->hidden_size, I = c->intermediate_size, h2 = sizeof(uint16_t);
  Arena a;
  DecodeBufs& b = e->db;
  b.hidden = a.take(H * h2);
  b.normed = a.take(H * h2);
  b.hidden_after_attn = a.take(H * h2);
  b.qkv = a.take(e->qkv_dim * h2);
  b.attn_out = a.take(e->q_dim * h2);
  b.attn_proj = a.take(H * h2);
  b.gate_up = a.take(2 * I * h2);
  b.ff = a.take(I * h2);
  b.ff_down = a.take(H * h2);
  b.logits = a.take((size_t)c->vocab_size * h2);
  b.argmax_max = a.take((size_t)e->argmax_blocks * sizeof(float));
  b.argmax_idx = a.take((size_t)e->argmax_blocks * sizeof(uint32_t));
  b.token = a.take(sizeof(uint32_t));
  b.pos = a.take(sizeof(uint32_t));
  b.workspace = a.take(e->ws_bytes);
  e->deq_bytes = dequant_scratch_bytes(e);

  GROUT_CHECK(hip_status(hipSetDevice(device), "hipSetDevice"));
  // VRAM preflight before the caches are allocated (src/model.rs:1491-1506);
  // the caller's weights are resident already.
  size_t free_b = 0, total_b = 0;
  GROUT_CHECK(hip_status(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo"));
  GROUT_CHECK(grout_engine_vram_preflight(c, 0, a.used + e->deq_bytes, free_b, total_b, nullptr));

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

  GROUT_CHECK(hip_status(hipMalloc(&a.base, a.used), "hipMalloc(decode buffers)"));
  e->dec = a;
  GROUT_CHECK(hip_status(hipMemsetAsync(a.base, 0, a.used, e->stream), "hipMemset(decode)"));

  GROUT_CHECK(hip_status(hipHostMalloc(reinterpret_cast<void**>(&e->h_logits),
                                       (size_t)c->vocab_size * h2, hipHostMallocDefault),
                         "hipHostMalloc(logits)"));
  GROUT_CHECK(hip_status(hipHostMalloc(reinterpret_cast<void**>(&e->h_token), sizeof(uint32_t),
                                       hipHostMallocDefault),
                         "hipHostMalloc(token)"));
  if (e->deq_bytes)
    GROUT_CHECK(hip_status(hipMalloc(&e->deq, e->deq_bytes), "hipMalloc(dequant scratch)"));
  GROUT_CHECK(hip_status(hipStreamSynchronize(e->stream), "hipStreamSynchronize"));
  return setup_decode_graph(e);
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

// True when the byte ranges [a, a + an) and [b, b + bn) share a byte.
static bool ranges_overlap(const void* a, size_t an, const void* b, size_t bn) {
  if (a == nullptr || b == nullptr || an == 0 || bn == 0) return false;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + bn && pb < pa + an;
}

// One workgroup of the fused-norm GEMVs writes residual_out[0, k) while the
// others still read residual and x: any overlap of those f16 vectors races,
// not only the same start address.
static int check_residual_out(const void* residual, const void* x, const void* residual_out,
                              int k) {
  const size_t bytes = (size_t)k * sizeof(uint16_t);
  GROUT_NEED(!ranges_overlap(residual_out, bytes, residual, bytes) &&
                 !ranges_overlap(residual_out, bytes, x, bytes),
             GROUT_EINVAL, "residual_out must not overlap residual or x");
  return GROUT_OK;
}

static int check_gemv_norm(const void* W, const void* residual, const void* x,
                           const void* gamma, void* residual_out, void* y, int n, int k,
                           float eps) {
  GROUT_NEED(n >= 1, GROUT_EINVAL, "n=%d", n);
  GROUT_CHECK(check_norm(1, k, eps));
  GROUT_CHECK(check_ptrs16({{W, "W"}, {x, "x"}, {gamma, "gamma"}}));
  if (residual) {  // residual_out is written only with a residual
    GROUT_CHECK(check_ptrs16({{residual, "residual"}, {residual_out, "residual_out"}}));
    GROUT_CHECK(check_residual_out(residual, x, residual_out, k));
  }
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
  GROUT_NEED(fmt == GROUT_WFMT_Q8_0 || fmt == GROUT_WFMT_Q4_K || fmt == GROUT_WFMT_Q5_K ||
                 fmt == GROUT_WFMT_Q6_K,
             GROUT_ENOTSUP, "weight format %d: Q8_0 (8), Q4_K (12), Q5_K (13) or Q6_K (14) expected",
             fmt);
  GROUT_NEED(grout::qweight_bytes(fmt, n, k) != 0, GROUT_EINVAL,
             "[%d][%d] of format %d: k must be a multiple of the block size and <= 32768", n, k,
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

static int check_q_norm(const void* wq, const void* residual, const void* x, const void* gamma,
                        const void* residual_out, const void* y, int k, float eps) {
  GROUT_CHECK(check_ptrs16({{wq, "wq"}, {x, "x"}, {gamma, "gamma"}}));
  if (residual) GROUT_CHECK(check_ptrs16({{residual, "residual"}}));
  if (residual_out) {
    GROUT_CHECK(check_ptrs16({{residual_out, "residual_out"}}));
    GROUT_CHECK(check_residual_out(residual, x, residual_out, k));
  }
  GROUT_NEED(y != nullptr && (reinterpret_cast<uintptr_t>(y) & 1u) == 0, GROUT_EALIGN,
             "y is NULL or not 2-byte aligned");
  GROUT_NEED(std::isfinite(eps) && eps > 0.f, GROUT_EINVAL, "eps=%g", (double)eps);
  return GROUT_OK;
}

int grout_gemv_q_rms_norm(int fmt, const void* wq, const void* residual, const void* x,
                          const void* gamma, void* residual_out, void* y, int n, int k, float eps,
                          void* stream) {
  GROUT_CHECK(check_q(fmt, n, k));
  GROUT_CHECK(check_q_norm(wq, residual, x, gamma, residual_out, y, k, eps));
  return hip_status(grout::launch_gemv_q_norm(fmt, wq, residual, x, gamma, residual_out, eps, y, n,
                                              k, false, as_stream(stream)),
                    "gemv_q_rms_norm launch");
}

int grout_gemv_q_rms_norm_silu_mul(int fmt, const void* wq, const void* residual, const void* x,
                                   const void* gamma, void* residual_out, void* y, int inter,
                                   int k, float eps, void* stream) {
  GROUT_CHECK(check_q(fmt, 2 * inter, k));
  GROUT_CHECK(check_q_norm(wq, residual, x, gamma, residual_out, y, k, eps));
  return hip_status(grout::launch_gemv_q_norm(fmt, wq, residual, x, gamma, residual_out, eps, y,
                                              inter, k, true, as_stream(stream)),
                    "gemv_q_rms_norm_silu_mul launch");
}

int grout_qweight_gather(int fmt, const void* wq, int n, int k, const uint32_t* ids, int rows,
                         void* out, void* stream) {
  GROUT_CHECK(check_q(fmt, n, k));
  GROUT_NEED(rows >= 1, GROUT_EINVAL, "rows=%d", rows);
  GROUT_CHECK(check_ptrs16({{wq, "wq"}, {out, "out"}}));
  GROUT_NEED(ids != nullptr, GROUT_EINVAL, "ids is NULL");
  return hip_status(grout::launch_qgather(fmt, wq, n, k, ids, rows, out, as_stream(stream)),
                    "qweight gather launch");
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

}  // extern "C"

namespace {

template <class Convert>
int create_common(const grout_qwen3_config* config, const void* norm, int device,
                  grout_engine** out, Convert convert) {
  GROUT_NEED(out != nullptr, GROUT_EINVAL, "out is NULL");
  *out = nullptr;
  GROUT_CHECK(validate_config(config));
  Mat embed, lm_head;
  std::vector<LayerW> layers;
  GROUT_CHECK(convert(embed, lm_head, layers));
  int ndev = 0;
  GROUT_CHECK(hip_status(hipGetDeviceCount(&ndev), "hipGetDeviceCount"));
  GROUT_NEED(device >= 0 && device < ndev, GROUT_EINVAL, "device %d of %d", device, ndev);
  grout_engine* e = new (std::nothrow) grout_engine();
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "out of host memory");
  const int rc = create_impl(e, config, norm, embed, lm_head, std::move(layers), device);
  if (rc != GROUT_OK) {
    const std::string msg = g_last_error;
    grout_engine_destroy(e);
    g_last_error = msg;
    return rc;
  }
  *out = e;
  return GROUT_OK;
}

}  // namespace

extern "C" {

int grout_engine_create(const grout_qwen3_config* config, const grout_qwen3_weights* weights,
                        int device, grout_engine** out) {
  const void* norm = weights ? weights->norm : nullptr;
  return create_common(config, norm, device, out, [&](Mat& em, Mat& lm, std::vector<LayerW>& ls) {
    return convert_f16(config, weights, em, lm, ls);
  });
}

int grout_engine_create_q(const grout_qwen3_config* config, const grout_qwen3_qweights* weights,
                          int device, grout_engine** out) {
  const void* norm = weights ? weights->norm : nullptr;
  return create_common(config, norm, device, out, [&](Mat& em, Mat& lm, std::vector<LayerW>& ls) {
    return convert_q(config, weights, em, lm, ls);
  });
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
  e->dev_token = -1;  // the prefill's head writes the token word
  e->dev_pos = -1;
  GROUT_CHECK(ensure_prefill_capacity(e, n));
  const PrefillBufs& b = e->pb;
  hipStream_t s = e->stream;
  GROUT_CHECK(hip_status(hipMemcpyAsync(e->p(b.ids), tokens, (size_t)n * sizeof(uint32_t),
                                        hipMemcpyHostToDevice, s),
                         "tokens H2D"));
  GROUT_CHECK(embed_rows(e, e->p<uint32_t>(b.ids), e->p(b.hidden), n));
  const int H = c.hidden_size, I = c.intermediate_size;
  const int qd = e->q_dim, kd = e->kv_dim;
  const int qkvd = e->qkv_dim;
  uint16_t* const qkv = e->p<uint16_t>(b.qkv);
  for (int l = 0; l < c.num_layers; ++l) {
    const LayerW& w = e->layers[l];
    if (l == 0)
      GROUT_CHECK(norm(e, nullptr, e->p(b.hidden), w.input_norm, e->p(b.normed), nullptr, n));
    else
      GROUT_CHECK(norm(e, e->p(b.hidden_after_attn), e->p(b.ff_down), w.input_norm,
                       e->p(b.normed), e->p(b.hidden), n));
    // one projection per part into its columns of the fused [n][Q|K|V] rows
    // (one GEMM of 6144 columns measured 26-28 us at 512 tokens against 48 us
    // for separate Q, K and V GEMMs, Qwen3-4B)
    int row0 = 0;
    for (int i = 0; i < w.nqkv; ++i) {
      const Mat& m = w.qkv[i];
      const void* wf = nullptr;
      GROUT_CHECK(mat_f16(e, m, H, &wf));
      if (n == 1 && m.fmt == GROUT_WFMT_F16)
        GROUT_CHECK(hip_status(grout::launch_gemv(wf, e->p(b.normed), qkv + row0, m.rows, H, s),
                               "gemv"));
      else
        GROUT_CHECK(gemm_rows(e, wf, e->p(b.normed), qkv + row0, n, m.rows, H, qkvd));
      row0 += m.rows;
    }
    GROUT_CHECK(hip_status(
        grout::launch_qk_norm_rope_kv_prefill(
            qkv, qkv + qd, qkv + qd + kd, w.q_norm, w.k_norm, e->rope_cos(), e->rope_sin(),
            e->p(b.q_rope), e->k_cache(l), e->v_cache(l), pos0, n, c.num_q_heads,
            c.num_kv_heads, e->head_stride, c.max_ctx, c.rms_norm_eps, s, qkvd, qkvd),
        "qk_norm_rope_kv_prefill"));
    GROUT_CHECK(grout_fmha_prefill(e->p(b.q_rope), e->k_cache(l), e->v_cache(l),
                                   e->p(b.attn_out), n, pos0, c.num_q_heads, c.num_kv_heads, 128,
                                   e->head_stride, e->qk_scale, s));
    GROUT_CHECK(mat_project(e, w.o, e->p(b.attn_out), e->p(b.attn_proj), n, qd, H));
    GROUT_CHECK(norm(e, e->p(b.hidden), e->p(b.attn_proj), w.post_norm, e->p(b.ff_normed),
                     e->p(b.hidden_after_attn), n));
    row0 = 0;
    for (int i = 0; i < w.ngu; ++i) {
      GROUT_CHECK(mat_project(e, w.gu[i], e->p(b.ff_normed), e->p<uint16_t>(b.gate_up) + row0, n,
                              H, 2 * I));
      row0 += w.gu[i].rows;
    }
    GROUT_CHECK(hip_status(grout::launch_silu_mul(e->p(b.gate_up), e->p(b.ff), n, I, s),
                           "silu_mul"));
    GROUT_CHECK(mat_project(e, w.down, e->p(b.ff), e->p(b.ff_down), n, I, H));
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
  uint32_t greedy = 0;  // 4 more bytes in the same read-back
  GROUT_CHECK(copy_logits_out(e, logits_out, &greedy));
  e->dev_token = greedy;
  return GROUT_OK;
}

int grout_engine_decode_greedy(grout_engine* e, uint32_t token, uint32_t* next_token) {
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "engine is NULL");
  GROUT_NEED(next_token != nullptr, GROUT_EINVAL, "next_token is NULL");
  GROUT_CHECK(decode_common(e, token));
  GROUT_CHECK(copy_logits_out(e, nullptr, next_token));
  e->dev_token = *next_token;
  return GROUT_OK;
}

int grout_engine_reset(grout_engine* e) {
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "engine is NULL");
  e->next_pos = 0;
  e->session_active = false;
  e->dev_token = -1;
  e->dev_pos = -1;
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

int grout_engine_warmup(grout_engine* e) {
  GROUT_NEED(e != nullptr, GROUT_EINVAL, "engine is NULL");
  GROUT_CHECK(take_pending(e));
  // The model's first stop token, else 0 (src/api.rs:153-162).
  uint32_t token = 0;
  grout_model_info info{};
  if (e->owned_model && grout_model_get_info(e->owned_model, &info) == GROUT_OK &&
      info.num_eos > 0)
    token = info.eos_token_ids[0];
  GROUT_NEED(token < (uint32_t)e->cfg.vocab_size, GROUT_EINVAL,
             "warmup token %u >= vocab_size=%d", token, e->cfg.vocab_size);
  // One-token steps at positions 0 and 1 (src/model.rs:2204-2212): the
  // prefill path (library GEMMs, prefill kernels) and one decode-graph
  // replay, then the caches are zeroed and the session ends.
  int rc = run_chunk(e, &token, 1, 0, nullptr, nullptr);
  if (rc == GROUT_OK) rc = decode_common(e, token);
  if (rc == GROUT_OK) rc = copy_logits_out(e, nullptr, nullptr);
  const std::string first = g_last_error;
  const int rr = grout_engine_reset(e);
  if (rc != GROUT_OK) {
    g_last_error = first;
    return rc;
  }
  return rr;
}

int grout_engine_position(const grout_engine* e) { return e ? e->next_pos : -1; }

int grout_env_flag(const char* value, int default_value) {
  return parse_bool_or(value, default_value != 0) ? 1 : 0;
}

long grout_env_usize(const char* value, long default_value) {
  return parse_usize_or(value, default_value);
}

int grout_engine_num_splits(const grout_engine* e) { return e ? e->num_splits : -1; }

int grout_engine_vram_preflight(const grout_qwen3_config* c, size_t weight_bytes,
                                size_t scratch_bytes, size_t free_bytes, size_t total_bytes,
                                size_t* required) {
  GROUT_NEED(c != nullptr, GROUT_EINVAL, "config is NULL");
  GROUT_NEED(c->num_layers >= 1 && c->num_kv_heads >= 1 && c->max_ctx >= 1, GROUT_EINVAL,
             "num_layers=%d num_kv_heads=%d max_ctx=%d", c->num_layers, c->num_kv_heads,
             c->max_ctx);
  constexpr size_t kSlack = (size_t)700 << 20;  // src/model.rs:181
  const size_t kv_per_token = (size_t)c->num_layers * c->num_kv_heads * 128 * 2 * sizeof(uint16_t);
  const size_t kv = kv_per_token * (size_t)c->max_ctx;
  const size_t rope = (size_t)c->max_ctx * 128 * sizeof(float);
  const size_t need = weight_bytes + kv + rope + scratch_bytes + kSlack;
  if (required) *required = need;
  const double MiB = 1024.0 * 1024.0;
  char summary[400];
  std::snprintf(summary, sizeof(summary),
                "max_ctx=%d: weights=%.1f MiB + KV=%d tokens * %.1f KiB/token = %.1f MiB + "
                "rope=%.1f MiB + scratch=%.1f MiB + slack=%.1f MiB => required=%.1f MiB; "
                "free=%.1f MiB / total=%.1f MiB",
                c->max_ctx, weight_bytes / MiB, c->max_ctx, kv_per_token / 1024.0, kv / MiB,
                rope / MiB, scratch_bytes / MiB, kSlack / MiB, need / MiB, free_bytes / MiB,
                total_bytes / MiB);
  GROUT_NEED(need <= free_bytes, GROUT_ENOMEM, "VRAM preflight failed: %s", summary);
  return GROUT_OK;
}

int grout_engine_uses_decode_graph(const grout_engine* e) { return e && e->exec ? 1 : 0; }

const char* grout_engine_decode_graph_error(const grout_engine* e) {
  return e ? e->graph_error.c_str() : "";
}

int grout_engine_destroy(grout_engine* e) {
  if (!e) return GROUT_OK;
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  if (e->exec) (void)hipGraphExecDestroy(e->exec);
  if (e->graph) (void)hipGraphDestroy(e->graph);
  if (e->blas) (void)rocblas_destroy_handle(e->blas);
  if (e->pre.base) (void)hipFree(e->pre.base);
  if (e->deq) (void)hipFree(e->deq);
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
  GROUT_NEED(max_ctx >= 0 && max_ctx <= GROUT_MAX_CTX, GROUT_EINVAL,
             "max_ctx=%d outside [0, %d]", max_ctx, GROUT_MAX_CTX);
  // VRAM preflight with the model's weights before any of them is uploaded
  // (src/model.rs:1491-1506); create repeats it for the engine's own state.
  {
    grout_model_info pre{};
    GROUT_CHECK(grout_model_inspect(model_dir, &pre));
    grout_qwen3_config pc = pre.config;
    if (max_ctx > 0) pc.max_ctx = max_ctx;
    GROUT_NEED(pc.max_ctx >= 1 && pc.max_ctx <= GROUT_MAX_CTX, GROUT_ENOTSUP,
               "max_position_embeddings=%d exceeds GROUT_MAX_CTX=%d: pass a smaller max_ctx",
               pc.max_ctx, GROUT_MAX_CTX);
    int ndev = 0;
    GROUT_CHECK(hip_status(hipGetDeviceCount(&ndev), "hipGetDeviceCount"));
    GROUT_NEED(device >= 0 && device < ndev, GROUT_EINVAL, "device %d of %d", device, ndev);
    GROUT_CHECK(hip_status(hipSetDevice(device), "hipSetDevice"));
    size_t free_b = 0, total_b = 0;
    GROUT_CHECK(hip_status(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo"));
    GROUT_CHECK(grout_engine_vram_preflight(&pc, pre.weight_bytes, 0, free_b, total_b, nullptr));
  }
  grout_model* m = nullptr;
  GROUT_CHECK(grout_model_load(model_dir, device, &m));
  grout_model_info info;
  (void)grout_model_get_info(m, &info);
  grout_qwen3_config cfg = info.config;
  if (max_ctx > 0) cfg.max_ctx = max_ctx;
  grout_engine* e = nullptr;
  grout_qwen3_weights w;
  grout_qwen3_qweights qw;
  int rc;
  if (grout_model_weights(m, &w) == GROUT_OK) {
    rc = grout_engine_create(&cfg, &w, device, &e);
  } else {
    (void)grout_model_qweights(m, &qw);
    rc = grout_engine_create_q(&cfg, &qw, device, &e);
  }
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
