// C ABI of the gfx950 attention hot path: argument validation (the
// reference's `ensure!` checks before each launch), split selection, RoPE
// tables and the decode-step HIP graph runner.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "../../include/grout_attn.h"
#include "abi_util.hpp"
#include "kernels.hpp"

using namespace grout_abi;

extern "C" {

const char* grout_last_error(void) { return g_last_error.c_str(); }

int grout_abi_version(void) { return (1 << 16) | 1; }

int grout_rope_inv_freq(int head_dim, float theta, float* inv_freq) {
  GROUT_NEED(head_dim > 0 && head_dim % 2 == 0, GROUT_EINVAL, "head_dim=%d must be even",
             head_dim);
  GROUT_NEED(std::isfinite(theta) && theta > 0.f, GROUT_EINVAL, "rope theta=%g", (double)theta);
  GROUT_NEED(inv_freq != nullptr, GROUT_EINVAL, "inv_freq is NULL");
  for (int i = 0; i < head_dim; i += 2) {
    const float p = (float)i / (float)head_dim;
    inv_freq[i / 2] = 1.0f / powf(theta, p);
  }
  return GROUT_OK;
}

int grout_rope_table_host(int max_ctx, int head_dim, float theta, float* cos_out,
                          float* sin_out) {
  GROUT_NEED(max_ctx > 0, GROUT_EINVAL, "max_ctx=%d", max_ctx);
  GROUT_NEED(cos_out != nullptr && sin_out != nullptr, GROUT_EINVAL, "table pointer is NULL");
  const int half = head_dim / 2;
  float inv[512];
  GROUT_NEED(half <= 512, GROUT_ENOTSUP, "head_dim=%d too large", head_dim);
  GROUT_CHECK(grout_rope_inv_freq(head_dim, theta, inv));
  for (int p = 0; p < max_ctx; ++p) {
    const float pf = (float)p;
    for (int i = 0; i < half; ++i) {
      const float ang = pf * inv[i];
      cos_out[(size_t)p * half + i] = (float)std::cos((double)ang);
      sin_out[(size_t)p * half + i] = (float)std::sin((double)ang);
    }
  }
  return GROUT_OK;
}

int grout_qk_norm_rope_kv_prefill(const void* q, const void* k, const void* v,
                                  const void* gamma_q, const void* gamma_k,
                                  const float* rope_cos, const float* rope_sin, void* q_out,
                                  void* k_cache, void* v_cache, int pos0, int seq_len,
                                  int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                                  long kv_head_stride, float eps, void* stream) {
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, head_dim, 1 << 20));
  GROUT_NEED(seq_len >= 1, GROUT_EINVAL, "prefill requires at least one token");
  GROUT_NEED(pos0 >= 0 && (long)pos0 + seq_len <= max_ctx, GROUT_EINVAL,
             "fused qk/rope/kv range [%d..%ld) exceeds max_seq_len %d", pos0,
             (long)pos0 + seq_len, max_ctx);
  GROUT_NEED(std::isfinite(eps) && eps > 0.f, GROUT_EINVAL, "rms_norm_eps=%g must be positive",
             (double)eps);
  GROUT_CHECK(check_ptrs16({{q, "q"}, {k, "k"}, {v, "v"}, {gamma_q, "gamma_q"},
                            {gamma_k, "gamma_k"}, {rope_cos, "rope_cos"},
                            {rope_sin, "rope_sin"}, {q_out, "q_out"}, {k_cache, "k_cache"},
                            {v_cache, "v_cache"}}));
  GROUT_CHECK(check_stride(kv_head_stride, max_ctx));
  return hip_status(grout::launch_qk_norm_rope_kv_prefill(
                        q, k, v, gamma_q, gamma_k, rope_cos, rope_sin, q_out, k_cache, v_cache,
                        pos0, seq_len, num_q_heads, num_kv_heads, kv_head_stride, max_ctx, eps,
                        as_stream(stream)),
                    "qk_norm_rope_kv_prefill launch");
}

int grout_qk_norm_rope_kv_decode(const void* qkv, const void* gamma_q, const void* gamma_k,
                                 const float* rope_cos, const float* rope_sin, void* q_out,
                                 void* k_cache, void* v_cache, const uint32_t* d_pos,
                                 int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                                 long kv_head_stride, float eps, void* stream) {
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, head_dim, 1 << 20));
  GROUT_NEED(max_ctx >= 1, GROUT_EINVAL, "max_ctx=%d", max_ctx);
  GROUT_NEED(std::isfinite(eps) && eps > 0.f, GROUT_EINVAL, "rms_norm_eps=%g must be positive",
             (double)eps);
  GROUT_NEED(d_pos != nullptr, GROUT_EINVAL, "d_pos is NULL");
  GROUT_CHECK(check_ptrs16({{qkv, "qkv"}, {gamma_q, "gamma_q"}, {gamma_k, "gamma_k"},
                            {rope_cos, "rope_cos"}, {rope_sin, "rope_sin"}, {q_out, "q_out"},
                            {k_cache, "k_cache"}, {v_cache, "v_cache"}}));
  GROUT_CHECK(check_stride(kv_head_stride, max_ctx));
  return hip_status(grout::launch_qk_norm_rope_kv_decode(
                        qkv, gamma_q, gamma_k, rope_cos, rope_sin, q_out, k_cache, v_cache,
                        d_pos, num_q_heads, num_kv_heads, kv_head_stride, max_ctx, eps,
                        as_stream(stream)),
                    "qk_norm_rope_kv_decode launch");
}

int grout_fmha_prefill(const void* q, const void* k_cache, const void* v_cache, void* out,
                       int seq_len, int pos0, int num_q_heads, int num_kv_heads, int head_dim,
                       long kv_head_stride, float qk_scale, void* stream) {
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, head_dim, 1 << 20));
  GROUT_NEED(seq_len >= 1, GROUT_EINVAL, "attention requires q_len >= 1");
  GROUT_NEED(pos0 >= 0, GROUT_EINVAL, "pos0=%d", pos0);
  GROUT_NEED(std::isfinite(qk_scale) && qk_scale > 0.f, GROUT_EINVAL, "qk_scale=%g",
             (double)qk_scale);
  GROUT_CHECK(check_ptrs16({{q, "q"}, {k_cache, "k_cache"}, {v_cache, "v_cache"}, {out, "out"}}));
  GROUT_CHECK(check_stride(kv_head_stride, (long)pos0 + seq_len));
  return hip_status(grout::launch_fmha_prefill(q, k_cache, v_cache, out, seq_len, pos0,
                                               num_q_heads, num_kv_heads, kv_head_stride,
                                               qk_scale, as_stream(stream)),
                    "fmha_prefill launch");
}

int grout_fmha_prefill_plan(int seq_len, int num_q_heads, int num_kv_heads, int* form,
                            int* paired, long* workgroups) {
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, 128, 1 << 20));
  GROUT_NEED(seq_len >= 1 && seq_len <= GROUT_MAX_CTX, GROUT_EINVAL,
             "seq_len=%d outside [1, GROUT_MAX_CTX=%d]", seq_len, GROUT_MAX_CTX);
  const grout::PrefillPlan p = grout::plan_fmha_prefill(seq_len, num_q_heads, num_kv_heads);
  if (form) *form = p.shared ? 0 : p.wave_rows == 32 ? 1 : 2;
  if (paired) *paired = p.paired;
  if (workgroups) *workgroups = p.workgroups;
  return GROUT_OK;
}

int grout_attn_decode_default_splits(int ctx_len, int num_q_heads, int num_kv_heads) {
  if (ctx_len < 1 || num_kv_heads < 1) return 1;
  (void)num_q_heads;
  const int tiles = (ctx_len + 31) / 32;
  // Up to 128 positions: one split (one workgroup per kv head, no merge
  // launch).  Beyond: one 32-position tile per split, capped at one
  // workgroup per CU over the 256 CUs (measured best on MI355X for 4k..32k;
  // more splits only add merge work).  At 512..1024 positions 16-32 splits
  // measured 0.4-0.6 us per layer faster than 8 (Qwen3-4B shapes).
  if (tiles <= 4) return 1;
  int by_work = tiles;
  int by_grid = (256 + num_kv_heads - 1) / num_kv_heads;
  int n = by_work < by_grid ? by_work : by_grid;
  if (n < 1) n = 1;
  if (n > kMaxSplits) n = kMaxSplits;
  return n;
}

size_t grout_attn_decode_workspace_bytes(int num_q_heads, int num_kv_heads, int head_dim,
                                         int num_splits) {
  if (head_dim != 128 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      num_splits <= 0)
    return 0;
  return decode_ws_bytes(num_q_heads, num_kv_heads, num_splits);
}

int grout_fmha_decode_gqa_split(const void* q, const void* k_cache, const void* v_cache,
                                float* part_acc, float* part_ml, const uint32_t* d_pos,
                                int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                                long kv_head_stride, int num_splits, float qk_scale,
                                void* stream) {
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, head_dim, kMaxDecodeGroup));
  GROUT_NEED(max_ctx >= 1, GROUT_EINVAL, "max_ctx=%d", max_ctx);
  GROUT_NEED(num_splits >= 1 && num_splits <= kMaxSplits, GROUT_EINVAL,
             "num_splits=%d outside [1, %d]", num_splits, kMaxSplits);
  GROUT_NEED(std::isfinite(qk_scale) && qk_scale > 0.f, GROUT_EINVAL, "qk_scale=%g",
             (double)qk_scale);
  GROUT_NEED(d_pos != nullptr, GROUT_EINVAL, "d_pos is NULL");
  GROUT_CHECK(check_ptrs16({{q, "q"}, {k_cache, "k_cache"}, {v_cache, "v_cache"},
                            {part_acc, "part_acc"}, {part_ml, "part_ml"}}));
  GROUT_CHECK(check_stride(kv_head_stride, max_ctx));
  return hip_status(grout::launch_attn_decode_split(q, k_cache, v_cache, kv_head_stride, d_pos,
                                                    max_ctx, num_q_heads, num_kv_heads,
                                                    num_splits, qk_scale, part_acc, part_ml,
                                                    as_stream(stream)),
                    "fmha_decode_gqa_split launch");
}

int grout_splitk_reduce_merge(const float* part_acc, const float* part_ml, void* out,
                              int num_q_heads, int num_kv_heads, int head_dim, int num_splits,
                              void* stream) {
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, head_dim, kMaxDecodeGroup));
  GROUT_NEED(num_splits >= 1 && num_splits <= kMaxSplits, GROUT_EINVAL,
             "num_splits=%d outside [1, %d]", num_splits, kMaxSplits);
  GROUT_CHECK(check_ptrs16({{part_acc, "part_acc"}, {part_ml, "part_ml"}, {out, "out"}}));
  return hip_status(grout::launch_attn_decode_merge(part_acc, part_ml, out, num_q_heads,
                                                    num_kv_heads, num_splits,
                                                    as_stream(stream)),
                    "splitk_reduce_merge launch");
}

int grout_attn_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
                      void* workspace, size_t workspace_bytes, const uint32_t* d_pos,
                      int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                      long kv_head_stride, int num_splits, float qk_scale, void* stream) {
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, head_dim, kMaxDecodeGroup));
  if (num_splits <= 0) num_splits = grout_attn_decode_default_splits(max_ctx, num_q_heads, num_kv_heads);
  GROUT_NEED(num_splits <= kMaxSplits, GROUT_EINVAL, "num_splits=%d > %d", num_splits, kMaxSplits);
  GROUT_NEED(max_ctx >= 1, GROUT_EINVAL, "max_ctx=%d", max_ctx);
  GROUT_NEED(std::isfinite(qk_scale) && qk_scale > 0.f, GROUT_EINVAL, "qk_scale=%g",
             (double)qk_scale);
  GROUT_NEED(d_pos != nullptr, GROUT_EINVAL, "d_pos is NULL");
  const size_t need = decode_ws_bytes(num_q_heads, num_kv_heads, num_splits);
  GROUT_NEED(workspace != nullptr && workspace_bytes >= need, GROUT_EINVAL,
             "workspace of %zu bytes < %zu needed for %d splits", workspace_bytes, need,
             num_splits);
  GROUT_CHECK(check_ptrs16({{q, "q"}, {k_cache, "k_cache"}, {v_cache, "v_cache"}, {out, "out"},
                            {workspace, "workspace"}}));
  GROUT_CHECK(check_stride(kv_head_stride, max_ctx));
  float* part_acc = static_cast<float*>(workspace);
  const size_t G = (size_t)(num_q_heads / num_kv_heads);
  float* part_ml = part_acc + (size_t)num_kv_heads * num_splits * G * 128;
  GROUT_CHECK(hip_status(grout::launch_attn_decode_split(q, k_cache, v_cache, kv_head_stride,
                                                         d_pos, max_ctx, num_q_heads, num_kv_heads,
                                                         num_splits, qk_scale, part_acc, part_ml,
                                                         as_stream(stream)),
                         "attn_decode split launch"));
  return hip_status(grout::launch_attn_decode_merge(part_acc, part_ml, out, num_q_heads,
                                                    num_kv_heads, num_splits, as_stream(stream)),
                    "attn_decode merge launch");
}

}  // extern "C"

// grout_attn_decode_fused, plus the captured decode graph's option of having
// the merge of its last layer move the position word on (advance_pos).
static int attn_decode_fused_impl(const void* qkv, const void* gamma_q, const void* gamma_k,
                                  const float* rope_cos, const float* rope_sin, void* k_cache,
                                  void* v_cache, void* out, void* workspace,
                                  size_t workspace_bytes, const uint32_t* d_pos,
                                  int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                                  long kv_head_stride, int num_splits, float eps, float qk_scale,
                                  void* stream, uint32_t* advance_pos) {
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, head_dim, kMaxDecodeGroup));
  if (num_splits <= 0) num_splits = grout_attn_decode_default_splits(max_ctx, num_q_heads, num_kv_heads);
  GROUT_NEED(num_splits <= kMaxSplits, GROUT_EINVAL, "num_splits=%d > %d", num_splits, kMaxSplits);
  GROUT_NEED(max_ctx >= 1, GROUT_EINVAL, "max_ctx=%d", max_ctx);
  GROUT_NEED(std::isfinite(eps) && eps > 0.f, GROUT_EINVAL, "eps=%g", (double)eps);
  GROUT_NEED(std::isfinite(qk_scale) && qk_scale > 0.f, GROUT_EINVAL, "qk_scale=%g",
             (double)qk_scale);
  GROUT_NEED(d_pos != nullptr && rope_cos != nullptr && rope_sin != nullptr, GROUT_EINVAL,
             "d_pos or a rope table is NULL");
  GROUT_CHECK(check_ptrs16({{qkv, "qkv"}, {gamma_q, "gamma_q"}, {gamma_k, "gamma_k"},
                            {k_cache, "k_cache"}, {v_cache, "v_cache"}, {out, "out"}}));
  GROUT_CHECK(check_stride(kv_head_stride, max_ctx));
  float* part_acc = nullptr;
  float* part_ml = nullptr;
  if (num_splits > 1) {
    const size_t need = decode_ws_bytes(num_q_heads, num_kv_heads, num_splits);
    GROUT_NEED(workspace != nullptr && workspace_bytes >= need, GROUT_EINVAL,
               "workspace of %zu bytes < %zu needed for %d splits", workspace_bytes, need,
               num_splits);
    GROUT_CHECK(check_ptrs16({{workspace, "workspace"}}));
    part_acc = static_cast<float*>(workspace);
    part_ml = part_acc + (size_t)num_kv_heads * num_splits * (num_q_heads / num_kv_heads) * 128;
  }
  return hip_status(grout::launch_attn_decode_fused(qkv, gamma_q, gamma_k, rope_cos, rope_sin,
                                                    k_cache, v_cache, kv_head_stride, d_pos,
                                                    max_ctx, num_q_heads, num_kv_heads,
                                                    num_splits, eps, qk_scale, part_acc, part_ml,
                                                    out, as_stream(stream), advance_pos),
                    "attn_decode_fused launch");
}

extern "C" {

int grout_attn_decode_fused(const void* qkv, const void* gamma_q, const void* gamma_k,
                            const float* rope_cos, const float* rope_sin, void* k_cache,
                            void* v_cache, void* out, void* workspace, size_t workspace_bytes,
                            const uint32_t* d_pos, int num_q_heads, int num_kv_heads,
                            int head_dim, int max_ctx, long kv_head_stride, int num_splits,
                            float eps, float qk_scale, void* stream) {
  return attn_decode_fused_impl(qkv, gamma_q, gamma_k, rope_cos, rope_sin, k_cache, v_cache, out,
                                workspace, workspace_bytes, d_pos, num_q_heads, num_kv_heads,
                                head_dim, max_ctx, kv_head_stride, num_splits, eps, qk_scale,
                                stream, nullptr);
}

}  // extern "C"

// ------------------------------------------------------- no-allocation decode
//
// grout_attn_decode_noalloc keeps the split partials in this file-scope
// device array instead of a caller workspace.  In host code `scratch` only
// names the symbol: its device address (one per GPU) comes from
// hipGetSymbolAddress, looked up once per device with that device current,
// and only that address is passed to kernels.
namespace {

static __device__ __align__(256) unsigned char scratch[GROUT_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` belongs to.
int noalloc_scratch(hipStream_t stream, void** out) {
  int cur = 0;
  GROUT_CHECK(hip_status(hipGetDevice(&cur), "hipGetDevice"));
  int dev = cur;
  if (stream != nullptr) GROUT_CHECK(hip_status(hipStreamGetDevice(stream, &dev), "hipStreamGetDevice"));
  GROUT_NEED(dev >= 0 && dev < kMaxDevices, GROUT_ENOTSUP, "device %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    if (dev != cur) GROUT_CHECK(hip_status(hipSetDevice(dev), "hipSetDevice"));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    GROUT_CHECK(hip_status(e, "hipGetSymbolAddress(scratch)"));
    GROUT_NEED(p != nullptr, GROUT_EINVAL, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return GROUT_OK;
}

}  // namespace

extern "C" {

int grout_attn_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, void* out,
                              const uint32_t* d_pos, int num_q_heads, int num_kv_heads,
                              int head_dim, int max_ctx, long kv_head_stride, int num_splits,
                              float qk_scale, void* stream) {
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, head_dim, kMaxDecodeGroup));
  if (num_splits <= 0) num_splits = grout_attn_decode_default_splits(max_ctx, num_q_heads, num_kv_heads);
  GROUT_NEED(num_splits <= kMaxSplits, GROUT_EINVAL, "num_splits=%d > %d", num_splits, kMaxSplits);
  GROUT_NEED(max_ctx >= 1, GROUT_EINVAL, "max_ctx=%d", max_ctx);
  GROUT_NEED(std::isfinite(qk_scale) && qk_scale > 0.f, GROUT_EINVAL, "qk_scale=%g",
             (double)qk_scale);
  GROUT_NEED(d_pos != nullptr, GROUT_EINVAL, "d_pos is NULL");
  const size_t need = decode_ws_bytes(num_q_heads, num_kv_heads, num_splits);
  GROUT_NEED(need <= (size_t)GROUT_NOALLOC_SCRATCH_BYTES, GROUT_EINVAL,
             "%d splits need %zu bytes of scratch, more than the %d-byte static scratch of "
             "grout_attn_decode_noalloc (use fewer splits, or grout_attn_decode)",
             num_splits, need, GROUT_NOALLOC_SCRATCH_BYTES);
  GROUT_CHECK(check_ptrs16({{q, "q"}, {k_cache, "k_cache"}, {v_cache, "v_cache"}, {out, "out"}}));
  GROUT_CHECK(check_stride(kv_head_stride, max_ctx));
  void* ws = nullptr;
  GROUT_CHECK(noalloc_scratch(as_stream(stream), &ws));
  // Every split workgroup writes all of its partials (empty splits write a
  // zero sum), so the merge never reads a value left by an earlier call.
  float* part_acc = static_cast<float*>(ws);
  const size_t G = (size_t)(num_q_heads / num_kv_heads);
  float* part_ml = part_acc + (size_t)num_kv_heads * num_splits * G * 128;
  GROUT_CHECK(hip_status(grout::launch_attn_decode_split(q, k_cache, v_cache, kv_head_stride,
                                                         d_pos, max_ctx, num_q_heads, num_kv_heads,
                                                         num_splits, qk_scale, part_acc, part_ml,
                                                         as_stream(stream)),
                         "attn_decode_noalloc split launch"));
  return hip_status(grout::launch_attn_decode_merge(part_acc, part_ml, out, num_q_heads,
                                                    num_kv_heads, num_splits, as_stream(stream)),
                    "attn_decode_noalloc merge launch");
}

// ------------------------------------------------------------------ graph

struct grout_decode_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  uint32_t* d_pos = nullptr;
  int max_ctx = 0;
  // The last layer's merge leaves position + 1 in d_pos (split count > 1):
  // a launch at that position needs no write of its own.  -1: unknown.
  bool advances = false;
  long next_pos = -1;
};

}  // extern "C"

namespace {
__global__ void set_position_kernel(uint32_t* d_pos, uint32_t value) { *d_pos = value; }
}  // namespace

extern "C" {

int grout_decode_graph_create(const grout_decode_layer* layers, int num_layers,
                              const float* rope_cos, const float* rope_sin, void* workspace,
                              size_t workspace_bytes, int num_q_heads, int num_kv_heads,
                              int head_dim, int max_ctx, int num_splits, float eps,
                              float qk_scale, void* stream, grout_decode_graph** out) {
  GROUT_NEED(out != nullptr, GROUT_EINVAL, "out is NULL");
  *out = nullptr;
  GROUT_NEED(layers != nullptr && num_layers >= 1, GROUT_EINVAL, "num_layers=%d", num_layers);
  GROUT_CHECK(check_heads(num_q_heads, num_kv_heads, head_dim, kMaxDecodeGroup));
  GROUT_NEED(max_ctx >= 1, GROUT_EINVAL, "max_ctx=%d", max_ctx);
  if (num_splits <= 0) num_splits = grout_attn_decode_default_splits(max_ctx, num_q_heads, num_kv_heads);
  const long stride = (long)max_ctx * 128;
  // Validate every layer up front so a failed capture never leaves a half-built graph.
  for (int i = 0; i < num_layers; ++i) {
    const grout_decode_layer& L = layers[i];
    const int rc = check_ptrs16({{L.qkv, "qkv"}, {L.gamma_q, "gamma_q"}, {L.gamma_k, "gamma_k"},
                                 {L.k_cache, "k_cache"}, {L.v_cache, "v_cache"},
                                 {L.attn_out, "attn_out"}});
    if (rc != GROUT_OK) return fail(rc, "layer %d: %s", i, g_last_error.c_str());
  }
  const size_t need = decode_ws_bytes(num_q_heads, num_kv_heads, num_splits);
  GROUT_NEED(workspace != nullptr && workspace_bytes >= need, GROUT_EINVAL,
             "workspace of %zu bytes < %zu needed", workspace_bytes, need);

  grout_decode_graph* g = new (std::nothrow) grout_decode_graph();
  GROUT_NEED(g != nullptr, GROUT_EINVAL, "out of host memory");
  g->max_ctx = max_ctx;
  // Capture on the caller's stream; the legacy NULL stream cannot be
  // captured, so a NULL stream gets a private one for the capture only.
  hipStream_t cap = as_stream(stream);
  hipStream_t own = nullptr;
  int rc = hip_status(hipMalloc(&g->d_pos, sizeof(uint32_t)), "hipMalloc(position)");
  if (rc == GROUT_OK) rc = hip_status(hipMemset(g->d_pos, 0, sizeof(uint32_t)), "hipMemset(position)");
  if (rc == GROUT_OK && cap == nullptr) {
    rc = hip_status(hipStreamCreateWithFlags(&own, hipStreamNonBlocking), "hipStreamCreate");
    cap = own;
  }
  if (rc == GROUT_OK) {
    rc = hip_status(hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal), "BeginCapture");
    if (rc == GROUT_OK) {
      // Per layer: the fused norm/RoPE/KV write + split-K pass, then the
      // merge; the last merge moves the position word on to the next step's.
      g->advances = num_splits > 1;
      for (int i = 0; i < num_layers && rc == GROUT_OK; ++i) {
        const grout_decode_layer& L = layers[i];
        rc = attn_decode_fused_impl(L.qkv, L.gamma_q, L.gamma_k, rope_cos, rope_sin, L.k_cache,
                                    L.v_cache, L.attn_out, workspace, workspace_bytes, g->d_pos,
                                    num_q_heads, num_kv_heads, head_dim, max_ctx, stride,
                                    num_splits, eps, qk_scale, cap,
                                    i + 1 == num_layers && g->advances ? g->d_pos : nullptr);
      }
      hipGraph_t graph = nullptr;
      const hipError_t e = hipStreamEndCapture(cap, &graph);
      if (rc == GROUT_OK) rc = hip_status(e, "EndCapture");
      g->graph = graph;
    }
  }
  if (rc == GROUT_OK)
    rc = hip_status(hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0),
                    "hipGraphInstantiate");
  if (own) (void)hipStreamDestroy(own);
  if (rc != GROUT_OK) {
    const std::string msg = g_last_error;
    grout_decode_graph_destroy(g);
    g_last_error = msg;
    return rc;
  }
  *out = g;
  return GROUT_OK;
}

int grout_decode_graph_launch(grout_decode_graph* graph, uint32_t position, void* stream) {
  GROUT_NEED(graph != nullptr && graph->exec != nullptr, GROUT_EINVAL, "graph is NULL");
  GROUT_NEED((long)position < (long)graph->max_ctx, GROUT_EINVAL,
             "decode position %u exceeds max_ctx=%d", position, graph->max_ctx);
  // Consecutive steps (position = the previous launch's + 1) find the word
  // already moved on by the previous replay: one hipGraphLaunch per step.
  // Any other position is written first by a one-thread kernel whose
  // argument carries it, so queued launches never race on a host staging
  // buffer.
  if (!(graph->advances && (long)position == graph->next_pos)) {
    graph->next_pos = -1;
    set_position_kernel<<<1, 1, 0, as_stream(stream)>>>(graph->d_pos, position);
    GROUT_CHECK(hip_status(hipGetLastError(), "set position"));
  }
  graph->next_pos = -1;
  GROUT_CHECK(hip_status(hipGraphLaunch(graph->exec, as_stream(stream)), "hipGraphLaunch"));
  graph->next_pos = (long)position + 1;
  return GROUT_OK;
}

const uint32_t* grout_decode_graph_position_ptr(const grout_decode_graph* graph) {
  return graph ? graph->d_pos : nullptr;
}

int grout_decode_graph_destroy(grout_decode_graph* graph) {
  if (!graph) return GROUT_OK;
  if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
  if (graph->graph) (void)hipGraphDestroy(graph->graph);
  if (graph->d_pos) (void)hipFree(graph->d_pos);
  delete graph;
  return GROUT_OK;
}

int grout_diag_mfma_layout(float* out, void* stream) {
  GROUT_NEED(out != nullptr, GROUT_EINVAL, "out is NULL");
  return hip_status(grout::launch_mfma_layout_probe(out, as_stream(stream)), "mfma probe");
}

}  // extern "C"
