// Qwen3 checkpoint loader: config.json + safetensors shards (mmapped) ->
// fp16 device weights in the engine's fused layouts.
//
// Reference: Loader (src/loader.rs:24-171, cast_to_f16 702-740), the
// per-layer weight assembly of Qwen3Engine::load (src/model.rs:1508-1600:
// q/k/v rows concatenated into qkv_proj, gate/up into gate_up_proj, lm_head =
// embed_tokens when tie_word_embeddings), Qwen3Config / GenerationConfig
// (src/config.rs:7-160, with its range checks).  Same rules: shard names from
// the index must be plain file names; bf16, f32 and f64 tensors become f16
// through f32 (round to nearest even).  The conversion runs on the GPU, one
// tensor at a time through a staging buffer, straight into the fused device
// buffers; every tensor's dtype, shape and byte range is validated against the
// config before anything is allocated on the device.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "../../include/grout_attn.h"
#include "../../include/grout_engine.h"
#include "abi_util.hpp"
#include "json.hpp"
#include "kernels.hpp"
#include "model_internal.hpp"

using namespace grout_abi;

namespace {

using grout_json::Value;

struct Mapped {
  void* p = nullptr;
  size_t n = 0;
  ~Mapped() {
    if (p) munmap(p, n);
  }
};

int read_file(const std::string& path, std::string& out) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) return fail(GROUT_EINVAL, "cannot open %s", path.c_str());
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size > (64 << 20)) {
    ::close(fd);
    return fail(GROUT_EINVAL, "%s: unreadable or larger than 64 MiB", path.c_str());
  }
  out.resize((size_t)st.st_size);
  size_t got = 0;
  while (got < out.size()) {
    const ssize_t r = ::read(fd, &out[got], out.size() - got);
    if (r <= 0) break;
    got += (size_t)r;
  }
  ::close(fd);
  if (got != out.size()) return fail(GROUT_EINVAL, "short read of %s", path.c_str());
  return GROUT_OK;
}

int parse_json_file(const std::string& path, Value& v) {
  std::string text;
  GROUT_CHECK(read_file(path, text));
  grout_json::Parser p(text.data(), text.size());
  if (!p.parse(v)) return fail(GROUT_EINVAL, "%s: %s", path.c_str(), p.error().c_str());
  return GROUT_OK;
}

bool file_exists(const std::string& path) {
  struct stat st;
  return ::stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

int get_uint(const Value& o, const char* key, long max, long* out, const char* file) {
  const Value* v = o.get(key);
  if (!v || v->kind != Value::kNumber || !v->is_int)
    return fail(GROUT_EINVAL, "%s: integer field %s missing or not an integer", file, key);
  if (v->i < 1 || v->i > max)
    return fail(GROUT_EINVAL, "%s: config %s=%lld out of range [1, %ld]", file, key,
                (long long)v->i, max);
  *out = (long)v->i;
  return GROUT_OK;
}

int get_float(const Value& o, const char* key, float* out, const char* file) {
  const Value* v = o.get(key);
  if (!v || v->kind != Value::kNumber)
    return fail(GROUT_EINVAL, "%s: number field %s missing", file, key);
  const float f = (float)v->num;
  if (!std::isfinite(f) || f <= 0.f)
    return fail(GROUT_EINVAL, "%s: %s=%g must be a positive finite float", file, key, v->num);
  *out = f;
  return GROUT_OK;
}

int get_bool(const Value& o, const char* key, bool* out, const char* file) {
  const Value* v = o.get(key);
  if (!v || v->kind != Value::kBool) return fail(GROUT_EINVAL, "%s: bool field %s missing", file, key);
  *out = v->b;
  return GROUT_OK;
}

// src/config.rs:44-95 (range checks) and src/model.rs:1443-1446 (no sliding
// window, head_dim 128).
int parse_config(const std::string& dir, grout_model_info* info) {
  const std::string path = dir + "/config.json";
  Value cfg;
  GROUT_CHECK(parse_json_file(path, cfg));
  if (cfg.kind != Value::kObject) return fail(GROUT_EINVAL, "%s: not a JSON object", path.c_str());
  const char* f = path.c_str();
  long vocab, hidden, inter, layers, hq, hkv, hd, maxpos;
  GROUT_CHECK(get_uint(cfg, "vocab_size", 1L << 24, &vocab, f));
  GROUT_CHECK(get_uint(cfg, "hidden_size", 1L << 20, &hidden, f));
  GROUT_CHECK(get_uint(cfg, "intermediate_size", 1L << 22, &inter, f));
  GROUT_CHECK(get_uint(cfg, "num_hidden_layers", 1L << 12, &layers, f));
  GROUT_CHECK(get_uint(cfg, "num_attention_heads", 1L << 12, &hq, f));
  GROUT_CHECK(get_uint(cfg, "num_key_value_heads", 1L << 12, &hkv, f));
  GROUT_CHECK(get_uint(cfg, "head_dim", 1L << 12, &hd, f));
  GROUT_CHECK(get_uint(cfg, "max_position_embeddings", 1L << 25, &maxpos, f));
  float eps, theta;
  GROUT_CHECK(get_float(cfg, "rms_norm_eps", &eps, f));
  GROUT_CHECK(get_float(cfg, "rope_theta", &theta, f));
  bool tie, sliding;
  GROUT_CHECK(get_bool(cfg, "tie_word_embeddings", &tie, f));
  GROUT_CHECK(get_bool(cfg, "use_sliding_window", &sliding, f));
  GROUT_NEED(!sliding, GROUT_ENOTSUP, "%s: use_sliding_window is not supported", f);
  GROUT_NEED(hq % hkv == 0, GROUT_EINVAL, "%s: num_attention_heads=%ld not divisible by %ld", f,
             hq, hkv);
  GROUT_NEED(hd == 128, GROUT_ENOTSUP, "%s: head_dim=%ld: only 128 is supported", f, hd);
  const Value* eos = cfg.get("eos_token_id");
  GROUT_NEED(eos && eos->kind == Value::kNumber && eos->is_int && eos->i >= 0 &&
                 eos->i <= 0xffffffffLL,
             GROUT_EINVAL, "%s: eos_token_id missing or not a u32", f);

  std::memset(info, 0, sizeof(*info));
  grout_qwen3_config& c = info->config;
  c.num_layers = (int)layers;
  c.hidden_size = (int)hidden;
  c.intermediate_size = (int)inter;
  c.num_q_heads = (int)hq;
  c.num_kv_heads = (int)hkv;
  c.head_dim = (int)hd;
  c.vocab_size = (int)vocab;
  c.rms_norm_eps = eps;
  c.rope_theta = theta;
  c.max_ctx = (int)maxpos;
  info->tie_word_embeddings = tie ? 1 : 0;
  info->num_eos = 1;
  info->eos_token_ids[0] = (uint32_t)eos->i;
  // generation_config.json, when present, lists the stop tokens
  // (src/config.rs:97-160).
  const std::string gpath = dir + "/generation_config.json";
  if (file_exists(gpath)) {
    Value g;
    GROUT_CHECK(parse_json_file(gpath, g));
    const Value* ge = g.get("eos_token_id");
    if (ge && ge->kind == Value::kNumber && ge->is_int && ge->i >= 0 && ge->i <= 0xffffffffLL) {
      info->eos_token_ids[0] = (uint32_t)ge->i;
    } else if (ge && ge->kind == Value::kArray && !ge->arr.empty()) {
      int n = 0;
      for (const Value& e : ge->arr) {
        GROUT_NEED(e.kind == Value::kNumber && e.is_int && e.i >= 0 && e.i <= 0xffffffffLL,
                   GROUT_EINVAL, "%s: eos_token_id entries must be u32", gpath.c_str());
        if (n < GROUT_MAX_EOS) info->eos_token_ids[n++] = (uint32_t)e.i;
      }
      info->num_eos = n;
    }
  }
  return GROUT_OK;
}

enum Dtype { kF16 = 0, kBF16 = 1, kF32 = 2, kF64 = 3 };

int dtype_of(const std::string& s, int* d, size_t* size) {
  if (s == "F16") { *d = kF16; *size = 2; return GROUT_OK; }
  if (s == "BF16") { *d = kBF16; *size = 2; return GROUT_OK; }
  if (s == "F32") { *d = kF32; *size = 4; return GROUT_OK; }
  if (s == "F64") { *d = kF64; *size = 8; return GROUT_OK; }
  return fail(GROUT_ENOTSUP, "unsupported dtype for fp16 cast: %s", s.c_str());
}

struct TensorRef {
  int dtype = 0;
  size_t elem = 0;
  std::vector<int64_t> shape;
  const unsigned char* data = nullptr;
  size_t bytes = 0;
};

struct Checkpoint {
  std::string dir;
  grout_model_info info{};
  std::map<std::string, std::unique_ptr<Mapped>> shards;
  std::map<std::string, TensorRef> tensors;
  size_t max_raw = 0;  // largest non-f16 tensor, for the staging buffer

  int map_shard(const std::string& name) {
    if (shards.count(name)) return GROUT_OK;
    // Names come from an untrusted index: plain file names only
    // (src/loader.rs:53-66).
    GROUT_NEED(!name.empty() && name != "." && name != ".." &&
                   name.find('/') == std::string::npos && name.find('\\') == std::string::npos,
               GROUT_EINVAL, "shard `%s` must be a plain file name", name.c_str());
    const std::string path = dir + "/" + name;
    const int fd = ::open(path.c_str(), O_RDONLY);
    GROUT_NEED(fd >= 0, GROUT_EINVAL, "cannot open shard %s", path.c_str());
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 8) {
      ::close(fd);
      return fail(GROUT_EINVAL, "shard %s is shorter than a safetensors header", path.c_str());
    }
    auto m = std::make_unique<Mapped>();
    m->n = (size_t)st.st_size;
    m->p = mmap(nullptr, m->n, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m->p == MAP_FAILED) {
      m->p = nullptr;
      return fail(GROUT_EINVAL, "cannot map shard %s", path.c_str());
    }
    const unsigned char* base = static_cast<const unsigned char*>(m->p);
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | base[i];
    GROUT_NEED(hlen <= m->n - 8 && hlen <= (100u << 20), GROUT_EINVAL,
               "shard %s: header length %llu exceeds the file", path.c_str(),
               (unsigned long long)hlen);
    Value hdr;
    grout_json::Parser p(reinterpret_cast<const char*>(base + 8), (size_t)hlen);
    if (!p.parse(hdr) || hdr.kind != Value::kObject)
      return fail(GROUT_EINVAL, "shard %s: bad header: %s", path.c_str(), p.error().c_str());
    const unsigned char* data = base + 8 + hlen;
    const size_t data_len = m->n - 8 - (size_t)hlen;
    for (const auto& kv : hdr.obj) {
      if (kv.first == "__metadata__") continue;
      const Value& t = kv.second;
      const Value* dt = t.get("dtype");
      const Value* sh = t.get("shape");
      const Value* off = t.get("data_offsets");
      GROUT_NEED(dt && dt->kind == Value::kString && sh && sh->kind == Value::kArray && off &&
                     off->kind == Value::kArray && off->arr.size() == 2,
                 GROUT_EINVAL, "shard %s: malformed entry for %s", path.c_str(), kv.first.c_str());
      TensorRef r;
      if (dtype_of(dt->str, &r.dtype, &r.elem) != GROUT_OK) {
        // other tensors may use dtypes this loader never needs; reject only
        // when a needed tensor has one (checked in lookup)
        r.dtype = -1;
      }
      uint64_t numel = 1;
      for (const Value& d : sh->arr) {
        GROUT_NEED(d.kind == Value::kNumber && d.is_int && d.i >= 0 && d.i < (1LL << 40),
                   GROUT_EINVAL, "shard %s: bad shape for %s", path.c_str(), kv.first.c_str());
        r.shape.push_back(d.i);
        GROUT_NEED(numel <= (1ULL << 40) / ((uint64_t)d.i + 1), GROUT_EINVAL,
                   "shard %s: %s too large", path.c_str(), kv.first.c_str());
        numel *= (uint64_t)d.i;
      }
      const Value& b0 = off->arr[0];
      const Value& b1 = off->arr[1];
      GROUT_NEED(b0.kind == Value::kNumber && b0.is_int && b1.kind == Value::kNumber &&
                     b1.is_int && b0.i >= 0 && b0.i <= b1.i && (uint64_t)b1.i <= data_len,
                 GROUT_EINVAL, "shard %s: data_offsets of %s outside the file", path.c_str(),
                 kv.first.c_str());
      r.data = data + b0.i;
      r.bytes = (size_t)(b1.i - b0.i);
      if (r.dtype >= 0)
        GROUT_NEED(r.bytes == numel * r.elem, GROUT_EINVAL,
                   "shard %s: %s holds %zu bytes for %llu elements of %s", path.c_str(),
                   kv.first.c_str(), r.bytes, (unsigned long long)numel, dt->str.c_str());
      tensors[kv.first] = std::move(r);
    }
    shards[name] = std::move(m);
    return GROUT_OK;
  }

  int open(const char* model_dir) {
    GROUT_NEED(model_dir != nullptr && model_dir[0] != 0, GROUT_EINVAL, "model_dir is empty");
    dir = model_dir;
    GROUT_CHECK(parse_config(dir, &info));
    const std::string index = dir + "/model.safetensors.index.json";
    if (file_exists(index)) {
      Value idx;
      GROUT_CHECK(parse_json_file(index, idx));
      const Value* wm = idx.get("weight_map");
      GROUT_NEED(wm && wm->kind == Value::kObject, GROUT_EINVAL, "%s: no weight_map object",
                 index.c_str());
      for (const auto& kv : wm->obj) {
        GROUT_NEED(kv.second.kind == Value::kString, GROUT_EINVAL,
                   "%s: weight_map values must be file names", index.c_str());
        GROUT_CHECK(map_shard(kv.second.str));
      }
    } else {
      GROUT_CHECK(map_shard("model.safetensors"));
    }
    return GROUT_OK;
  }

  int lookup(const std::string& name, std::initializer_list<int64_t> shape, const TensorRef** out) {
    auto it = tensors.find(name);
    GROUT_NEED(it != tensors.end(), GROUT_EINVAL, "missing tensor %s", name.c_str());
    const TensorRef& r = it->second;
    GROUT_NEED(r.dtype >= 0, GROUT_ENOTSUP, "tensor %s: unsupported dtype for fp16 cast",
               name.c_str());
    const std::vector<int64_t> want(shape);
    if (r.shape != want) {
      std::string got, exp;
      for (auto d : r.shape) got += std::to_string(d) + ",";
      for (auto d : want) exp += std::to_string(d) + ",";
      return fail(GROUT_EINVAL, "tensor %s has shape [%s], expected [%s]", name.c_str(),
                  got.c_str(), exp.c_str());
    }
    if (r.dtype != kF16 && r.bytes > max_raw) max_raw = r.bytes;
    *out = &r;
    return GROUT_OK;
  }
};

// Planned upload: a tensor into the weight arena at an element offset.
struct Piece {
  const TensorRef* src;
  size_t dst_elem;
};

struct Plan {
  size_t total_elems = 0;
  std::vector<Piece> pieces;
  // element offsets of every engine weight
  size_t embed = 0, norm = 0, lm_head = 0;
  struct Layer {
    size_t in_ln, qkv, q_norm, k_norm, o, post_ln, gate_up, down;
  };
  std::vector<Layer> layers;

  size_t take(size_t elems) {
    const size_t off = total_elems;
    total_elems += (elems + 127) / 128 * 128;  // 256-byte alignment
    return off;
  }
};

int plan_weights(Checkpoint& ck, Plan& pl) {
  const grout_qwen3_config& c = ck.info.config;
  const int64_t H = c.hidden_size, I = c.intermediate_size, V = c.vocab_size;
  const int64_t qd = (int64_t)c.num_q_heads * 128, kd = (int64_t)c.num_kv_heads * 128;
  const TensorRef* t;
  GROUT_CHECK(ck.lookup("model.embed_tokens.weight", {V, H}, &t));
  pl.embed = pl.take((size_t)(V * H));
  pl.pieces.push_back({t, pl.embed});
  GROUT_CHECK(ck.lookup("model.norm.weight", {H}, &t));
  pl.norm = pl.take((size_t)H);
  pl.pieces.push_back({t, pl.norm});
  if (ck.info.tie_word_embeddings) {
    pl.lm_head = pl.embed;
  } else {
    GROUT_CHECK(ck.lookup("lm_head.weight", {V, H}, &t));
    pl.lm_head = pl.take((size_t)(V * H));
    pl.pieces.push_back({t, pl.lm_head});
  }
  for (int l = 0; l < c.num_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    Plan::Layer L{};
    auto one = [&](const char* name, std::initializer_list<int64_t> shape, size_t elems,
                   size_t* off) -> int {
      const TensorRef* r;
      GROUT_CHECK(ck.lookup(p + name, shape, &r));
      *off = pl.take(elems);
      pl.pieces.push_back({r, *off});
      return GROUT_OK;
    };
    GROUT_CHECK(one("input_layernorm.weight", {H}, (size_t)H, &L.in_ln));
    GROUT_CHECK(one("post_attention_layernorm.weight", {H}, (size_t)H, &L.post_ln));
    GROUT_CHECK(one("self_attn.q_norm.weight", {128}, 128, &L.q_norm));
    GROUT_CHECK(one("self_attn.k_norm.weight", {128}, 128, &L.k_norm));
    GROUT_CHECK(one("self_attn.o_proj.weight", {H, qd}, (size_t)(H * qd), &L.o));
    GROUT_CHECK(one("mlp.down_proj.weight", {H, I}, (size_t)(H * I), &L.down));
    // qkv_proj = rows of q_proj | k_proj | v_proj (src/model.rs:1526-1532)
    const TensorRef *tq, *tk, *tv;
    GROUT_CHECK(ck.lookup(p + "self_attn.q_proj.weight", {qd, H}, &tq));
    GROUT_CHECK(ck.lookup(p + "self_attn.k_proj.weight", {kd, H}, &tk));
    GROUT_CHECK(ck.lookup(p + "self_attn.v_proj.weight", {kd, H}, &tv));
    L.qkv = pl.take((size_t)((qd + 2 * kd) * H));
    pl.pieces.push_back({tq, L.qkv});
    pl.pieces.push_back({tk, L.qkv + (size_t)(qd * H)});
    pl.pieces.push_back({tv, L.qkv + (size_t)((qd + kd) * H)});
    // gate_up_proj = rows of gate_proj | up_proj (src/model.rs:1534-1538)
    const TensorRef *tg, *tu;
    GROUT_CHECK(ck.lookup(p + "mlp.gate_proj.weight", {I, H}, &tg));
    GROUT_CHECK(ck.lookup(p + "mlp.up_proj.weight", {I, H}, &tu));
    L.gate_up = pl.take((size_t)(2 * I * H));
    pl.pieces.push_back({tg, L.gate_up});
    pl.pieces.push_back({tu, L.gate_up + (size_t)(I * H)});
    pl.layers.push_back(L);
  }
  return GROUT_OK;
}

}  // namespace


extern "C" {

int grout_model_inspect(const char* model_dir, grout_model_info* info) {
  GROUT_NEED(info != nullptr, GROUT_EINVAL, "info is NULL");
  if (grout_gguf::is_gguf_path(model_dir)) return grout_gguf::inspect(model_dir, info);
  Checkpoint ck;
  GROUT_CHECK(ck.open(model_dir));
  Plan pl;
  GROUT_CHECK(plan_weights(ck, pl));
  *info = ck.info;
  info->weight_bytes = pl.total_elems * 2;
  return GROUT_OK;
}

int grout_model_load(const char* model_dir, int device, grout_model** out) {
  GROUT_NEED(out != nullptr, GROUT_EINVAL, "out is NULL");
  *out = nullptr;
  if (grout_gguf::is_gguf_path(model_dir)) return grout_gguf::load(model_dir, device, out);
  Checkpoint ck;
  GROUT_CHECK(ck.open(model_dir));
  Plan pl;
  GROUT_CHECK(plan_weights(ck, pl));
  int ndev = 0;
  GROUT_CHECK(hip_status(hipGetDeviceCount(&ndev), "hipGetDeviceCount"));
  GROUT_NEED(device >= 0 && device < ndev, GROUT_EINVAL, "device %d of %d", device, ndev);
  GROUT_CHECK(hip_status(hipSetDevice(device), "hipSetDevice"));

  std::unique_ptr<grout_model> m(new (std::nothrow) grout_model());
  GROUT_NEED(m != nullptr, GROUT_EINVAL, "out of host memory");
  m->info = ck.info;
  m->info.weight_bytes = pl.total_elems * 2;
  m->device = device;
  void* staging = nullptr;
  hipStream_t s = nullptr;
  int rc = hip_status(hipMalloc(&m->arena, pl.total_elems * 2), "hipMalloc(weights)");
  if (rc == GROUT_OK && ck.max_raw)
    rc = hip_status(hipMalloc(&staging, ck.max_raw), "hipMalloc(staging)");
  if (rc == GROUT_OK) rc = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "stream");
  uint16_t* base = static_cast<uint16_t*>(m->arena);
  for (size_t i = 0; rc == GROUT_OK && i < pl.pieces.size(); ++i) {
    const Piece& pc = pl.pieces[i];
    const TensorRef& t = *pc.src;
    if (t.dtype == kF16) {
      rc = hip_status(hipMemcpyAsync(base + pc.dst_elem, t.data, t.bytes, hipMemcpyHostToDevice, s),
                      "weights H2D");
    } else {
      rc = hip_status(hipMemcpyAsync(staging, t.data, t.bytes, hipMemcpyHostToDevice, s),
                      "weights H2D");
      if (rc == GROUT_OK)
        rc = hip_status(grout::launch_convert_to_f16(staging, t.dtype, t.bytes / t.elem,
                                                     base + pc.dst_elem, s),
                        "convert to f16");
      // the staging buffer is reused by the next tensor
      if (rc == GROUT_OK) rc = hip_status(hipStreamSynchronize(s), "hipStreamSynchronize");
    }
  }
  if (rc == GROUT_OK) rc = hip_status(hipStreamSynchronize(s), "hipStreamSynchronize");
  if (s) (void)hipStreamDestroy(s);
  if (staging) (void)hipFree(staging);
  if (rc != GROUT_OK) {
    const std::string msg = g_last_error;
    if (m->arena) (void)hipFree(m->arena);
    g_last_error = msg;
    return rc;
  }
  m->embed = base + pl.embed;
  m->norm = base + pl.norm;
  m->lm_head = base + pl.lm_head;
  for (const Plan::Layer& L : pl.layers) {
    grout_qwen3_layer g;
    g.input_layernorm = base + L.in_ln;
    g.qkv_proj = base + L.qkv;
    g.q_norm = base + L.q_norm;
    g.k_norm = base + L.k_norm;
    g.o_proj = base + L.o;
    g.post_attention_layernorm = base + L.post_ln;
    g.gate_up_proj = base + L.gate_up;
    g.down_proj = base + L.down;
    m->layers.push_back(g);
  }
  *out = m.release();
  return GROUT_OK;
}

int grout_model_get_info(const grout_model* m, grout_model_info* info) {
  GROUT_NEED(m != nullptr && info != nullptr, GROUT_EINVAL, "model or info is NULL");
  *info = m->info;
  return GROUT_OK;
}

int grout_model_weights(const grout_model* m, grout_qwen3_weights* w) {
  GROUT_NEED(m != nullptr && w != nullptr, GROUT_EINVAL, "model or weights is NULL");
  GROUT_NEED(!m->low_bit, GROUT_EINVAL, "the model holds GGUF weights: use grout_model_qweights");
  w->embed_tokens = m->embed;
  w->norm = m->norm;
  w->lm_head = m->lm_head;
  w->layers = m->layers.data();
  return GROUT_OK;
}

int grout_model_qweights(const grout_model* m, grout_qwen3_qweights* w) {
  GROUT_NEED(m != nullptr && w != nullptr, GROUT_EINVAL, "model or weights is NULL");
  GROUT_NEED(m->low_bit, GROUT_EINVAL, "the model holds fp16 weights: use grout_model_weights");
  w->embed_tokens = m->qembed;
  w->norm = m->norm;
  w->lm_head = m->qlm_head;
  w->layers = m->qlayers.data();
  return GROUT_OK;
}

int grout_model_free(grout_model* m) {
  if (!m) return GROUT_OK;
  if (m->arena) {
    (void)hipSetDevice(m->device);
    (void)hipFree(m->arena);
  }
  delete m;
  return GROUT_OK;
}

}  // extern "C"
