// GGUF (v2 / v3) Qwen3 checkpoints -> device weights for
// grout_engine_create_q.
//
// Reference: the GGUF reader (src/gguf.rs:212-445) with its bounds (strings
// at most 1 GiB and within the file, arrays at most 2^30 elements, at most
// 16M metadata array elements over the whole file, value nesting at most 64,
// at most 4 tensor dimensions, format versions 2 and 3, general.alignment
// default 32), config_from_gguf (src/loader.rs:276-330: the qwen3.* keys,
// vocab = token_embd rows, tied head when output.weight is absent), the
// tensor names of map_engine_tensor_name (src/loader.rs:660-698) and the
// per-type load policy of load_device_weight_gguf (src/loader.rs:340-379):
// Q8_0 / Q4_K / Q5_K / Q6_K matrices in the decode layout, F16 / F32 / BF16
// tensors as f16, the token embedding gathered from its blocks and reused as
// the head when tied.  The file is mmapped; every tensor's type, shape and
// byte range is validated before the device is touched.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "abi_util.hpp"
#include "kernels.hpp"
#include "model_internal.hpp"

using namespace grout_abi;

namespace {

constexpr uint64_t kMaxString = 1ull << 30;
constexpr uint64_t kMaxArray = 1ull << 30;
constexpr uint64_t kMaxMetaElems = 16ull << 20;
constexpr int kMaxDepth = 64;
constexpr uint32_t kMaxDims = 4;
constexpr uint64_t kDefaultAlign = 32;

// GGUF metadata value types.
enum : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7, kString = 8,
  kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12
};

// ggml tensor types this loader reads.
enum : uint32_t { kTF32 = 0, kTF16 = 1, kTQ8_0 = 8, kTQ4_K = 12, kTQ5_K = 13, kTQ6_K = 14, kTBF16 = 30 };
// ggml types a GGUF file may hold that this loader refuses (named in errors)
enum : uint32_t { kTQ4_0 = 2, kTQ4_1 = 3, kTQ5_0 = 6, kTQ5_1 = 7, kTQ8_1 = 9, kTQ2_K = 10, kTQ3_K = 11, kTQ8_K = 15 };

// (weights per block, bytes per block), or (0, 0) for types not read here.
void type_block(uint32_t t, uint64_t* be, uint64_t* bb) {
  *be = 0;
  *bb = 0;
  switch (t) {
    case kTF32: *be = 1; *bb = 4; break;
    case kTF16: case kTBF16: *be = 1; *bb = 2; break;
    case kTQ8_0: *be = 32; *bb = 34; break;
    case kTQ4_K: *be = 256; *bb = 144; break;
    case kTQ5_K: *be = 256; *bb = 176; break;
    case kTQ6_K: *be = 256; *bb = 210; break;
    default: break;
  }
}

const char* type_name(uint32_t t) {
  switch (t) {
    case kTF32: return "F32";
    case kTF16: return "F16";
    case kTBF16: return "BF16";
    case kTQ8_0: return "Q8_0";
    case kTQ4_K: return "Q4_K";
    case kTQ5_K: return "Q5_K";
    case kTQ6_K: return "Q6_K";
    case kTQ4_0: return "Q4_0";
    case kTQ4_1: return "Q4_1";
    case kTQ5_0: return "Q5_0";
    case kTQ5_1: return "Q5_1";
    case kTQ8_1: return "Q8_1";
    case kTQ2_K: return "Q2_K";
    case kTQ3_K: return "Q3_K";
    case kTQ8_K: return "Q8_K";
    default: return "?";
  }
}

uint64_t min_disk_size(uint32_t t) {
  switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    case kString: return 8;
    case kArray: return 12;
    default: return 1;
  }
}

// A scalar metadata value (arrays keep only their element type and length).
struct Meta {
  uint32_t type = 0;
  uint64_t u = 0;     // unsigned integers, bool
  int64_t i = 0;      // signed integers
  double f = 0.0;     // floats
  std::string str;
  uint32_t elem = 0;  // arrays
  uint64_t count = 0;
};

struct Reader {
  const uint8_t* p = nullptr;
  uint64_t n = 0, pos = 0;
  uint64_t budget = kMaxMetaElems;

  uint64_t remaining() const { return n - pos; }
  int take(void* out, uint64_t k) {
    GROUT_NEED(k <= remaining(), GROUT_EINVAL, "GGUF file truncated at byte %llu",
               (unsigned long long)pos);
    std::memcpy(out, p + pos, k);
    pos += k;
    return GROUT_OK;
  }
  int u32(uint32_t* v) { return take(v, 4); }
  int u64(uint64_t* v) { return take(v, 8); }
  int str(std::string* s) {
    uint64_t len;
    GROUT_CHECK(u64(&len));
    GROUT_NEED(len <= kMaxString, GROUT_EINVAL, "GGUF string length %llu exceeds max %llu",
               (unsigned long long)len, (unsigned long long)kMaxString);
    GROUT_NEED(len <= remaining(), GROUT_EINVAL,
               "GGUF string length %llu exceeds remaining file bytes %llu",
               (unsigned long long)len, (unsigned long long)remaining());
    s->assign(reinterpret_cast<const char*>(p + pos), (size_t)len);
    pos += len;
    while (!s->empty() && s->back() == '\0') s->pop_back();
    return GROUT_OK;
  }
  // One value of type t into m (scalars) or skipped (array contents).
  int value(uint32_t t, int depth, Meta* m) {
    GROUT_NEED(depth <= kMaxDepth, GROUT_EINVAL, "GGUF value nesting depth exceeds max %d",
               kMaxDepth);
    if (m) m->type = t;
    uint8_t b1;
    uint16_t b2;
    uint32_t b4;
    uint64_t b8;
    switch (t) {
      case kU8: GROUT_CHECK(take(&b1, 1)); if (m) m->u = b1; return GROUT_OK;
      case kI8: GROUT_CHECK(take(&b1, 1)); if (m) m->i = (int8_t)b1; return GROUT_OK;
      case kU16: GROUT_CHECK(take(&b2, 2)); if (m) m->u = b2; return GROUT_OK;
      case kI16: GROUT_CHECK(take(&b2, 2)); if (m) m->i = (int16_t)b2; return GROUT_OK;
      case kU32: GROUT_CHECK(take(&b4, 4)); if (m) m->u = b4; return GROUT_OK;
      case kI32: GROUT_CHECK(take(&b4, 4)); if (m) m->i = (int32_t)b4; return GROUT_OK;
      case kU64: GROUT_CHECK(take(&b8, 8)); if (m) m->u = b8; return GROUT_OK;
      case kI64: GROUT_CHECK(take(&b8, 8)); if (m) m->i = (int64_t)b8; return GROUT_OK;
      case kF32: {
        float f;
        GROUT_CHECK(take(&f, 4));
        if (m) m->f = f;
        return GROUT_OK;
      }
      case kF64: {
        double f;
        GROUT_CHECK(take(&f, 8));
        if (m) m->f = f;
        return GROUT_OK;
      }
      case kBool:
        GROUT_CHECK(take(&b1, 1));
        GROUT_NEED(b1 <= 1, GROUT_EINVAL, "GGUF invalid bool value %u", (unsigned)b1);
        if (m) m->u = b1;
        return GROUT_OK;
      case kString: {
        std::string s;
        GROUT_CHECK(str(&s));
        if (m) m->str = std::move(s);
        return GROUT_OK;
      }
      case kArray: {
        uint32_t et;
        uint64_t len;
        GROUT_CHECK(u32(&et));
        GROUT_NEED(et <= kF64, GROUT_EINVAL, "GGUF unrecognized value type %u", et);
        GROUT_CHECK(u64(&len));
        GROUT_NEED(len <= kMaxArray, GROUT_EINVAL, "GGUF array length %llu exceeds max %llu",
                   (unsigned long long)len, (unsigned long long)kMaxArray);
        GROUT_NEED(len <= budget, GROUT_EINVAL,
                   "GGUF metadata arrays exceed the total element budget %llu (array of %llu "
                   "elements, %llu remaining)",
                   (unsigned long long)kMaxMetaElems, (unsigned long long)len,
                   (unsigned long long)budget);
        budget -= len;
        const uint64_t need = len * min_disk_size(et);
        GROUT_NEED(need <= remaining(), GROUT_EINVAL,
                   "GGUF array of %llu elements needs at least %llu bytes, only %llu remaining",
                   (unsigned long long)len, (unsigned long long)need,
                   (unsigned long long)remaining());
        if (m) {
          m->elem = et;
          m->count = len;
        }
        for (uint64_t k = 0; k < len; ++k) GROUT_CHECK(value(et, depth + 1, nullptr));
        return GROUT_OK;
      }
      default:
        return fail(GROUT_EINVAL, "GGUF unrecognized value type %u", t);
    }
  }
};

struct Tensor {
  uint32_t type = 0;
  std::vector<uint64_t> shape;  // outermost first (ggml order reversed)
  const uint8_t* data = nullptr;
  uint64_t bytes = 0;
};

struct File {
  std::string path;
  void* map = nullptr;
  uint64_t size = 0;
  std::map<std::string, Meta> meta;
  std::map<std::string, Tensor> tensors;

  ~File() {
    if (map) munmap(map, size);
  }

  int open(const char* p) {
    path = p;
    const int fd = ::open(p, O_RDONLY);
    GROUT_NEED(fd >= 0, GROUT_EINVAL, "cannot open %s", p);
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode) || st.st_size < 24) {
      ::close(fd);
      return fail(GROUT_EINVAL, "%s is not a GGUF file (too short)", p);
    }
    size = (uint64_t)st.st_size;
    map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map == MAP_FAILED) {
      map = nullptr;
      return fail(GROUT_EINVAL, "cannot map %s", p);
    }
    return parse();
  }

  int parse() {
    Reader r;
    r.p = static_cast<const uint8_t*>(map);
    r.n = size;
    uint32_t magic, version;
    GROUT_CHECK(r.u32(&magic));
    GROUT_NEED(magic == 0x46554747u, GROUT_EINVAL,
               "%s: GGUF magic must be little-endian 0x46554747, got 0x%08x", path.c_str(), magic);
    GROUT_CHECK(r.u32(&version));
    GROUT_NEED(version == 2 || version == 3, GROUT_EINVAL,
               "%s: GGUF version %u is unsupported; expected v2 or v3", path.c_str(), version);
    uint64_t n_tensors, n_kv;
    GROUT_CHECK(r.u64(&n_tensors));
    GROUT_CHECK(r.u64(&n_kv));
    GROUT_NEED(n_tensors <= kMaxArray && n_kv <= kMaxArray, GROUT_EINVAL,
               "%s: GGUF tensor_count %llu or metadata_kv_count %llu exceeds max", path.c_str(),
               (unsigned long long)n_tensors, (unsigned long long)n_kv);
    for (uint64_t k = 0; k < n_kv; ++k) {
      std::string key;
      uint32_t t;
      GROUT_CHECK(r.str(&key));
      GROUT_CHECK(r.u32(&t));
      Meta m;
      GROUT_CHECK(r.value(t, 0, &m));
      meta[key] = std::move(m);  // duplicate keys: the last one wins, as in the reference
    }
    struct Info {
      std::string name;
      Tensor t;
      uint64_t offset;
    };
    std::vector<Info> infos;
    infos.reserve((size_t)std::min<uint64_t>(n_tensors, 1 << 16));
    for (uint64_t k = 0; k < n_tensors; ++k) {
      Info in;
      GROUT_CHECK(r.str(&in.name));
      uint32_t nd;
      GROUT_CHECK(r.u32(&nd));
      GROUT_NEED(nd <= kMaxDims, GROUT_EINVAL, "GGUF tensor `%s` has %u dimensions, max is %u",
                 in.name.c_str(), nd, kMaxDims);
      for (uint32_t d = 0; d < nd; ++d) {
        uint64_t dim;
        GROUT_CHECK(r.u64(&dim));
        in.t.shape.push_back(dim);
      }
      std::reverse(in.t.shape.begin(), in.t.shape.end());
      GROUT_CHECK(r.u32(&in.t.type));
      GROUT_CHECK(r.u64(&in.offset));
      infos.push_back(std::move(in));
    }
    uint64_t align = kDefaultAlign;
    auto it = meta.find("general.alignment");
    if (it != meta.end()) {
      const Meta& a = it->second;
      if (a.type == kU8 || a.type == kU16 || a.type == kU32 || a.type == kU64)
        align = a.u;
      else if ((a.type == kI8 || a.type == kI16 || a.type == kI32 || a.type == kI64) && a.i >= 0)
        align = (uint64_t)a.i;
      GROUT_NEED(align > 0, GROUT_EINVAL, "%s: GGUF general.alignment must be positive",
                 path.c_str());
    }
    GROUT_NEED(r.pos <= UINT64_MAX - (align - 1), GROUT_EINVAL, "GGUF alignment overflow");
    const uint64_t data_off = (r.pos + align - 1) / align * align;
    GROUT_NEED(data_off <= size, GROUT_EINVAL,
               "%s: GGUF tensor data offset %llu exceeds file size %llu", path.c_str(),
               (unsigned long long)data_off, (unsigned long long)size);
    for (Info& in : infos) {
      // byte range: only for the types read here (others are checked when needed)
      uint64_t be, bb;
      type_block(in.t.type, &be, &bb);
      if (be != 0) {
        uint64_t elems = 1;
        for (uint64_t d : in.t.shape) {
          GROUT_NEED(d == 0 || elems <= (1ull << 48) / d, GROUT_EINVAL,
                     "GGUF tensor `%s` element count overflows", in.name.c_str());
          elems *= d;
        }
        GROUT_NEED(elems % be == 0, GROUT_EINVAL,
                   "GGUF tensor `%s` has %llu elements, not divisible by %s block size %llu",
                   in.name.c_str(), (unsigned long long)elems, type_name(in.t.type),
                   (unsigned long long)be);
        in.t.bytes = elems / be * bb;
        GROUT_NEED(in.offset <= size - data_off && in.t.bytes <= size - data_off - in.offset,
                   GROUT_EINVAL, "GGUF tensor `%s` data (%llu bytes at %llu) is outside the file",
                   in.name.c_str(), (unsigned long long)in.t.bytes,
                   (unsigned long long)in.offset);
        in.t.data = static_cast<const uint8_t*>(map) + data_off + in.offset;
      }
      tensors[in.name] = std::move(in.t);
    }
    return GROUT_OK;
  }

  const Meta* get(const char* key) const {
    auto it = meta.find(key);
    return it == meta.end() ? nullptr : &it->second;
  }
  int need_uint(const char* key, uint64_t max, uint64_t* out) const {
    const Meta* m = get(key);
    GROUT_NEED(m != nullptr, GROUT_EINVAL, "%s: GGUF metadata key %s is missing", path.c_str(),
               key);
    uint64_t v;
    if (m->type == kU8 || m->type == kU16 || m->type == kU32 || m->type == kU64)
      v = m->u;
    else if ((m->type == kI8 || m->type == kI16 || m->type == kI32 || m->type == kI64) &&
             m->i >= 0)
      v = (uint64_t)m->i;
    else
      return fail(GROUT_EINVAL, "%s: GGUF metadata %s is not an unsigned integer", path.c_str(),
                  key);
    GROUT_NEED(v <= max, GROUT_EINVAL, "%s: GGUF metadata %s = %llu exceeds %llu", path.c_str(),
               key, (unsigned long long)v, (unsigned long long)max);
    *out = v;
    return GROUT_OK;
  }
  int need_float(const char* key, float* out) const {
    const Meta* m = get(key);
    GROUT_NEED(m != nullptr, GROUT_EINVAL, "%s: GGUF metadata key %s is missing", path.c_str(),
               key);
    GROUT_NEED(m->type == kF32 || m->type == kF64, GROUT_EINVAL,
               "%s: GGUF metadata %s is not f32/f64", path.c_str(), key);
    GROUT_NEED(std::isfinite(m->f), GROUT_EINVAL, "%s: GGUF metadata %s is not finite",
               path.c_str(), key);
    *out = (float)m->f;
    return GROUT_OK;
  }
};

// src/loader.rs:276-330 with the range checks of src/config.rs:44-95.
int read_config(const File& f, grout_model_info* info) {
  const Meta* arch = f.get("general.architecture");
  GROUT_NEED(arch != nullptr && arch->type == kString, GROUT_EINVAL,
             "%s: GGUF metadata general.architecture is missing", f.path.c_str());
  GROUT_NEED(arch->str == "qwen3", GROUT_ENOTSUP,
             "%s: unsupported GGUF architecture `%s`; this engine only supports qwen3",
             f.path.c_str(), arch->str.c_str());
  uint64_t layers, hidden, inter, hq, hkv, hd, ctx, eos;
  float eps, theta;
  GROUT_CHECK(f.need_uint("qwen3.block_count", 1 << 12, &layers));
  GROUT_CHECK(f.need_uint("qwen3.embedding_length", 1 << 20, &hidden));
  GROUT_CHECK(f.need_uint("qwen3.feed_forward_length", 1 << 22, &inter));
  GROUT_CHECK(f.need_uint("qwen3.attention.head_count", 1 << 12, &hq));
  GROUT_CHECK(f.need_uint("qwen3.attention.head_count_kv", 1 << 12, &hkv));
  GROUT_CHECK(f.need_uint("qwen3.attention.key_length", 1 << 12, &hd));
  GROUT_CHECK(f.need_float("qwen3.rope.freq_base", &theta));
  GROUT_CHECK(f.need_float("qwen3.attention.layer_norm_rms_epsilon", &eps));
  GROUT_CHECK(f.need_uint("qwen3.context_length", 1u << 25, &ctx));
  GROUT_CHECK(f.need_uint("tokenizer.ggml.eos_token_id", 0xffffffffull, &eos));
  auto te = f.tensors.find("token_embd.weight");
  GROUT_NEED(te != f.tensors.end(), GROUT_EINVAL, "%s: missing tensor token_embd.weight",
             f.path.c_str());
  GROUT_NEED(te->second.shape.size() == 2, GROUT_EINVAL,
             "%s: token_embd.weight must be rank-2", f.path.c_str());
  const uint64_t vocab = te->second.shape[0];
  GROUT_NEED(vocab >= 1 && vocab <= (1u << 24), GROUT_EINVAL, "%s: vocab size %llu",
             f.path.c_str(), (unsigned long long)vocab);
  GROUT_NEED(layers >= 1 && hidden >= 1 && inter >= 1 && hq >= 1 && hkv >= 1 && ctx >= 1,
             GROUT_EINVAL, "%s: zero-sized dimension in the qwen3 metadata", f.path.c_str());
  GROUT_NEED(hq % hkv == 0, GROUT_EINVAL, "%s: head_count=%llu not divisible by %llu",
             f.path.c_str(), (unsigned long long)hq, (unsigned long long)hkv);
  GROUT_NEED(hd == 128, GROUT_ENOTSUP, "%s: key_length=%llu: only 128 is supported",
             f.path.c_str(), (unsigned long long)hd);
  GROUT_NEED(eps > 0.f && theta > 0.f, GROUT_EINVAL, "%s: rms epsilon / rope base must be > 0",
             f.path.c_str());
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
  c.max_ctx = (int)ctx;
  info->tie_word_embeddings = f.tensors.count("output.weight") ? 0 : 1;
  info->num_eos = 1;
  info->eos_token_ids[0] = (uint32_t)eos;
  return GROUT_OK;
}

// Engine format of a ggml tensor type (GROUT_WFMT_F16 for the types cast to
// f16), or -1.
int engine_fmt(uint32_t t) {
  switch (t) {
    case kTF32: case kTF16: case kTBF16: return GROUT_WFMT_F16;
    case kTQ8_0: return GROUT_WFMT_Q8_0;
    case kTQ4_K: return GROUT_WFMT_Q4_K;
    case kTQ5_K: return GROUT_WFMT_Q5_K;
    case kTQ6_K: return GROUT_WFMT_Q6_K;
    default: return -1;
  }
}

// Upload plan: device byte offsets and the tensors behind them.
struct Part {
  int fmt = GROUT_WFMT_F16;
  int rows = 0, k = 0;
  size_t off = 0;
  std::vector<const Tensor*> src;  // consecutive row blocks
};
struct Vec {
  size_t off = 0;
  const Tensor* src = nullptr;
};
struct Plan {
  size_t total = 0;
  size_t staging = 0;  // largest low-bit run or cast tensor
  Part embed, head;
  bool tied = false;
  Vec norm;
  struct Layer {
    Vec in_ln, post_ln, q_norm, k_norm;
    std::vector<Part> qkv, gate_up;
    Part o, down;
  };
  std::vector<Layer> layers;
  size_t take(size_t bytes) {
    const size_t o = total;
    total += (bytes + 255) / 256 * 256;
    return o;
  }
};

int lookup(const File& f, const std::string& name, std::initializer_list<uint64_t> shape,
           bool matrix, const Tensor** out) {
  auto it = f.tensors.find(name);
  GROUT_NEED(it != f.tensors.end(), GROUT_EINVAL, "%s: missing tensor %s", f.path.c_str(),
             name.c_str());
  const Tensor& t = it->second;
  const int fmt = engine_fmt(t.type);
  GROUT_NEED(fmt >= 0 && (matrix || fmt == GROUT_WFMT_F16), GROUT_ENOTSUP,
             "%s: unsupported ggml type %s (%u) for tensor `%s`", f.path.c_str(),
             type_name(t.type), t.type, name.c_str());
  const std::vector<uint64_t> want(shape);
  if (t.shape != want) {
    std::string got, exp;
    for (auto d : t.shape) got += std::to_string(d) + ",";
    for (auto d : want) exp += std::to_string(d) + ",";
    return fail(GROUT_EINVAL, "%s: tensor %s has shape [%s], expected [%s]", f.path.c_str(),
                name.c_str(), got.c_str(), exp.c_str());
  }
  *out = &t;
  return GROUT_OK;
}

// Splits the row-ordered matrices into parts of one engine format each.
int plan_parts(Plan& pl, const std::vector<const Tensor*>& mats, const std::vector<int>& rows,
               int k, std::vector<Part>& out, const std::string& what) {
  size_t i = 0;
  while (i < mats.size()) {
    Part p;
    p.fmt = engine_fmt(mats[i]->type);
    p.k = k;
    size_t raw = 0;
    size_t j = i;
    for (; j < mats.size() && engine_fmt(mats[j]->type) == p.fmt; ++j) {
      p.rows += rows[j];
      p.src.push_back(mats[j]);
      raw += mats[j]->bytes;
      if (p.fmt == GROUT_WFMT_F16 && mats[j]->type != kTF16)
        pl.staging = std::max(pl.staging, (size_t)mats[j]->bytes);
    }
    size_t bytes;
    if (p.fmt == GROUT_WFMT_F16) {
      bytes = (size_t)p.rows * k * 2;
    } else {
      bytes = grout::qweight_bytes(p.fmt, p.rows, k);
      GROUT_NEED(bytes != 0, GROUT_ENOTSUP,
                 "%s: format %d does not fit k=%d (a multiple of the block size, at most 32768)",
                 what.c_str(), p.fmt, k);
      pl.staging = std::max(pl.staging, raw);
    }
    p.off = pl.take(bytes);
    out.push_back(std::move(p));
    i = j;
  }
  return GROUT_OK;
}

int plan_vec(Plan& pl, const File& f, const std::string& name, uint64_t n, Vec* v) {
  GROUT_CHECK(lookup(f, name, {n}, false, &v->src));
  if (v->src->type != kTF16) pl.staging = std::max(pl.staging, (size_t)v->src->bytes);
  v->off = pl.take(n * 2);
  return GROUT_OK;
}

int plan_weights(const File& f, const grout_model_info& info, Plan& pl) {
  const grout_qwen3_config& c = info.config;
  const uint64_t H = c.hidden_size, I = c.intermediate_size, V = c.vocab_size;
  const uint64_t qd = (uint64_t)c.num_q_heads * 128, kd = (uint64_t)c.num_kv_heads * 128;
  const Tensor* t;
  std::vector<Part> one;
  GROUT_CHECK(lookup(f, "token_embd.weight", {V, H}, true, &t));
  GROUT_CHECK(plan_parts(pl, {t}, {(int)V}, (int)H, one, "token_embd.weight"));
  pl.embed = one[0];
  GROUT_CHECK(plan_vec(pl, f, "output_norm.weight", H, &pl.norm));
  pl.tied = info.tie_word_embeddings != 0;
  if (pl.tied) {
    pl.head = pl.embed;
  } else {
    one.clear();
    GROUT_CHECK(lookup(f, "output.weight", {V, H}, true, &t));
    GROUT_CHECK(plan_parts(pl, {t}, {(int)V}, (int)H, one, "output.weight"));
    pl.head = one[0];
  }
  for (int l = 0; l < c.num_layers; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    Plan::Layer L;
    GROUT_CHECK(plan_vec(pl, f, p + "attn_norm.weight", H, &L.in_ln));
    GROUT_CHECK(plan_vec(pl, f, p + "ffn_norm.weight", H, &L.post_ln));
    GROUT_CHECK(plan_vec(pl, f, p + "attn_q_norm.weight", 128, &L.q_norm));
    GROUT_CHECK(plan_vec(pl, f, p + "attn_k_norm.weight", 128, &L.k_norm));
    const Tensor *tq, *tk, *tv, *tg, *tu, *to, *td;
    GROUT_CHECK(lookup(f, p + "attn_q.weight", {qd, H}, true, &tq));
    GROUT_CHECK(lookup(f, p + "attn_k.weight", {kd, H}, true, &tk));
    GROUT_CHECK(lookup(f, p + "attn_v.weight", {kd, H}, true, &tv));
    GROUT_CHECK(lookup(f, p + "attn_output.weight", {H, qd}, true, &to));
    GROUT_CHECK(lookup(f, p + "ffn_gate.weight", {I, H}, true, &tg));
    GROUT_CHECK(lookup(f, p + "ffn_up.weight", {I, H}, true, &tu));
    GROUT_CHECK(lookup(f, p + "ffn_down.weight", {H, I}, true, &td));
    GROUT_CHECK(plan_parts(pl, {tq, tk, tv}, {(int)qd, (int)kd, (int)kd}, (int)H, L.qkv,
                           p + "attn_q/k/v"));
    GROUT_CHECK(plan_parts(pl, {tg, tu}, {(int)I, (int)I}, (int)H, L.gate_up, p + "ffn_gate/up"));
    one.clear();
    GROUT_CHECK(plan_parts(pl, {to}, {(int)H}, (int)qd, one, p + "attn_output.weight"));
    L.o = one[0];
    one.clear();
    GROUT_CHECK(plan_parts(pl, {td}, {(int)H}, (int)I, one, p + "ffn_down.weight"));
    L.down = one[0];
    pl.layers.push_back(std::move(L));
  }
  return GROUT_OK;
}

// One tensor of a cast type into f16 at dst (through the staging buffer).
int upload_f16(const Tensor& t, void* dst, void* staging, hipStream_t s) {
  if (t.type == kTF16)
    return hip_status(hipMemcpyAsync(dst, t.data, t.bytes, hipMemcpyHostToDevice, s), "H2D");
  GROUT_CHECK(hip_status(hipMemcpyAsync(staging, t.data, t.bytes, hipMemcpyHostToDevice, s), "H2D"));
  const int dtype = t.type == kTF32 ? 2 : 1;  // f32 / bf16
  const size_t n = t.bytes / (t.type == kTF32 ? 4 : 2);
  GROUT_CHECK(hip_status(grout::launch_convert_to_f16(staging, dtype, n, dst, s), "cast to f16"));
  return hip_status(hipStreamSynchronize(s), "hipStreamSynchronize");  // staging is reused
}

int upload_part(const Part& p, char* base, void* staging, hipStream_t s) {
  if (p.fmt == GROUT_WFMT_F16) {
    size_t row = 0;
    for (const Tensor* t : p.src) {
      GROUT_CHECK(upload_f16(*t, base + p.off + row * p.k * 2, staging, s));
      row += (size_t)t->shape[0];
    }
    return GROUT_OK;
  }
  size_t at = 0;
  for (const Tensor* t : p.src) {
    GROUT_CHECK(hip_status(hipMemcpyAsync(static_cast<char*>(staging) + at, t->data, t->bytes,
                                          hipMemcpyHostToDevice, s),
                           "H2D"));
    at += t->bytes;
  }
  GROUT_CHECK(hip_status(grout::launch_qweight_repack(p.fmt, staging, p.rows, p.k, base + p.off, s),
                         "repack"));
  return hip_status(hipStreamSynchronize(s), "hipStreamSynchronize");
}

grout_wpart wpart(const Part& p, char* base) { return grout_wpart{p.fmt, p.rows, base + p.off}; }

}  // namespace

namespace grout_gguf {

bool is_gguf_path(const char* path) {
  if (!path) return false;
  const size_t n = std::strlen(path);
  if (n < 5) return false;
  const char* e = path + n - 5;
  return e[0] == '.' && (e[1] | 32) == 'g' && (e[2] | 32) == 'g' && (e[3] | 32) == 'u' &&
         (e[4] | 32) == 'f';
}

int inspect(const char* path, grout_model_info* info) {
  File f;
  GROUT_CHECK(f.open(path));
  GROUT_CHECK(read_config(f, info));
  Plan pl;
  GROUT_CHECK(plan_weights(f, *info, pl));
  info->weight_bytes = pl.total;
  return GROUT_OK;
}

int load(const char* path, int device, grout_model** out) {
  File f;
  GROUT_CHECK(f.open(path));
  grout_model_info info;
  GROUT_CHECK(read_config(f, &info));
  Plan pl;
  GROUT_CHECK(plan_weights(f, info, pl));
  info.weight_bytes = pl.total;
  int ndev = 0;
  GROUT_CHECK(hip_status(hipGetDeviceCount(&ndev), "hipGetDeviceCount"));
  GROUT_NEED(device >= 0 && device < ndev, GROUT_EINVAL, "device %d of %d", device, ndev);
  GROUT_CHECK(hip_status(hipSetDevice(device), "hipSetDevice"));
  std::unique_ptr<grout_model> m(new (std::nothrow) grout_model());
  GROUT_NEED(m != nullptr, GROUT_EINVAL, "out of host memory");
  m->info = info;
  m->device = device;
  m->low_bit = true;
  void* staging = nullptr;
  hipStream_t s = nullptr;
  int rc = hip_status(hipMalloc(&m->arena, pl.total), "hipMalloc(weights)");
  if (rc == GROUT_OK && pl.staging)
    rc = hip_status(hipMalloc(&staging, pl.staging), "hipMalloc(staging)");
  if (rc == GROUT_OK) rc = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "stream");
  char* base = static_cast<char*>(m->arena);
  auto vec = [&](const Vec& v) { return upload_f16(*v.src, base + v.off, staging, s); };
  if (rc == GROUT_OK) rc = upload_part(pl.embed, base, staging, s);
  if (rc == GROUT_OK && !pl.tied) rc = upload_part(pl.head, base, staging, s);
  if (rc == GROUT_OK) rc = vec(pl.norm);
  for (size_t l = 0; rc == GROUT_OK && l < pl.layers.size(); ++l) {
    const Plan::Layer& L = pl.layers[l];
    for (const Vec* v : {&L.in_ln, &L.post_ln, &L.q_norm, &L.k_norm})
      if (rc == GROUT_OK) rc = vec(*v);
    for (const Part& p : L.qkv)
      if (rc == GROUT_OK) rc = upload_part(p, base, staging, s);
    for (const Part& p : L.gate_up)
      if (rc == GROUT_OK) rc = upload_part(p, base, staging, s);
    if (rc == GROUT_OK) rc = upload_part(L.o, base, staging, s);
    if (rc == GROUT_OK) rc = upload_part(L.down, base, staging, s);
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
  m->qembed = wpart(pl.embed, base);
  m->qlm_head = pl.tied ? m->qembed : wpart(pl.head, base);
  m->norm = base + pl.norm.off;
  for (const Plan::Layer& L : pl.layers) {
    grout_qwen3_qlayer q{};
    q.input_layernorm = base + L.in_ln.off;
    q.post_attention_layernorm = base + L.post_ln.off;
    q.q_norm = base + L.q_norm.off;
    q.k_norm = base + L.k_norm.off;
    q.num_qkv_parts = (int)L.qkv.size();
    for (size_t i = 0; i < L.qkv.size(); ++i) q.qkv[i] = wpart(L.qkv[i], base);
    q.num_gate_up_parts = (int)L.gate_up.size();
    for (size_t i = 0; i < L.gate_up.size(); ++i) q.gate_up[i] = wpart(L.gate_up[i], base);
    q.o_proj = wpart(L.o, base);
    q.down_proj = wpart(L.down, base);
    m->qlayers.push_back(q);
  }
  *out = m.release();
  return GROUT_OK;
}

}  // namespace grout_gguf
