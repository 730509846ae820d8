/* grout.hpp -- C++17 host mirror of the reference's synchronous engine API
 * (grout::Engine, src/api.rs:11-183) over the C ABI of grout_engine.h.
 *
 * Header only: link against libgrout_attn.so.  Every member that can fail
 * throws grout::Error carrying the ABI status code and grout_last_error()'s
 * message, where the reference returns anyhow::Result.  Same names, argument
 * meaning and checks as the Rust API:
 *
 *   auto eng = grout::Engine::load("/models/Qwen3-4B", {4096, 0});
 *   eng.warmup();
 *   grout::Logits l = eng.prefill(prompt_ids);
 *   uint32_t tok = argmax(l.values);
 *   while (...) tok = eng.decode_greedy(tok);
 *   eng.reset();
 *
 * One engine, one thread at a time (as the reference's Engine, which is not
 * Sync); calls block until their work on the engine's stream is done. */
#ifndef GROUT_HPP
#define GROUT_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "grout_engine.h"

namespace grout {

/* An ABI status (GROUT_E*, or a hipError_t when > 0) and its message. */
class Error : public std::runtime_error {
 public:
  Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
  int code() const noexcept { return code_; }

 private:
  int code_;
};

inline void check(int rc, const char* call) {
  if (rc != GROUT_OK) throw Error(rc, std::string(call) + ": " + grout_last_error());
}

/* Model load options (src/api.rs:21-38). */
struct LoadOpts {
  std::size_t max_ctx = 0;  // maximum context to allocate; 0 = the model's default
  int device_ord = 0;       // HIP device ordinal
};

/* Last-token logits copied to the host as f32 (src/api.rs:40-45, 186-196). */
struct Logits {
  std::vector<float> values;  // meta().vocab_size entries
  const std::vector<float>& as_slice() const noexcept { return values; }
  std::vector<float> into_vec() && { return std::move(values); }
};

/* Static model metadata (src/api.rs:47-57). */
struct ModelMeta {
  std::size_t vocab_size = 0;
  std::vector<std::uint32_t> eos_token_ids;
  std::string arch;
  std::size_t max_ctx = 0;  // allocated maximum context
};

class Engine {
 public:
  /* A safetensors model directory, or a path ending in ".gguf"
   * (Engine::load, src/api.rs:60-84). */
  static Engine load(const std::string& path, LoadOpts opts = {}) {
    if (opts.max_ctx > static_cast<std::size_t>(GROUT_MAX_CTX))
      throw Error(GROUT_EINVAL, "max_ctx " + std::to_string(opts.max_ctx) +
                                    " exceeds GROUT_MAX_CTX=" + std::to_string(GROUT_MAX_CTX));
    grout_engine* e = nullptr;
    check(grout_engine_load(path.c_str(), static_cast<int>(opts.max_ctx), opts.device_ord, &e),
          "grout_engine_load");
    grout_model_info info{};
    const int rc = grout_engine_model_info(e, &info);
    if (rc != GROUT_OK) {
      const std::string msg = std::string("grout_engine_model_info: ") + grout_last_error();
      grout_engine_destroy(e);
      throw Error(rc, msg);
    }
    ModelMeta m;
    m.vocab_size = static_cast<std::size_t>(info.config.vocab_size);
    m.eos_token_ids.assign(info.eos_token_ids, info.eos_token_ids + info.num_eos);
    m.arch = "qwen3";
    m.max_ctx = static_cast<std::size_t>(info.config.max_ctx);
    return Engine(e, std::move(m));
  }

  /* Takes ownership of an engine made by grout_engine_create /
   * grout_engine_create_q (caller-owned weights stay the caller's). */
  Engine(grout_engine* engine, ModelMeta meta) : e_(engine), meta_(std::move(meta)) {}

  Engine(const Engine&) = delete;
  Engine& operator=(const Engine&) = delete;
  Engine(Engine&& o) noexcept : e_(o.e_), meta_(std::move(o.meta_)) { o.e_ = nullptr; }
  Engine& operator=(Engine&& o) noexcept {
    if (this != &o) {
      if (e_) grout_engine_destroy(e_);
      e_ = o.e_;
      meta_ = std::move(o.meta_);
      o.e_ = nullptr;
    }
    return *this;
  }
  ~Engine() {
    if (e_) grout_engine_destroy(e_);
  }

  /* New-session prefill over `tokens`; last-token logits (src/api.rs:86-101). */
  Logits prefill(const std::vector<std::uint32_t>& tokens) {
    need();
    if (tokens.empty()) throw Error(GROUT_EINVAL, "prefill requires at least one token");
    if (tokens.size() > meta_.max_ctx)
      throw Error(GROUT_EINVAL, "prefill length " + std::to_string(tokens.size()) +
                                    " exceeds max_ctx=" + std::to_string(meta_.max_ctx));
    Logits l;
    l.values.resize(meta_.vocab_size);
    check(grout_engine_prefill(e_, tokens.data(), static_cast<int>(tokens.size()),
                               l.values.data(), nullptr),
          "grout_engine_prefill");
    return l;
  }

  /* One token into the current session; next-token logits (src/api.rs:103-114). */
  Logits decode(std::uint32_t token) {
    need();
    Logits l;
    l.values.resize(meta_.vocab_size);
    check(grout_engine_decode(e_, token, l.values.data()), "grout_engine_decode");
    return l;
  }

  /* One token; the greedy next token from the device argmax (src/api.rs:116-129). */
  std::uint32_t decode_greedy(std::uint32_t token) {
    need();
    std::uint32_t next = 0;
    check(grout_engine_decode_greedy(e_, token, &next), "grout_engine_decode_greedy");
    return next;
  }

  /* Clears the KV state and ends the session; a failure is also stashed and
   * reported by the next call (src/api.rs:131-146). */
  void reset() {
    need();
    check(grout_engine_reset(e_), "grout_engine_reset");
  }

  /* A dummy one-token prefill and decode with the first stop token, then a
   * fresh session (src/api.rs:153-162). */
  void warmup() {
    need();
    check(grout_engine_warmup(e_), "grout_engine_warmup");
  }

  const ModelMeta& meta() const noexcept { return meta_; }

  /* Position the next decode writes (the reference's next_pos). */
  std::size_t position() const {
    need();
    return static_cast<std::size_t>(grout_engine_position(e_));
  }

  grout_engine* raw() const noexcept { return e_; }

 private:
  void need() const {
    if (e_ == nullptr) throw Error(GROUT_EINVAL, "engine was moved from");
  }

  grout_engine* e_ = nullptr;
  ModelMeta meta_;
};

}  // namespace grout

#endif  // GROUT_HPP
