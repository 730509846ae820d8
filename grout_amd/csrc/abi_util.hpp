// Host-side helpers shared by the C ABI sources: the thread-local error
// message, status conversion and the argument checks every entry point runs
// before it launches anything (the reference's `ensure!` checks).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <initializer_list>
#include <string>
#include <utility>

#include "../../include/grout_attn.h"

namespace grout_abi {

inline thread_local std::string g_last_error;

inline int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

inline int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return GROUT_OK;
  fail((int)e, "%s: %s", what, hipGetErrorString(e));
  return (int)e;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int check_heads(int hq, int hkv, int head_dim, int max_group) {
  if (head_dim != 128)
    return fail(GROUT_ENOTSUP, "head_dim=%d: only 128 is supported (src/model.rs:1446)", head_dim);
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0)
    return fail(GROUT_EINVAL, "num_q_heads=%d must be a positive multiple of num_kv_heads=%d", hq,
                hkv);
  if (hq / hkv > max_group)
    return fail(GROUT_ENOTSUP, "GQA group %d exceeds %d", hq / hkv, max_group);
  return GROUT_OK;
}

#define GROUT_CHECK(expr)            \
  do {                               \
    const int _rc = (expr);          \
    if (_rc != GROUT_OK) return _rc; \
  } while (0)

#define GROUT_NEED(cond, code, ...)                \
  do {                                             \
    if (!(cond)) return ::grout_abi::fail((code), __VA_ARGS__); \
  } while (0)

inline int check_ptrs16(std::initializer_list<std::pair<const void*, const char*>> ptrs) {
  for (const auto& p : ptrs) {
    if (p.first == nullptr) return fail(GROUT_EINVAL, "%s is NULL", p.second);
    if (!aligned16(p.first)) return fail(GROUT_EALIGN, "%s is not 16-byte aligned", p.second);
  }
  return GROUT_OK;
}

inline int check_stride(long kv_head_stride, long min_rows) {
  GROUT_NEED(min_rows <= GROUT_MAX_CTX, GROUT_ENOTSUP,
             "cache length %ld exceeds GROUT_MAX_CTX=%d (32-bit row offsets)", min_rows,
             GROUT_MAX_CTX);
  GROUT_NEED(kv_head_stride % 8 == 0, GROUT_EALIGN,
             "kv_head_stride=%ld elements is not a multiple of 8 (16 bytes)", kv_head_stride);
  GROUT_NEED(kv_head_stride >= min_rows * 128, GROUT_EINVAL,
             "kv_head_stride=%ld is smaller than %ld rows of 128", kv_head_stride, min_rows);
  return GROUT_OK;
}

constexpr int kMaxDecodeGroup = 16;
constexpr int kMaxSplits = GROUT_MAX_SPLITS;

// Workspace layout: part_acc [Hkv][splits][G][128] f32 | part_ml [Hkv][splits][G][2] f32.
inline size_t decode_ws_bytes(int hq, int hkv, int nsplit) {
  const size_t g = (size_t)(hq / hkv);
  return (size_t)hkv * nsplit * g * (128 + 2) * sizeof(float);
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// A boolean switch's value as the reference's env_bool_or reads one
// (src/model.rs:212-224): surrounding whitespace trimmed, case ignored,
// "1"/"true"/"on"/"yes" on, "0"/"false"/"off"/"no"/"" off, anything else (or
// an unset variable, raw == NULL) the default.
inline bool parse_bool_or(const char* raw, bool dflt) {
  if (raw == nullptr) return dflt;
  std::string v(raw);
  const char* ws = " \t\n\r\f\v";
  const size_t b = v.find_first_not_of(ws);
  if (b == std::string::npos) return false;
  v = v.substr(b, v.find_last_not_of(ws) - b + 1);
  for (char& c : v)
    if (c >= 'A' && c <= 'Z') c = (char)(c - 'A' + 'a');
  if (v == "1" || v == "true" || v == "on" || v == "yes") return true;
  if (v == "0" || v == "false" || v == "off" || v == "no") return false;
  return dflt;
}

// A positive integer setting as the reference's env_usize_or reads one
// (src/model.rs:204-210, Rust's usize parsing): an optional '+' and decimal
// digits, nothing else (no whitespace); zero, a value past 2^63 - 1 (the
// result is a long), anything else or an unset variable (raw == NULL) give
// the default.
inline long parse_usize_or(const char* raw, long dflt) {
  if (raw == nullptr) return dflt;
  const char* c = raw;
  if (*c == '+') ++c;
  if (*c == '\0') return dflt;
  unsigned long long v = 0;
  for (; *c; ++c) {
    if (*c < '0' || *c > '9') return dflt;
    if (v > (~0ULL - 9) / 10) return dflt;  // past 64 bits: Rust's parse fails
    v = v * 10 + (unsigned long long)(*c - '0');
  }
  if (v == 0) return dflt;
  return v > (unsigned long long)0x7fffffffffffffffLL ? dflt : (long)v;
}

}  // namespace grout_abi
