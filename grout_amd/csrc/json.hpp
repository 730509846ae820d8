// Minimal JSON reader for model metadata (config.json, the safetensors shard
// index and safetensors headers).  The input is untrusted: every read is
// bounds-checked, nesting is limited, and any malformed text yields an error
// message instead of a value.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace grout_json {

struct Value {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  bool b = false;
  double num = 0.0;
  bool is_int = false;     // the number had no fraction or exponent
  int64_t i = 0;           // exact value when is_int and in range
  std::string str;
  std::vector<Value> arr;
  std::map<std::string, Value> obj;

  const Value* get(const std::string& key) const {
    if (kind != kObject) return nullptr;
    auto it = obj.find(key);
    return it == obj.end() ? nullptr : &it->second;
  }
};

class Parser {
 public:
  Parser(const char* p, size_t n) : p_(p), end_(p + n) {}

  // Parses one document; false with error() set on malformed input.
  bool parse(Value& out) {
    skip_ws();
    if (!value(out, 0)) return false;
    skip_ws();
    if (p_ != end_) return fail("trailing characters after the JSON value");
    return true;
  }
  const std::string& error() const { return err_; }

 private:
  static constexpr int kMaxDepth = 64;
  const char* p_;
  const char* end_;
  std::string err_;

  bool fail(const char* msg) {
    if (err_.empty()) err_ = msg;
    return false;
  }
  void skip_ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool literal(const char* word) {
    const char* q = p_;
    for (; *word; ++word, ++q)
      if (q >= end_ || *q != *word) return fail("invalid literal");
    p_ = q;
    return true;
  }
  bool value(Value& v, int depth) {
    if (depth > kMaxDepth) return fail("JSON nested too deeply");
    if (p_ >= end_) return fail("unexpected end of JSON");
    switch (*p_) {
      case '{': return object(v, depth);
      case '[': return array(v, depth);
      case '"': v.kind = Value::kString; return string(v.str);
      case 't': v.kind = Value::kBool; v.b = true; return literal("true");
      case 'f': v.kind = Value::kBool; v.b = false; return literal("false");
      case 'n': v.kind = Value::kNull; return literal("null");
      default: return number(v);
    }
  }
  bool object(Value& v, int depth) {
    v.kind = Value::kObject;
    ++p_;  // '{'
    skip_ws();
    if (p_ < end_ && *p_ == '}') {
      ++p_;
      return true;
    }
    for (;;) {
      skip_ws();
      if (p_ >= end_ || *p_ != '"') return fail("expected a string key");
      std::string key;
      if (!string(key)) return false;
      skip_ws();
      if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
      ++p_;
      skip_ws();
      Value child;
      if (!value(child, depth + 1)) return false;
      v.obj[key] = std::move(child);
      skip_ws();
      if (p_ >= end_) return fail("unterminated object");
      if (*p_ == ',') {
        ++p_;
        continue;
      }
      if (*p_ == '}') {
        ++p_;
        return true;
      }
      return fail("expected ',' or '}'");
    }
  }
  bool array(Value& v, int depth) {
    v.kind = Value::kArray;
    ++p_;  // '['
    skip_ws();
    if (p_ < end_ && *p_ == ']') {
      ++p_;
      return true;
    }
    for (;;) {
      skip_ws();
      Value child;
      if (!value(child, depth + 1)) return false;
      v.arr.push_back(std::move(child));
      skip_ws();
      if (p_ >= end_) return fail("unterminated array");
      if (*p_ == ',') {
        ++p_;
        continue;
      }
      if (*p_ == ']') {
        ++p_;
        return true;
      }
      return fail("expected ',' or ']'");
    }
  }
  static int hexval(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }
  void put_utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xC0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += (char)(0xE0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    } else {
      s += (char)(0xF0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3F));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& cp) {
    if (end_ - p_ < 4) return fail("truncated \\u escape");
    cp = 0;
    for (int k = 0; k < 4; ++k) {
      const int h = hexval(p_[k]);
      if (h < 0) return fail("invalid \\u escape");
      cp = cp * 16 + (uint32_t)h;
    }
    p_ += 4;
    return true;
  }
  bool string(std::string& s) {
    ++p_;  // opening quote
    for (;;) {
      if (p_ >= end_) return fail("unterminated string");
      const char c = *p_++;
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return fail("control character in string");
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
            p_ += 2;
            uint32_t lo;
            if (!hex4(lo)) return false;
            if (lo < 0xDC00 || lo >= 0xE000) return fail("invalid surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return fail("lone surrogate");
          }
          put_utf8(s, cp);
          break;
        }
        default: return fail("invalid escape");
      }
    }
  }
  bool number(Value& v) {
    const char* start = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("invalid value");
    if (*p_ == '0') {
      ++p_;
    } else {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    bool integral = true;
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      ++p_;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("invalid number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("invalid number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    const std::string text(start, p_);
    v.kind = Value::kNumber;
    v.num = std::strtod(text.c_str(), nullptr);
    v.is_int = false;
    if (integral && text.size() <= 18) {  // fits int64 exactly
      v.is_int = true;
      v.i = std::strtoll(text.c_str(), nullptr, 10);
    }
    return true;
  }
};

}  // namespace grout_json
