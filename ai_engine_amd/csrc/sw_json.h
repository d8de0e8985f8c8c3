// sw_json.h -- a small JSON reader for the .sw container's graph
// (crates/ai-core/src/format/model.rs:1-404 defines the schema; the reference
// reads it with serde_json). Builds a value tree; numbers are kept as double
// (every integer in a .sw graph is a u32/u64 offset well inside 2^53) and
// the text of the number is not kept. Unknown fields are simply present in
// the tree and ignored by the reader, as serde does (model.rs:393-401).
#pragma once

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace aih {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;

  bool is_null() const { return kind == Null; }
  bool has(const char *k) const {
    if (kind != Object) return false;
    for (auto &kv : obj)
      if (kv.first == k) return true;
    return false;
  }
  const Value &operator[](const char *k) const {
    if (kind != Object) throw std::runtime_error(std::string("json: not an object looking for '") + k + "'");
    for (auto &kv : obj)
      if (kv.first == k) return kv.second;
    throw std::runtime_error(std::string("json: missing field '") + k + "'");
  }
  const Value &at(size_t i) const {
    if (kind != Array || i >= arr.size()) throw std::runtime_error("json: array index out of range");
    return arr[i];
  }
  size_t size() const { return kind == Array ? arr.size() : kind == Object ? obj.size() : 0; }
  uint64_t u64() const {
    // range first: converting a double at or above 2^64 (or NaN) to an
    // integer is undefined behaviour
    if (kind != Number || !(num >= 0.0 && num < 18446744073709551616.0) || num != (double)(uint64_t)num)
      throw std::runtime_error("json: expected an unsigned integer");
    return (uint64_t)num;
  }
  uint32_t u32() const {
    const uint64_t v = u64();
    if (v > 0xffffffffull) throw std::runtime_error("json: integer above u32");
    return (uint32_t)v;
  }
  float f32() const {
    if (kind != Number) throw std::runtime_error("json: expected a number");
    return (float)num;
  }
  const std::string &s() const {
    if (kind != String) throw std::runtime_error("json: expected a string");
    return str;
  }
};

class Parser {
 public:
  Parser(const char *p, size_t n) : p_(p), end_(p + n) {}

  Value parse() {
    Value v = value(0);
    ws();
    if (p_ != end_) fail("trailing characters");
    return v;
  }

 private:
  const char *p_, *end_;

  [[noreturn]] void fail(const char *what) { throw std::runtime_error(std::string("json: ") + what); }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
  }
  bool lit(const char *s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end_ - p_) >= n && std::memcmp(p_, s, n) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }
  Value value(int depth) {
    if (depth > 64) fail("nesting too deep");
    ws();
    if (p_ >= end_) fail("unexpected end");
    Value v;
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = Value::Object;
      ws();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return v;
      }
      for (;;) {
        ws();
        if (p_ >= end_ || *p_ != '"') fail("expected a key");
        std::string k = string();
        ws();
        if (p_ >= end_ || *p_ != ':') fail("expected ':'");
        ++p_;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          ++p_;
          return v;
        }
        fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = Value::Array;
      ws();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return v;
      }
      for (;;) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          ++p_;
          return v;
        }
        fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Value::String;
      v.str = string();
      return v;
    }
    if (lit("true")) {
      v.kind = Value::Bool;
      v.b = true;
      return v;
    }
    if (lit("false")) {
      v.kind = Value::Bool;
      return v;
    }
    if (lit("null")) return v;
    if (c == '-' || (c >= '0' && c <= '9')) {
      const char *q = p_;
      if (*q == '-') ++q;
      while (q < end_ && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' || *q == '+' || *q == '-'))
        ++q;
      const std::string t(p_, q);
      char *e = nullptr;
      v.kind = Value::Number;
      v.num = std::strtod(t.c_str(), &e);
      if (!e || *e) fail("bad number");
      p_ = q;
      return v;
    }
    fail("unexpected character");
  }
  // string with the escapes JSON defines; \u escapes become UTF-8
  std::string string() {
    ++p_;  // opening quote
    std::string out;
    while (p_ < end_ && *p_ != '"') {
      char c = *p_++;
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (p_ >= end_) fail("bad escape");
      c = *p_++;
      switch (c) {
        case '"': out.push_back('"'); break;
        case '\\': out.push_back('\\'); break;
        case '/': out.push_back('/'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          if (end_ - p_ < 4) fail("bad \\u escape");
          uint32_t cp = (uint32_t)std::strtoul(std::string(p_, p_ + 4).c_str(), nullptr, 16);
          p_ += 4;
          if (cp >= 0xD800 && cp <= 0xDBFF && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            const uint32_t lo = (uint32_t)std::strtoul(std::string(p_ + 2, p_ + 6).c_str(), nullptr, 16);
            if (lo >= 0xDC00 && lo <= 0xDFFF) {
              cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
              p_ += 6;
            }
          }
          if (cp < 0x80) {
            out.push_back((char)cp);
          } else if (cp < 0x800) {
            out.push_back((char)(0xC0 | (cp >> 6)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
          } else if (cp < 0x10000) {
            out.push_back((char)(0xE0 | (cp >> 12)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
          } else {
            out.push_back((char)(0xF0 | (cp >> 18)));
            out.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
          }
          break;
        }
        default: fail("bad escape");
      }
    }
    if (p_ >= end_) fail("unterminated string");
    ++p_;  // closing quote
    return out;
  }
};

inline Value parse(const char *p, size_t n) { return Parser(p, n).parse(); }

}  // namespace json
}  // namespace aih
