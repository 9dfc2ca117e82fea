// json_min.h -- a small JSON reader for the documents this library reads:
// allocator events (the ALLOCATOR_EVENTS section of a .cugraph archive) and
// graph manifests.  Values keep non-negative integers exactly as uint64;
// other numbers are kept as text.  Errors carry the byte offset.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace fdy {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  bool is_uint = false;  // Number: a non-negative integer that fits in 64 bits
  uint64_t u = 0;
  std::string s;         // String, or the text of a Number
  std::vector<Value> items;
  std::vector<std::pair<std::string, Value>> members;  // in document order

  const Value* get(const std::string& key) const {
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

class Reader {
 public:
  Reader(const char* p, size_t n) : p_(p), n_(n) {}

  // Parses one document; returns false with `error` set on failure.
  bool parse(Value& out, std::string& error) {
    i_ = 0;
    err_.clear();
    if (!value(out, 0)) {
      error = err_;
      return false;
    }
    ws();
    if (i_ != n_) {
      error = "trailing characters at byte " + std::to_string(i_);
      return false;
    }
    return true;
  }

 private:
  const char* p_;
  size_t n_;
  size_t i_ = 0;
  std::string err_;

  bool fail(const std::string& what) {
    if (err_.empty()) err_ = what + " at byte " + std::to_string(i_);
    return false;
  }
  void ws() {
    while (i_ < n_ && (p_[i_] == ' ' || p_[i_] == '\t' || p_[i_] == '\n' || p_[i_] == '\r')) ++i_;
  }
  bool lit(const char* w) {
    size_t k = 0;
    while (w[k]) {
      if (i_ + k >= n_ || p_[i_ + k] != w[k]) return fail("bad literal");
      ++k;
    }
    i_ += k;
    return true;
  }
  bool value(Value& v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (i_ >= n_) return fail("unexpected end");
    const char c = p_[i_];
    if (c == '{') return object(v, depth);
    if (c == '[') return array(v, depth);
    if (c == '"') {
      v.kind = Value::String;
      return string(v.s);
    }
    if (c == 't') {
      v.kind = Value::Bool;
      v.b = true;
      return lit("true");
    }
    if (c == 'f') {
      v.kind = Value::Bool;
      v.b = false;
      return lit("false");
    }
    if (c == 'n') {
      v.kind = Value::Null;
      return lit("null");
    }
    if (c == '-' || (c >= '0' && c <= '9')) return number(v);
    return fail("unexpected character");
  }
  bool number(Value& v) {
    v.kind = Value::Number;
    const size_t start = i_;
    bool neg = false, frac = false;
    if (p_[i_] == '-') {
      neg = true;
      ++i_;
    }
    uint64_t acc = 0;
    bool overflow = false, digits = false;
    while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') {
      const uint64_t d = (uint64_t)(p_[i_] - '0');
      if (acc > (UINT64_MAX - d) / 10) overflow = true;
      acc = acc * 10 + d;
      digits = true;
      ++i_;
    }
    if (!digits) return fail("bad number");
    if (i_ < n_ && p_[i_] == '.') {
      frac = true;
      ++i_;
      while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') ++i_;
    }
    if (i_ < n_ && (p_[i_] == 'e' || p_[i_] == 'E')) {
      frac = true;
      ++i_;
      if (i_ < n_ && (p_[i_] == '+' || p_[i_] == '-')) ++i_;
      while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') ++i_;
    }
    v.s.assign(p_ + start, i_ - start);
    v.is_uint = !neg && !frac && !overflow;
    v.u = v.is_uint ? acc : 0;
    return true;
  }
  bool string(std::string& s) {
    ++i_;  // opening quote
    s.clear();
    while (i_ < n_) {
      const char c = p_[i_++];
      if (c == '"') return true;
      if (c != '\\') {
        s.push_back(c);
        continue;
      }
      if (i_ >= n_) break;
      const char e = p_[i_++];
      switch (e) {
        case '"': s.push_back('"'); break;
        case '\\': s.push_back('\\'); break;
        case '/': s.push_back('/'); break;
        case 'b': s.push_back('\b'); break;
        case 'f': s.push_back('\f'); break;
        case 'n': s.push_back('\n'); break;
        case 'r': s.push_back('\r'); break;
        case 't': s.push_back('\t'); break;
        case 'u': {
          if (i_ + 4 > n_) return fail("bad escape");
          unsigned cp = 0;
          for (int k = 0; k < 4; ++k) {
            const char h = p_[i_++];
            cp <<= 4;
            if (h >= '0' && h <= '9') cp |= (unsigned)(h - '0');
            else if (h >= 'a' && h <= 'f') cp |= (unsigned)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') cp |= (unsigned)(h - 'A' + 10);
            else return fail("bad escape");
          }
          // UTF-8 encoding of the code unit (surrogate pairs are kept as two units).
          if (cp < 0x80) s.push_back((char)cp);
          else if (cp < 0x800) {
            s.push_back((char)(0xC0 | (cp >> 6)));
            s.push_back((char)(0x80 | (cp & 0x3F)));
          } else {
            s.push_back((char)(0xE0 | (cp >> 12)));
            s.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s.push_back((char)(0x80 | (cp & 0x3F)));
          }
          break;
        }
        default:
          return fail("bad escape");
      }
    }
    return fail("unterminated string");
  }
  bool array(Value& v, int depth) {
    v.kind = Value::Array;
    ++i_;
    ws();
    if (i_ < n_ && p_[i_] == ']') {
      ++i_;
      return true;
    }
    for (;;) {
      v.items.emplace_back();
      if (!value(v.items.back(), depth + 1)) return false;
      ws();
      if (i_ >= n_) return fail("unterminated array");
      if (p_[i_] == ',') {
        ++i_;
        continue;
      }
      if (p_[i_] == ']') {
        ++i_;
        return true;
      }
      return fail("expected ',' or ']'");
    }
  }
  bool object(Value& v, int depth) {
    v.kind = Value::Object;
    ++i_;
    ws();
    if (i_ < n_ && p_[i_] == '}') {
      ++i_;
      return true;
    }
    for (;;) {
      ws();
      if (i_ >= n_ || p_[i_] != '"') return fail("expected a key");
      std::string key;
      if (!string(key)) return false;
      ws();
      if (i_ >= n_ || p_[i_] != ':') return fail("expected ':'");
      ++i_;
      v.members.emplace_back(std::move(key), Value{});
      if (!value(v.members.back().second, depth + 1)) return false;
      ws();
      if (i_ >= n_) return fail("unterminated object");
      if (p_[i_] == ',') {
        ++i_;
        continue;
      }
      if (p_[i_] == '}') {
        ++i_;
        return true;
      }
      return fail("expected ',' or '}'");
    }
  }
};

}  // namespace json
}  // namespace fdy
