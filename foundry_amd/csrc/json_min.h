// json_min.h -- a small JSON reader for the documents this library reads:
// allocator events (the ALLOCATOR_EVENTS section of a .cugraph archive),
// graph manifests and graph documents (the .json a graph is saved as).
// Numbers are classified as a JSON library with 64-bit integers does it:
// an integer literal that fits int64 is a signed integer, one that fits
// only uint64 is unsigned, anything else (fraction, exponent, overflow) is
// a double; the text is kept too.  Strings are well-formed UTF-8 (a \u
// surrogate pair becomes one 4-byte sequence; lone surrogates, raw control
// characters and malformed sequences are errors); numbers follow the JSON
// grammar (no leading zeros, digits after '.' and after 'e').  Errors carry
// the byte offset.
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
  enum NumKind { Int, Uint, Double };
  bool b = false;
  NumKind num = Int;     // Number: its class
  bool is_uint = false;  // Number: a non-negative integer that fits in 64 bits
  uint64_t u = 0;
  int64_t i = 0;         // Number of class Int
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
    if (i_ + 1 < n_ && p_[i_] == '0' && p_[i_ + 1] >= '0' && p_[i_ + 1] <= '9') return fail("leading zero");
    while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') {
      const uint64_t d = (uint64_t)(p_[i_] - '0');
      if (acc > (UINT64_MAX - d) / 10) overflow = true;
      acc = acc * 10 + d;
      digits = true;
      ++i_;
    }
    if (!digits) return fail("bad number");
    auto digit_run = [&]() {
      const size_t d0 = i_;
      while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') ++i_;
      return i_ > d0;
    };
    if (i_ < n_ && p_[i_] == '.') {
      frac = true;
      ++i_;
      if (!digit_run()) return fail("bad number");
    }
    if (i_ < n_ && (p_[i_] == 'e' || p_[i_] == 'E')) {
      frac = true;
      ++i_;
      if (i_ < n_ && (p_[i_] == '+' || p_[i_] == '-')) ++i_;
      if (!digit_run()) return fail("bad number");
    }
    v.s.assign(p_ + start, i_ - start);
    v.is_uint = !neg && !frac && !overflow;
    v.u = v.is_uint ? acc : 0;
    if (frac || overflow || (neg && acc > (1ull << 63))) {
      v.num = Value::Double;
    } else if (neg) {
      v.num = Value::Int;
      v.i = acc == (1ull << 63) ? INT64_MIN : -(int64_t)acc;
    } else if (acc <= (uint64_t)INT64_MAX) {
      v.num = Value::Int;
      v.i = (int64_t)acc;
    } else {
      v.num = Value::Uint;
    }
    return true;
  }
  bool string(std::string& s) {
    ++i_;  // opening quote
    s.clear();
    while (i_ < n_) {
      const char c = p_[i_++];
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) {
        --i_;
        return fail("control character in string");
      }
      if (c != '\\') {
        const unsigned char u = (unsigned char)c;
        if (u >= 0x80) {  // one UTF-8 sequence, checked whole
          --i_;
          const size_t len = utf8_len();
          if (!len) return fail("invalid UTF-8");
          s.append(p_ + i_, len);
          i_ += len;
          continue;
        }
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
          unsigned cp = 0;
          if (!hex4(cp)) return fail("bad escape");
          if (cp >= 0xDC00 && cp <= 0xDFFF) return fail("lone low surrogate");
          if (cp >= 0xD800 && cp <= 0xDBFF) {  // a high surrogate needs its low half
            unsigned lo = 0;
            if (i_ + 2 > n_ || p_[i_] != '\\' || p_[i_ + 1] != 'u') return fail("lone high surrogate");
            i_ += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo > 0xDFFF) return fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          if (cp < 0x80) s.push_back((char)cp);
          else if (cp < 0x800) {
            s.push_back((char)(0xC0 | (cp >> 6)));
            s.push_back((char)(0x80 | (cp & 0x3F)));
          } else if (cp < 0x10000) {
            s.push_back((char)(0xE0 | (cp >> 12)));
            s.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s.push_back((char)(0x80 | (cp & 0x3F)));
          } else {
            s.push_back((char)(0xF0 | (cp >> 18)));
            s.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
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
  // Length of the well-formed UTF-8 sequence at i_ (shortest form, no
  // surrogates, at most U+10FFFF), or 0.
  size_t utf8_len() const {
    const unsigned char* q = reinterpret_cast<const unsigned char*>(p_ + i_);
    const size_t left = n_ - i_;
    auto cont = [&](size_t k) { return k < left && (q[k] & 0xC0) == 0x80; };
    if (q[0] >= 0xC2 && q[0] <= 0xDF) return cont(1) ? 2 : 0;
    if (q[0] >= 0xE0 && q[0] <= 0xEF) {
      if (!cont(1) || !cont(2)) return 0;
      if (q[0] == 0xE0 && q[1] < 0xA0) return 0;  // overlong
      if (q[0] == 0xED && q[1] >= 0xA0) return 0;  // surrogate
      return 3;
    }
    if (q[0] >= 0xF0 && q[0] <= 0xF4) {
      if (!cont(1) || !cont(2) || !cont(3)) return 0;
      if (q[0] == 0xF0 && q[1] < 0x90) return 0;  // overlong
      if (q[0] == 0xF4 && q[1] >= 0x90) return 0;  // past U+10FFFF
      return 4;
    }
    return 0;
  }
  bool hex4(unsigned& cp) {
    if (i_ + 4 > n_) return false;
    cp = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = p_[i_++];
      cp <<= 4;
      if (h >= '0' && h <= '9') cp |= (unsigned)(h - '0');
      else if (h >= 'a' && h <= 'f') cp |= (unsigned)(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') cp |= (unsigned)(h - 'A' + 10);
      else return false;
    }
    return true;
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
