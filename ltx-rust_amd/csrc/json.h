// Minimal JSON reader for safetensors headers (RFC 8259 syntax; numbers are
// kept as their source text and converted on demand).
#pragma once

#include <stdint.h>

#include <string>
#include <utility>
#include <vector>

namespace ltxw {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  std::string text;  // String: decoded UTF-8; Number: the literal
  std::vector<Value> items;
  std::vector<std::pair<std::string, Value>> members;  // in document order

  const Value* get(const std::string& key) const {
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
  // Non-negative integer literal (no sign, fraction or exponent) that fits u64.
  bool as_u64(uint64_t* out) const {
    if (kind != Number || text.empty() || text[0] == '-') return false;
    uint64_t v = 0;
    for (char c : text) {
      if (c < '0' || c > '9') return false;
      uint64_t d = (uint64_t)(c - '0');
      if (v > (UINT64_MAX - d) / 10) return false;
      v = v * 10 + d;
    }
    *out = v;
    return true;
  }
};

// True when [p, p+n) is well-formed UTF-8 (no overlongs, surrogates or > U+10FFFF).
inline bool valid_utf8(const unsigned char* p, size_t n) {
  size_t i = 0;
  while (i < n) {
    unsigned c = p[i];
    if (c < 0x80) { ++i; continue; }
    size_t len;
    uint32_t cp;
    if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
    else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
    else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
    else return false;
    if (i + len > n) return false;
    for (size_t k = 1; k < len; ++k) {
      if ((p[i + k] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (p[i + k] & 0x3F);
    }
    if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000)) return false;
    if (cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
    i += len;
  }
  return true;
}

class Parser {
 public:
  Parser(const char* p, size_t n) : p_(p), n_(n) {}

  // Parses one document (trailing whitespace allowed). On failure returns
  // false and sets *err to a message with the byte offset.
  bool parse(Value* out, std::string* err) {
    skip_ws();
    if (!value(out, 0)) { *err = err_ + " at byte " + std::to_string(i_); return false; }
    skip_ws();
    if (i_ != n_) { *err = "trailing characters at byte " + std::to_string(i_); return false; }
    return true;
  }

 private:
  static constexpr int kMaxDepth = 64;
  const char* p_;
  size_t n_;
  size_t i_ = 0;
  std::string err_;

  bool fail(const char* m) { err_ = m; return false; }
  void skip_ws() {
    while (i_ < n_ && (p_[i_] == ' ' || p_[i_] == '\t' || p_[i_] == '\n' || p_[i_] == '\r')) ++i_;
  }
  bool lit(const char* s) {
    size_t k = 0;
    while (s[k]) {
      if (i_ + k >= n_ || p_[i_ + k] != s[k]) return fail("invalid literal");
      ++k;
    }
    i_ += k;
    return true;
  }
  static void put_utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) s += (char)cp;
    else if (cp < 0x800) { s += (char)(0xC0 | (cp >> 6)); s += (char)(0x80 | (cp & 0x3F)); }
    else if (cp < 0x10000) {
      s += (char)(0xE0 | (cp >> 12)); s += (char)(0x80 | ((cp >> 6) & 0x3F)); s += (char)(0x80 | (cp & 0x3F));
    } else {
      s += (char)(0xF0 | (cp >> 18)); s += (char)(0x80 | ((cp >> 12) & 0x3F));
      s += (char)(0x80 | ((cp >> 6) & 0x3F)); s += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t* v) {
    if (i_ + 4 > n_) return fail("truncated \\u escape");
    uint32_t r = 0;
    for (int k = 0; k < 4; ++k) {
      char c = p_[i_ + k];
      r <<= 4;
      if (c >= '0' && c <= '9') r |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') r |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') r |= (uint32_t)(c - 'A' + 10);
      else return fail("invalid \\u escape");
    }
    i_ += 4;
    *v = r;
    return true;
  }
  bool string(std::string* s) {
    if (i_ >= n_ || p_[i_] != '"') return fail("expected string");
    ++i_;
    s->clear();
    while (true) {
      if (i_ >= n_) return fail("unterminated string");
      unsigned char c = (unsigned char)p_[i_++];
      if (c == '"') return true;
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') { *s += (char)c; continue; }
      if (i_ >= n_) return fail("unterminated escape");
      char e = p_[i_++];
      switch (e) {
        case '"': *s += '"'; break;
        case '\\': *s += '\\'; break;
        case '/': *s += '/'; break;
        case 'b': *s += '\b'; break;
        case 'f': *s += '\f'; break;
        case 'n': *s += '\n'; break;
        case 'r': *s += '\r'; break;
        case 't': *s += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp <= 0xDBFF) {
            uint32_t lo;
            if (i_ + 2 > n_ || p_[i_] != '\\' || p_[i_ + 1] != 'u') return fail("unpaired surrogate");
            i_ += 2;
            if (!hex4(&lo)) return false;
            if (lo < 0xDC00 || lo > 0xDFFF) return fail("unpaired surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
            return fail("unpaired surrogate");
          }
          put_utf8(*s, cp);
          break;
        }
        default: return fail("invalid escape");
      }
    }
  }
  bool number(Value* v) {
    size_t b = i_;
    if (i_ < n_ && p_[i_] == '-') ++i_;
    if (i_ >= n_) return fail("truncated number");
    if (p_[i_] == '0') ++i_;
    else if (p_[i_] >= '1' && p_[i_] <= '9') while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') ++i_;
    else return fail("invalid number");
    if (i_ < n_ && p_[i_] == '.') {
      ++i_;
      if (i_ >= n_ || p_[i_] < '0' || p_[i_] > '9') return fail("invalid fraction");
      while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') ++i_;
    }
    if (i_ < n_ && (p_[i_] == 'e' || p_[i_] == 'E')) {
      ++i_;
      if (i_ < n_ && (p_[i_] == '+' || p_[i_] == '-')) ++i_;
      if (i_ >= n_ || p_[i_] < '0' || p_[i_] > '9') return fail("invalid exponent");
      while (i_ < n_ && p_[i_] >= '0' && p_[i_] <= '9') ++i_;
    }
    v->kind = Value::Number;
    v->text.assign(p_ + b, i_ - b);
    return true;
  }
  bool value(Value* v, int depth) {
    if (depth > kMaxDepth) return fail("nesting too deep");
    if (i_ >= n_) return fail("unexpected end of input");
    char c = p_[i_];
    if (c == '{') {
      ++i_;
      v->kind = Value::Object;
      skip_ws();
      if (i_ < n_ && p_[i_] == '}') { ++i_; return true; }
      while (true) {
        skip_ws();
        std::string key;
        if (!string(&key)) return false;
        skip_ws();
        if (i_ >= n_ || p_[i_] != ':') return fail("expected ':'");
        ++i_;
        skip_ws();
        v->members.emplace_back(std::move(key), Value());
        if (!value(&v->members.back().second, depth + 1)) return false;
        skip_ws();
        if (i_ < n_ && p_[i_] == ',') { ++i_; continue; }
        if (i_ < n_ && p_[i_] == '}') { ++i_; return true; }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++i_;
      v->kind = Value::Array;
      skip_ws();
      if (i_ < n_ && p_[i_] == ']') { ++i_; return true; }
      while (true) {
        skip_ws();
        v->items.emplace_back();
        if (!value(&v->items.back(), depth + 1)) return false;
        skip_ws();
        if (i_ < n_ && p_[i_] == ',') { ++i_; continue; }
        if (i_ < n_ && p_[i_] == ']') { ++i_; return true; }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') { v->kind = Value::String; return string(&v->text); }
    if (c == 't') { v->kind = Value::Bool; v->b = true; return lit("true"); }
    if (c == 'f') { v->kind = Value::Bool; v->b = false; return lit("false"); }
    if (c == 'n') { v->kind = Value::Null; return lit("null"); }
    return number(v);
  }
};

}  // namespace json
}  // namespace ltxw
