// qnn_json.h -- the JSON subset the checkpoint formats need (host only).
//
// Safetensors headers, shard indexes and the INT4 cache's headers are JSON
// objects.  Value keeps object members in file order, duplicates included
// (the safetensors reader rejects duplicate tensor names itself), and keeps a
// number's literal text so integer fields can be read exactly.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace qnn {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  std::string text;  // String: decoded UTF-8; Number: the literal as written
  std::vector<Value> items;                           // Array
  std::vector<std::pair<std::string, Value>> members;  // Object, in order

  bool is_object() const { return kind == Object; }
  bool is_array() const { return kind == Array; }
  bool is_string() const { return kind == String; }
  bool is_number() const { return kind == Number; }
  // First member named `key`, or nullptr.
  const Value *get(const std::string &key) const {
    if (kind != Object) return nullptr;
    for (const auto &m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
  // Dotted path lookup through nested objects ("metadata.format").
  const Value *path(const std::string &dotted) const {
    const Value *v = this;
    size_t pos = 0;
    while (v) {
      const size_t dot = dotted.find('.', pos);
      v = v->get(dotted.substr(pos, dot == std::string::npos ? std::string::npos : dot - pos));
      if (dot == std::string::npos) break;
      pos = dot + 1;
    }
    return v;
  }
  std::string string_at(const std::string &dotted, const std::string &dflt = "") const {
    const Value *v = path(dotted);
    return v && v->kind == String ? v->text : dflt;
  }
  // The number's literal as a whole int64 (no fraction, exponent or overflow).
  bool to_int64(int64_t &out) const {
    if (kind != Number || text.empty()) return false;
    const char *s = text.c_str();
    bool neg = *s == '-';
    if (neg) ++s;
    if (!*s) return false;
    uint64_t acc = 0;
    for (; *s; ++s) {
      if (*s < '0' || *s > '9') return false;
      const uint64_t d = uint64_t(*s - '0');
      if (acc > (UINT64_MAX - d) / 10) return false;
      acc = acc * 10 + d;
    }
    if (!neg && acc > uint64_t(INT64_MAX)) return false;
    if (neg && acc > uint64_t(INT64_MAX) + 1) return false;
    out = neg ? int64_t(0 - acc) : int64_t(acc);
    return true;
  }
};

class Parser {
 public:
  Parser(const char *p, size_t n) : p_(p), end_(p + n) {}
  // Parses one value followed only by whitespace; false on any error.
  bool parse(Value &out) {
    ws();
    if (!value(out, 0)) return false;
    ws();
    return p_ == end_;
  }

 private:
  const char *p_, *end_;
  static constexpr int kMaxDepth = 512;

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char *w) {
    const size_t n = std::strlen(w);
    if (size_t(end_ - p_) < n || std::memcmp(p_, w, n) != 0) return false;
    p_ += n;
    return true;
  }
  bool value(Value &v, int depth) {
    if (p_ >= end_ || depth > kMaxDepth) return false;
    switch (*p_) {
      case '{': return object(v, depth);
      case '[': return array(v, depth);
      case '"': v.kind = Value::String; return string(v.text);
      case 't': v.kind = Value::Bool; v.b = true; return lit("true");
      case 'f': v.kind = Value::Bool; v.b = false; return lit("false");
      case 'n': v.kind = Value::Null; return lit("null");
      default: return number(v);
    }
  }
  bool object(Value &v, int depth) {
    v.kind = Value::Object;
    ++p_;
    ws();
    if (p_ < end_ && *p_ == '}') { ++p_; return true; }
    for (;;) {
      ws();
      std::string key;
      if (p_ >= end_ || *p_ != '"' || !string(key)) return false;
      ws();
      if (p_ >= end_ || *p_ != ':') return false;
      ++p_;
      ws();
      v.members.emplace_back(std::move(key), Value());
      if (!value(v.members.back().second, depth + 1)) return false;
      ws();
      if (p_ >= end_) return false;
      if (*p_ == ',') { ++p_; continue; }
      if (*p_ == '}') { ++p_; return true; }
      return false;
    }
  }
  bool array(Value &v, int depth) {
    v.kind = Value::Array;
    ++p_;
    ws();
    if (p_ < end_ && *p_ == ']') { ++p_; return true; }
    for (;;) {
      ws();
      v.items.emplace_back();
      if (!value(v.items.back(), depth + 1)) return false;
      ws();
      if (p_ >= end_) return false;
      if (*p_ == ',') { ++p_; continue; }
      if (*p_ == ']') { ++p_; return true; }
      return false;
    }
  }
  bool number(Value &v) {
    const char *s = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_) return false;
    if (*p_ == '0') {
      ++p_;
    } else if (*p_ >= '1' && *p_ <= '9') {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    } else {
      return false;
    }
    if (p_ < end_ && *p_ == '.') {
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    v.kind = Value::Number;
    v.text.assign(s, p_);
    return true;
  }
  static void put_utf8(std::string &o, uint32_t c) {
    if (c < 0x80) {
      o += char(c);
    } else if (c < 0x800) {
      o += char(0xC0 | (c >> 6));
      o += char(0x80 | (c & 63));
    } else if (c < 0x10000) {
      o += char(0xE0 | (c >> 12));
      o += char(0x80 | ((c >> 6) & 63));
      o += char(0x80 | (c & 63));
    } else {
      o += char(0xF0 | (c >> 18));
      o += char(0x80 | ((c >> 12) & 63));
      o += char(0x80 | ((c >> 6) & 63));
      o += char(0x80 | (c & 63));
    }
  }
  bool hex4(uint32_t &c) {
    if (end_ - p_ < 4) return false;
    c = 0;
    for (int i = 0; i < 4; ++i) {
      const char h = *p_++;
      c <<= 4;
      if (h >= '0' && h <= '9') c |= uint32_t(h - '0');
      else if (h >= 'a' && h <= 'f') c |= uint32_t(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') c |= uint32_t(h - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string &o) {
    ++p_;  // opening quote
    while (p_ < end_) {
      const unsigned char c = static_cast<unsigned char>(*p_);
      if (c == '"') { ++p_; return true; }
      if (c < 0x20) return false;
      if (c != '\\') { o += char(c); ++p_; continue; }
      if (++p_ >= end_) return false;
      const char e = *p_++;
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {
            uint32_t lo;
            if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return false;
            p_ += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return false;
          }
          put_utf8(o, cp);
          break;
        }
        default: return false;
      }
    }
    return false;
  }
};

// Strict UTF-8: no overlong forms, surrogates or code points above U+10FFFF.
inline bool valid_utf8(const char *s, size_t n) {
  const unsigned char *p = reinterpret_cast<const unsigned char *>(s), *e = p + n;
  while (p < e) {
    const unsigned c = *p;
    if (c < 0x80) { ++p; continue; }
    int len;
    uint32_t cp, min;
    if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; min = 0x80; }
    else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; min = 0x800; }
    else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; min = 0x10000; }
    else return false;
    if (e - p < len) return false;
    for (int i = 1; i < len; ++i) {
      if ((p[i] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (p[i] & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp < 0xE000)) return false;
    p += len;
  }
  return true;
}

// JSON string literal of s (UTF-8 passed through; quotes, backslashes and
// control characters escaped).
inline std::string quote(const std::string &s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    if (c == '"') o += "\\\"";
    else if (c == '\\') o += "\\\\";
    else if (c < 0x20) {
      static const char *hex = "0123456789abcdef";
      o += "\\u00";
      o += hex[c >> 4];
      o += hex[c & 15];
    } else {
      o += char(c);
    }
  }
  return o + "\"";
}

}  // namespace json
}  // namespace qnn
