// A small JSON reader (host only): a DOM of null / bool / number / string / array / object, enough for safetensors
// headers, config.json and tokenizer.json. Numbers keep an exact u64 when they are non-negative integer literals.
// Strings are UTF-8 (\u escapes, surrogate pairs joined); objects keep their keys in file order.
#pragma once
#include <stdint.h>

#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace moert {

struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0.0;
  bool is_uint = false;  // a non-negative integer literal that fits u64 exactly
  uint64_t u = 0;
  std::string s;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal* get(const std::string& k) const {
    if (kind != OBJ) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  JParser(const char* p, size_t n) : p_(p), end_(p + n) {}
  bool parse(JVal& v, std::string& err) {
    if (!value(v, 0)) {
      err = err_.empty() ? "malformed JSON" : err_;
      return false;
    }
    ws();
    if (p_ != end_) {
      err = "trailing bytes after the JSON value";
      return false;
    }
    return true;
  }

 private:
  const char* p_;
  const char* end_;
  std::string err_;
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
  }
  bool fail(const char* m) {
    if (err_.empty()) err_ = m;
    return false;
  }
  bool lit(const char* w) {
    size_t n = std::strlen(w);
    if ((size_t)(end_ - p_) < n || std::memcmp(p_, w, n)) return fail("bad literal");
    p_ += n;
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > 64) return fail("JSON nested too deeply");
    ws();
    if (p_ >= end_) return fail("unexpected end of JSON");
    const char c = *p_;
    if (c == '{') return object(v, depth);
    if (c == '[') return array(v, depth);
    if (c == '"') {
      v.kind = JVal::STR;
      return string(v.s);
    }
    if (c == 't') {
      v.kind = JVal::BOOL;
      v.b = true;
      return lit("true");
    }
    if (c == 'f') {
      v.kind = JVal::BOOL;
      v.b = false;
      return lit("false");
    }
    if (c == 'n') {
      v.kind = JVal::NUL;
      return lit("null");
    }
    return number(v);
  }
  bool object(JVal& v, int depth) {
    v.kind = JVal::OBJ;
    p_++;
    ws();
    if (p_ < end_ && *p_ == '}') {
      p_++;
      return true;
    }
    for (;;) {
      ws();
      std::string k;
      if (p_ >= end_ || *p_ != '"' || !string(k)) return fail("expected a string key");
      ws();
      if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
      p_++;
      JVal x;
      if (!value(x, depth + 1)) return false;
      v.obj.emplace_back(std::move(k), std::move(x));
      ws();
      if (p_ < end_ && *p_ == ',') {
        p_++;
        continue;
      }
      if (p_ < end_ && *p_ == '}') {
        p_++;
        return true;
      }
      return fail("expected ',' or '}'");
    }
  }
  bool array(JVal& v, int depth) {
    v.kind = JVal::ARR;
    p_++;
    ws();
    if (p_ < end_ && *p_ == ']') {
      p_++;
      return true;
    }
    for (;;) {
      JVal x;
      if (!value(x, depth + 1)) return false;
      v.arr.push_back(std::move(x));
      ws();
      if (p_ < end_ && *p_ == ',') {
        p_++;
        continue;
      }
      if (p_ < end_ && *p_ == ']') {
        p_++;
        return true;
      }
      return fail("expected ',' or ']'");
    }
  }
  static void utf8(std::string& s, unsigned cp) {
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
  bool hex4(unsigned& cp) {
    if (end_ - p_ < 4) return fail("short \\u escape");
    cp = 0;
    for (int i = 0; i < 4; i++) {
      const char c = p_[i];
      cp <<= 4;
      if (c >= '0' && c <= '9') cp |= (unsigned)(c - '0');
      else if (c >= 'a' && c <= 'f') cp |= (unsigned)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') cp |= (unsigned)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    p_ += 4;
    return true;
  }
  bool string(std::string& out) {
    p_++;  // opening quote
    while (p_ < end_ && *p_ != '"') {
      if ((unsigned char)*p_ < 0x20) return fail("control character in a string");
      if (*p_ != '\\') {
        out += *p_++;
        continue;
      }
      if (++p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          unsigned cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            p_ += 2;
            unsigned lo;
            if (!hex4(lo)) return false;
            if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p_ >= end_) return fail("unterminated string");
    p_++;  // closing quote
    return true;
  }
  bool number(JVal& v) {
    const char* s = p_;
    bool neg = false, frac = false;
    if (p_ < end_ && *p_ == '-') {
      neg = true;
      p_++;
    }
    if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad number");
    bool ovf = false;
    uint64_t u = 0;
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
      const unsigned d = (unsigned)(*p_ - '0');
      if (u > (UINT64_MAX - d) / 10) ovf = true;
      else u = u * 10 + d;
      p_++;
    }
    if (p_ < end_ && *p_ == '.') {
      frac = true;
      p_++;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      frac = true;
      p_++;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) p_++;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
    }
    v.kind = JVal::NUM;
    v.num = std::strtod(std::string(s, p_).c_str(), nullptr);
    v.is_uint = !neg && !frac && !ovf;
    v.u = v.is_uint ? u : 0;
    return true;
  }
};

}  // namespace moert
