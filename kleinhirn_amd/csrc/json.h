// Minimal JSON reader for plan documents: objects, arrays, strings (with \uXXXX escapes as
// UTF-8), numbers (as double), true/false/null. Throws std::runtime_error with the byte offset.
#pragma once

#include <cctype>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace kh {

struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double n = 0;
  std::string s;
  std::vector<Json> a;
  std::map<std::string, Json> o;

  bool has(const std::string &k) const { return kind == Obj && o.count(k) > 0; }
  const Json &at(const std::string &k) const {
    auto it = o.find(k);
    if (kind != Obj || it == o.end()) throw std::runtime_error("plan JSON: missing key '" + k + "'");
    return it->second;
  }
  double num() const {
    if (kind != Num) throw std::runtime_error("plan JSON: expected a number");
    return n;
  }
  int64_t integer() const {
    double v = num();
    if (v != (double)(int64_t)v) throw std::runtime_error("plan JSON: expected an integer");
    return (int64_t)v;
  }
  const std::string &str() const {
    if (kind != Str) throw std::runtime_error("plan JSON: expected a string");
    return s;
  }
  const std::vector<Json> &arr() const {
    if (kind != Arr) throw std::runtime_error("plan JSON: expected an array");
    return a;
  }
};

class JsonReader {
 public:
  JsonReader(const char *p, size_t n) : p_(p), n_(n) {}
  Json parse() {
    Json v = value();
    ws();
    if (i_ != n_) fail("trailing characters");
    return v;
  }

 private:
  const char *p_;
  size_t n_;
  size_t i_ = 0;
  int depth_ = 0;

  [[noreturn]] void fail(const char *what) {
    throw std::runtime_error(std::string("plan JSON: ") + what + " at byte " + std::to_string(i_));
  }
  void ws() {
    while (i_ < n_ && (p_[i_] == ' ' || p_[i_] == '\n' || p_[i_] == '\t' || p_[i_] == '\r')) i_++;
  }
  bool eat(char c) {
    ws();
    if (i_ < n_ && p_[i_] == c) {
      i_++;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!eat(c)) fail("unexpected character");
  }
  Json value() {
    ws();
    if (i_ >= n_) fail("unexpected end");
    if (++depth_ > 64) fail("nesting too deep");
    Json v;
    char c = p_[i_];
    if (c == '{') {
      i_++;
      v.kind = Json::Obj;
      if (!eat('}')) {
        do {
          ws();
          std::string k = string();
          expect(':');
          v.o[k] = value();
        } while (eat(','));
        expect('}');
      }
    } else if (c == '[') {
      i_++;
      v.kind = Json::Arr;
      if (!eat(']')) {
        do v.a.push_back(value());
        while (eat(','));
        expect(']');
      }
    } else if (c == '"') {
      v.kind = Json::Str;
      v.s = string();
    } else if (c == 't' && lit("true")) {
      v.kind = Json::Bool;
      v.b = true;
    } else if (c == 'f' && lit("false")) {
      v.kind = Json::Bool;
    } else if (c == 'n' && lit("null")) {
      v.kind = Json::Null;
    } else {
      v.kind = Json::Num;
      v.n = number();
    }
    depth_--;
    return v;
  }
  bool lit(const char *w) {
    size_t k = 0;
    while (w[k]) {
      if (i_ + k >= n_ || p_[i_ + k] != w[k]) fail("bad literal");
      k++;
    }
    i_ += k;
    return true;
  }
  double number() {
    size_t start = i_;
    while (i_ < n_ && (std::isdigit((unsigned char)p_[i_]) || p_[i_] == '-' || p_[i_] == '+' ||
                       p_[i_] == '.' || p_[i_] == 'e' || p_[i_] == 'E'))
      i_++;
    if (i_ == start) fail("bad value");
    std::string t(p_ + start, i_ - start);
    char *end = nullptr;
    double v = std::strtod(t.c_str(), &end);
    if (!end || *end) fail("bad number");
    return v;
  }
  static void utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (i_ + 4 > n_) fail("bad escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; k++) {
      char c = p_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else fail("bad escape");
    }
    return v;
  }
  std::string string() {
    if (i_ >= n_ || p_[i_] != '"') fail("expected a string");
    i_++;
    std::string out;
    while (true) {
      if (i_ >= n_) fail("unterminated string");
      char c = p_[i_++];
      if (c == '"') break;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= n_) fail("bad escape");
      char e = p_[i_++];
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
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00 && i_ + 6 <= n_ && p_[i_] == '\\' && p_[i_ + 1] == 'u') {
            i_ += 2;
            uint32_t lo = hex4();
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
    return out;
  }
};

}  // namespace kh
