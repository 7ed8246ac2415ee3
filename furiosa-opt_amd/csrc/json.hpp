// Minimal JSON reader/writer for the MappingSerde wire form and small descriptor objects.
// Only what the C ABI needs: objects, arrays, strings, non-negative/negative integers, null/bools.
#pragma once

#include <cmath>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace fo::json {

struct Value {
  enum Kind { Null, Bool, Int, Double, String, Array, Object } kind = Null;
  bool b = false;
  int64_t i = 0;
  double d = 0.0;
  std::string s;
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;  // insertion order kept

  const Value* get(const std::string& key) const {
    for (auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
  const Value& at(const std::string& key) const {
    const Value* v = get(key);
    if (!v) throw std::runtime_error("json: missing key '" + key + "'");
    return *v;
  }
  int64_t as_int() const {
    if (kind == Int) return i;
    // A double converts only when it is integral and inside int64's range (the cast of anything
    // else is undefined behaviour).
    if (kind == Double && d >= -9223372036854775808.0 && d < 9223372036854775808.0 && d == std::trunc(d))
      return (int64_t)d;
    throw std::runtime_error("json: expected an integer");
  }
  const std::string& as_str() const {
    if (kind != String) throw std::runtime_error("json: expected a string");
    return s;
  }
};

class Parser {
 public:
  // Nesting deeper than this is rejected instead of recursing further: the parser reads untrusted
  // text (a safetensors header), and a MappingSerde mapping nests two levels per axis.
  static constexpr int kMaxDepth = 256;
  explicit Parser(const std::string& t) : t_(t) {}
  Value parse() {
    Value v = value();
    ws();
    if (p_ != t_.size()) fail("trailing characters");
    return v;
  }

 private:
  const std::string& t_;
  size_t p_ = 0;
  int depth_ = 0;
  struct Nest {
    Parser& p;
    explicit Nest(Parser& q) : p(q) {
      if (++p.depth_ > kMaxDepth) p.fail("nesting too deep");
    }
    ~Nest() { --p.depth_; }
  };

  [[noreturn]] void fail(const char* what) {
    throw std::runtime_error(std::string("json: ") + what + " at offset " + std::to_string(p_));
  }
  void ws() {
    while (p_ < t_.size() && (t_[p_] == ' ' || t_[p_] == '\n' || t_[p_] == '\t' || t_[p_] == '\r')) ++p_;
  }
  bool lit(const char* w) {
    size_t n = std::char_traits<char>::length(w);
    if (t_.compare(p_, n, w) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }
  Value value() {
    ws();
    if (p_ >= t_.size()) fail("unexpected end");
    char c = t_[p_];
    Value v;
    if (c == '{') {
      Nest nest(*this);
      v.kind = Value::Object;
      ++p_;
      ws();
      if (p_ < t_.size() && t_[p_] == '}') {
        ++p_;
        return v;
      }
      for (;;) {
        ws();
        std::string k = str();
        ws();
        if (p_ >= t_.size() || t_[p_] != ':') fail("expected ':'");
        ++p_;
        Value item = value();
        v.obj.emplace_back(std::move(k), std::move(item));
        ws();
        if (p_ < t_.size() && t_[p_] == ',') {
          ++p_;
          continue;
        }
        if (p_ < t_.size() && t_[p_] == '}') {
          ++p_;
          return v;
        }
        fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      Nest nest(*this);
      v.kind = Value::Array;
      ++p_;
      ws();
      if (p_ < t_.size() && t_[p_] == ']') {
        ++p_;
        return v;
      }
      for (;;) {
        v.arr.push_back(value());
        ws();
        if (p_ < t_.size() && t_[p_] == ',') {
          ++p_;
          continue;
        }
        if (p_ < t_.size() && t_[p_] == ']') {
          ++p_;
          return v;
        }
        fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Value::String;
      v.s = str();
      return v;
    }
    if (lit("null")) return v;
    if (lit("true")) {
      v.kind = Value::Bool;
      v.b = true;
      return v;
    }
    if (lit("false")) {
      v.kind = Value::Bool;
      return v;
    }
    return number();
  }
  std::string str() {
    if (p_ >= t_.size() || t_[p_] != '"') fail("expected a string");
    ++p_;
    std::string out;
    while (p_ < t_.size() && t_[p_] != '"') {
      if (t_[p_] == '\\') {
        ++p_;
        if (p_ >= t_.size()) fail("bad escape");
        char e = t_[p_];
        switch (e) {
          case '"':
          case '\\':
          case '/':
            out.push_back(e);
            break;
          case 'b':
            out.push_back('\b');
            break;
          case 'f':
            out.push_back('\f');
            break;
          case 'n':
            out.push_back('\n');
            break;
          case 'r':
            out.push_back('\r');
            break;
          case 't':
            out.push_back('\t');
            break;
          case 'u': {
            uint32_t cp = hex4();
            if (cp >= 0xD800 && cp < 0xDC00) {  // a high surrogate must be followed by a low one
              if (p_ + 2 >= t_.size() || t_[p_ + 1] != '\\' || t_[p_ + 2] != 'u') fail("unpaired surrogate");
              p_ += 2;
              uint32_t lo = hex4();
              if (lo < 0xDC00 || lo >= 0xE000) fail("unpaired surrogate");
              cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            } else if (cp >= 0xDC00 && cp < 0xE000) {
              fail("unpaired surrogate");
            }
            utf8(out, cp);
            break;
          }
          default:
            fail("bad escape");
        }
      } else {
        out.push_back(t_[p_]);
      }
      ++p_;
    }
    if (p_ >= t_.size()) fail("unterminated string");
    ++p_;
    return out;
  }
  // The four hex digits after "\u" (p_ on the 'u'); leaves p_ on the last digit.
  uint32_t hex4() {
    if (p_ + 4 >= t_.size()) fail("bad \\u escape");
    uint32_t v = 0;
    for (int k = 1; k <= 4; ++k) {
      char h = t_[p_ + k];
      uint32_t d = h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10 : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99;
      if (d > 15) fail("bad \\u escape");
      v = v * 16 + d;
    }
    p_ += 4;
    return v;
  }
  static void utf8(std::string& out, uint32_t cp) {
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
  }
  Value number() {
    size_t start = p_;
    if (p_ < t_.size() && (t_[p_] == '-' || t_[p_] == '+')) ++p_;
    bool isfloat = false;
    while (p_ < t_.size()) {
      char c = t_[p_];
      if (c >= '0' && c <= '9') {
        ++p_;
      } else if (c == '.' || c == 'e' || c == 'E' || ((c == '-' || c == '+') && isfloat)) {
        isfloat = true;
        ++p_;
      } else {
        break;
      }
    }
    if (start == p_) fail("unexpected character");
    Value v;
    std::string tok = t_.substr(start, p_ - start);
    if (isfloat) {
      v.kind = Value::Double;
      v.d = std::stod(tok);
    } else {
      v.kind = Value::Int;
      v.i = std::stoll(tok);
    }
    return v;
  }
};

inline Value parse(const std::string& text) { return Parser(text).parse(); }

}  // namespace fo::json
