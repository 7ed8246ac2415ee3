// Minimal JSON reader/writer for the MappingSerde wire form and small descriptor objects.
// Only what the C ABI needs: objects, arrays, strings, non-negative/negative integers, null/bools.
#pragma once

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
    if (kind == Double && d == (double)(int64_t)d) return (int64_t)d;
    throw std::runtime_error("json: expected an integer");
  }
  const std::string& as_str() const {
    if (kind != String) throw std::runtime_error("json: expected a string");
    return s;
  }
};

class Parser {
 public:
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
        out.push_back(e == 'n' ? '\n' : e == 't' ? '\t' : e);
      } else {
        out.push_back(t_[p_]);
      }
      ++p_;
    }
    if (p_ >= t_.size()) fail("unterminated string");
    ++p_;
    return out;
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
