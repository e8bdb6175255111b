// json_lite.cpp -- see json_lite.hpp.
#include "json_lite.hpp"

#include <cmath>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <stdexcept>

namespace spock::hip::json {

class Parser {
 public:
  explicit Parser(const std::string& s) : s_(s) {}

  Value document() {
    Value v = value();
    skip_ws();
    if (pos_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char* what) const {
    throw std::runtime_error(std::string("JSON parse error at offset ") + std::to_string(pos_) + ": " + what);
  }
  void skip_ws() {
    while (pos_ < s_.size() && (s_[pos_] == ' ' || s_[pos_] == '\n' || s_[pos_] == '\r' || s_[pos_] == '\t')) ++pos_;
  }
  bool consume(char c) {
    skip_ws();
    if (pos_ < s_.size() && s_[pos_] == c) {
      ++pos_;
      return true;
    }
    return false;
  }
  void expect_word(const char* w) {
    for (const char* p = w; *p; ++p, ++pos_)
      if (pos_ >= s_.size() || s_[pos_] != *p) fail("bad literal");
  }

  Value value() {
    skip_ws();
    if (pos_ >= s_.size()) fail("unexpected end of input");
    Value v;
    const char c = s_[pos_];
    if (c == '{') {
      ++pos_;
      v.kind_ = Value::Kind::Object;
      if (consume('}')) return v;
      do {
        skip_ws();
        std::string key = string_body();
        if (!consume(':')) fail("expected ':'");
        v.obj_[key] = value();
      } while (consume(','));
      if (!consume('}')) fail("expected '}'");
    } else if (c == '[') {
      ++pos_;
      v.kind_ = Value::Kind::Array;
      if (consume(']')) return v;
      do v.arr_.push_back(value());
      while (consume(','));
      if (!consume(']')) fail("expected ']'");
    } else if (c == '"') {
      v.kind_ = Value::Kind::String;
      v.str_ = string_body();
    } else if (c == 't') {
      expect_word("true");
      v.kind_ = Value::Kind::Bool;
      v.b_ = true;
    } else if (c == 'f') {
      expect_word("false");
      v.kind_ = Value::Kind::Bool;
    } else if (c == 'n') {
      expect_word("null");
    } else {
      const char* begin = s_.c_str() + pos_;
      char* end = nullptr;
      v.num_ = std::strtod(begin, &end);
      if (end == begin) fail("expected a value");
      pos_ += static_cast<std::size_t>(end - begin);
      v.kind_ = Value::Kind::Number;
    }
    return v;
  }

  std::string string_body() {
    if (pos_ >= s_.size() || s_[pos_] != '"') fail("expected string");
    ++pos_;
    std::string out;
    while (pos_ < s_.size() && s_[pos_] != '"') {
      char c = s_[pos_++];
      if (c == '\\') {
        if (pos_ >= s_.size()) fail("bad escape");
        const char e = s_[pos_++];
        switch (e) {
          case '"': case '\\': case '/': out.push_back(e); break;
          case 'n': out.push_back('\n'); break;
          case 't': out.push_back('\t'); break;
          case 'r': out.push_back('\r'); break;
          case 'b': out.push_back('\b'); break;
          case 'f': out.push_back('\f'); break;
          case 'u': {
            if (pos_ + 4 > s_.size()) fail("bad \\u escape");
            const long cp = std::strtol(s_.substr(pos_, 4).c_str(), nullptr, 16);
            if (cp >= 0x80) fail("non-ASCII \\u escape not supported");
            out.push_back(static_cast<char>(cp));
            pos_ += 4;
            break;
          }
          default: fail("bad escape");
        }
      } else {
        out.push_back(c);
      }
    }
    if (pos_ >= s_.size()) fail("unterminated string");
    ++pos_;
    return out;
  }

  const std::string& s_;
  std::size_t pos_ = 0;
};

bool Value::as_bool() const {
  if (kind_ != Kind::Bool) throw std::runtime_error("JSON value is not a boolean");
  return b_;
}
double Value::as_double() const {
  if (kind_ != Kind::Number) throw std::runtime_error("JSON value is not a number");
  return num_;
}
const std::vector<Value>& Value::as_array() const {
  if (kind_ != Kind::Array) throw std::runtime_error("JSON value is not an array");
  return arr_;
}
const std::string& Value::as_string() const {
  if (kind_ != Kind::String) throw std::runtime_error("JSON value is not a string");
  return str_;
}
const std::string& Value::get_string(const std::string& key) const {
  const Value* v = get(key);
  if (v == nullptr) throw std::runtime_error("missing string field: " + key);
  return v->as_string();
}
const Value* Value::get(const std::string& key) const {
  if (kind_ != Kind::Object) return nullptr;
  auto it = obj_.find(key);
  return it == obj_.end() ? nullptr : &it->second;
}
std::int64_t Value::get_int(const std::string& key) const {
  const Value* v = get(key);
  if (v == nullptr) throw std::runtime_error("missing integer field: " + key);
  return get_int(key, 0);
}
std::int64_t Value::get_int(const std::string& key, std::int64_t fallback) const {
  const Value* v = get(key);
  if (v == nullptr) return fallback;
  const double d = v->as_double();
  if (d != std::floor(d)) throw std::runtime_error("field is not an integer: " + key);
  return static_cast<std::int64_t>(d);
}

Value Value::parse(const std::string& text) { return Parser(text).document(); }

Value read_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("cannot open " + path);
  std::ostringstream ss;
  ss << f.rdbuf();
  return Value::parse(ss.str());
}

}  // namespace spock::hip::json
