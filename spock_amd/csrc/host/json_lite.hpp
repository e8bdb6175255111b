// json_lite.hpp -- a small JSON reader for the command-line drivers.
//
// Enough JSON for the chunk-rule fixture files (objects, arrays, numbers,
// booleans, null, strings without unicode escapes beyond \uXXXX < 0x80).
// Errors are std::runtime_error with the byte offset.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace spock::hip::json {

class Value {
 public:
  enum class Kind { Null, Bool, Number, String, Array, Object };

  Kind kind() const { return kind_; }
  bool is_null() const { return kind_ == Kind::Null; }
  bool is_bool() const { return kind_ == Kind::Bool; }
  bool is_number() const { return kind_ == Kind::Number; }
  bool is_string() const { return kind_ == Kind::String; }
  bool is_array() const { return kind_ == Kind::Array; }
  bool is_object() const { return kind_ == Kind::Object; }

  bool as_bool() const;
  double as_double() const;
  const std::vector<Value>& as_array() const;
  const std::string& as_string() const;
  // String member; error when absent or not a string.
  const std::string& get_string(const std::string& key) const;
  // Member lookup on an object; nullptr when absent (or not an object).
  const Value* get(const std::string& key) const;
  // Integer member; `fallback` when absent, error when present but not integral.
  std::int64_t get_int(const std::string& key) const;
  std::int64_t get_int(const std::string& key, std::int64_t fallback) const;

  static Value parse(const std::string& text);

 private:
  friend class Parser;
  Kind kind_ = Kind::Null;
  bool b_ = false;
  double num_ = 0.0;
  std::string str_;
  std::vector<Value> arr_;
  std::map<std::string, Value> obj_;
};

Value read_file(const std::string& path);

}  // namespace spock::hip::json
