// A small JSON value for the HTTP API: parse (RFC 8259, UTF-8 passed through, \u escapes with surrogate pairs),
// build, and serialise. Integers that fit in 64 bits keep their exact value (seeds are uint64).
#pragma once

#include <cstdint>
#include <initializer_list>
#include <map>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace malkin_hip::json {

struct ParseError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

class Value {
 public:
  enum class Kind { Null, Bool, Int, Uint, Double, String, Array, Object };

  Value() = default;
  Value(std::nullptr_t) {}
  Value(bool b) : kind_(Kind::Bool), b_(b) {}
  Value(int v) : kind_(Kind::Int), i_(v) {}
  Value(int64_t v) : kind_(Kind::Int), i_(v) {}
  Value(uint64_t v) : kind_(Kind::Uint), u_(v) {}
  Value(double v) : kind_(Kind::Double), d_(v) {}
  Value(const char* s) : kind_(Kind::String), s_(s) {}
  Value(std::string s) : kind_(Kind::String), s_(std::move(s)) {}
  static Value array(std::vector<Value> items = {});
  static Value object(std::initializer_list<std::pair<const std::string, Value>> items = {});

  static Value parse(std::string_view text);
  std::string dump() const;

  Kind kind() const { return kind_; }
  bool is_null() const { return kind_ == Kind::Null; }
  bool is_bool() const { return kind_ == Kind::Bool; }
  bool is_number() const { return kind_ == Kind::Int || kind_ == Kind::Uint || kind_ == Kind::Double; }
  bool is_integer() const { return kind_ == Kind::Int || kind_ == Kind::Uint; }
  bool is_string() const { return kind_ == Kind::String; }
  bool is_array() const { return kind_ == Kind::Array; }
  bool is_object() const { return kind_ == Kind::Object; }

  bool as_bool() const;
  double as_double() const;
  int64_t as_int() const;    // integers only (range-checked)
  uint64_t as_uint() const;  // non-negative integers only
  const std::string& as_string() const;
  const std::vector<Value>& items() const;  // array elements

  // Objects: keys in insertion order.
  bool has(const std::string& key) const;
  const Value& operator[](const std::string& key) const;  // null value when absent
  Value& set(const std::string& key, Value v);
  Value& push(Value v);  // arrays

 private:
  void dump_to(std::string& out) const;

  Kind kind_ = Kind::Null;
  bool b_ = false;
  int64_t i_ = 0;
  uint64_t u_ = 0;
  double d_ = 0.0;
  std::string s_;
  std::vector<Value> a_;
  std::vector<std::pair<std::string, Value>> o_;
};

}  // namespace malkin_hip::json
