// json.hpp -- a small strict JSON document model for the tuning cache files.
//
// The tuning-cache envelope (tuning/schema.json) and the binaries manifest are
// read and written through this module.  Parsing follows RFC 8259 strictly: no
// comments, no trailing commas, no duplicate object keys, UTF-8 validated,
// nesting depth bounded.  Serialisation is compact (no whitespace) with object
// keys in byte order and numbers in their shortest round-trip form, so a given
// document always serialises to the same bytes.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace pk::json {

class Value;
using Array = std::vector<Value>;
// Object members keep their insertion order; lookups are linear (the tuning
// documents have objects of at most a dozen keys).
using Object = std::vector<std::pair<std::string, Value>>;

class Value {
 public:
  enum class Kind { Null, Bool, Number, String, Array, Object };

  Value() = default;  // null
  Value(std::nullptr_t) {}
  Value(bool b) : kind_(Kind::Bool), b_(b) {}
  Value(int v) : Value(static_cast<long long>(v)) {}
  Value(long v) : Value(static_cast<long long>(v)) {}
  Value(long long v) : kind_(Kind::Number), is_int_(true), i_(static_cast<int64_t>(v)), d_(static_cast<double>(v)) {}
  Value(double d) : kind_(Kind::Number), d_(d) {}
  Value(const char *s) : kind_(Kind::String), s_(std::make_shared<std::string>(s)) {}
  Value(std::string s) : kind_(Kind::String), s_(std::make_shared<std::string>(std::move(s))) {}
  Value(Array a) : kind_(Kind::Array), a_(std::make_shared<Array>(std::move(a))) {}
  Value(Object o) : kind_(Kind::Object), o_(std::make_shared<Object>(std::move(o))) {}

  Kind kind() const { return kind_; }
  bool is_null() const { return kind_ == Kind::Null; }

  std::optional<bool> as_bool() const;
  // Any number.
  std::optional<double> as_number() const;
  // An integer literal, or a number literal whose value is an integer that
  // fits in int64 (4096.0 reads as 4096).
  std::optional<int64_t> as_integer() const;
  const std::string *as_string() const { return kind_ == Kind::String ? s_.get() : nullptr; }
  const Array *as_array() const { return kind_ == Kind::Array ? a_.get() : nullptr; }
  const Object *as_object() const { return kind_ == Kind::Object ? o_.get() : nullptr; }

 private:
  Kind kind_ = Kind::Null;
  bool b_ = false;
  bool is_int_ = false;
  int64_t i_ = 0;
  double d_ = 0.0;
  std::shared_ptr<const std::string> s_;
  std::shared_ptr<const Array> a_;
  std::shared_ptr<const Object> o_;
};

// Member `key` of an object, or nullptr.
const Value *Get(const Object &obj, std::string_view key);

struct ParseResult {
  std::optional<Value> value;
  std::string error;  // "<message> at line L column C" when value is empty
  bool ok() const { return value.has_value(); }
};

ParseResult Parse(std::string_view text);
std::string Serialize(const Value &v);

}  // namespace pk::json
