// Minimal JSON reader for checkpoint metadata (safetensors headers, shard indexes, HF
// config.json), with the accessor semantics of io/json.rs: numbers keep their source text and
// are parsed on access (as_u64 accepts plain decimal digits only, as_f64 any JSON number);
// objects are ordered maps in which a repeated key keeps its last value; every failure is a
// Parse error.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace fr {

class JsonValue {
 public:
  enum class Kind { Null, Bool, Number, String, Array, Object };

  Kind kind() const { return kind_; }
  bool is_null() const { return kind_ == Kind::Null; }
  const std::map<std::string, JsonValue>& as_object() const;
  const std::vector<JsonValue>& as_array() const;
  const std::string& as_str() const;
  bool as_bool() const;
  uint64_t as_u64() const;  // a number whose text is decimal digits that fit 64 bits
  double as_f64() const;
  // Member of an object; Parse error naming the key when absent.
  const JsonValue& get(const std::string& key) const;
  // Member or nullptr (also for a non-object receiver: callers check the kind first).
  const JsonValue* find(const std::string& key) const;

  static JsonValue parse(const std::string& text);

 private:
  friend class JsonParser;
  Kind kind_ = Kind::Null;
  bool boolean_ = false;
  std::string text_;  // string contents, or a number's source text
  std::vector<JsonValue> array_;
  std::map<std::string, JsonValue> object_;
};

}  // namespace fr
