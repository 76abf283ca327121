// json.hpp -- a small JSON reader for the files checkpoint ingestion reads:
// the safetensors header, model.safetensors.index.json and config.json
// (the reference reads them with nlohmann::json, src/common/safetensors.cpp:23-77,
// src/common/base_config.cpp:28-73).  Objects keep their keys in a map;
// numbers are kept as double (every integer the files hold is exact in one).
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

namespace mlx_lm {
namespace mi355x {

class Json {
 public:
  enum class Type { null, boolean, number, string, array, object };

  Type type() const { return type_; }
  bool is_object() const { return type_ == Type::object; }
  bool is_array() const { return type_ == Type::array; }
  bool is_string() const { return type_ == Type::string; }
  bool is_number() const { return type_ == Type::number; }
  bool is_null() const { return type_ == Type::null; }

  // typed access; throws std::invalid_argument on a type mismatch
  const std::string& str() const;
  double num() const;
  int64_t integer() const;  // a number with an integral value
  bool boolean() const;
  const std::vector<Json>& items() const;
  const std::map<std::string, Json>& fields() const;

  bool contains(const std::string& key) const;
  const Json& at(const std::string& key) const;  // throws if absent
  // the member, or `fallback` when absent or null
  int64_t value(const std::string& key, int64_t fallback) const;
  double value(const std::string& key, double fallback) const;
  bool value(const std::string& key, bool fallback) const;

  friend Json parse_json(const std::string& text);

 private:
  Type type_ = Type::null;
  bool b_ = false;
  double n_ = 0.0;
  std::string s_;
  std::vector<Json> a_;
  std::map<std::string, Json> o_;
  friend class JsonParser;
};

// Parses a whole JSON text; throws std::invalid_argument with the offset of
// the first error.
Json parse_json(const std::string& text);

}  // namespace mi355x
}  // namespace mlx_lm
