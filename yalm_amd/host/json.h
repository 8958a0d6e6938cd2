// Minimal JSON reader/writer for the .yalm (safetensors) header: objects, arrays, strings,
// numbers, booleans and null. Written for this project; only what the header format needs.
#pragma once
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace yalm {

struct Json {
  enum class Kind { Null, Bool, Number, String, Array, Object };
  Kind kind = Kind::Null;
  bool b = false;
  double num = 0.0;
  bool is_integer = false;  // the literal had no fraction/exponent
  int64_t i64 = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;  // insertion order kept

  const Json* find(const std::string& key) const;
  bool is_object() const { return kind == Kind::Object; }
  bool is_array() const { return kind == Kind::Array; }
  bool is_string() const { return kind == Kind::String; }
  bool is_number() const { return kind == Kind::Number; }
};

// Parses `text`; on failure returns false and sets `err`.
bool json_parse(const std::string& text, Json& out, std::string& err);
// Escapes a string as a JSON string literal (with quotes).
std::string json_quote(const std::string& s);

}  // namespace yalm
