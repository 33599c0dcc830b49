// Minimal JSON reader for tokenizer.json / tokenizer_config.json / task
// schemas: a DOM of null, bool, number (double), string (UTF-8), array and
// object (keys in file order).  Parse errors throw std::runtime_error.
#pragma once

#include <string>
#include <utility>
#include <vector>

namespace gdf {

struct Json {
  enum Type { Null, Bool, Number, String, Array, Object };
  Type type = Null;
  bool boolean = false;
  double number = 0.0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  bool is_null() const { return type == Null; }
  bool is_string() const { return type == String; }
  bool is_number() const { return type == Number; }
  bool is_array() const { return type == Array; }
  bool is_object() const { return type == Object; }
  bool is_bool() const { return type == Bool; }
  // Member `key` of an object (the last one when a key repeats), or nullptr.
  const Json* get(const std::string& key) const;
};

Json parse_json(const char* text, size_t size);

}  // namespace gdf
