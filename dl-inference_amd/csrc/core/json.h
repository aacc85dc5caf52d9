#pragma once

// Minimal JSON document model shared by the graph (dli.graph.v1) and weights (dli.weights.v1)
// readers. Integers and non-integers are kept apart because dli.graph.v1 attribute types are
// inferred from the literal: 2 is int64, 2.0 / 2e0 are double.

#include <cstdint>
#include <map>
#include <string>
#include <string_view>
#include <vector>

namespace dli::json {

struct Value {
  enum class Kind { Null, Bool, Int, Double, String, Array, Object };
  Kind kind = Kind::Null;
  bool b = false;
  std::int64_t i = 0;
  double d = 0.0;
  std::string s;
  std::vector<Value> items;
  std::map<std::string, Value> fields;

  bool isObject() const { return kind == Kind::Object; }
  bool isArray() const { return kind == Kind::Array; }
  bool isString() const { return kind == Kind::String; }
  bool isNumber() const { return kind == Kind::Int || kind == Kind::Double; }
  // nullptr when the key is absent; throws when this is not an object.
  const Value* find(const std::string& key) const;
  const Value& at(const std::string& key) const;
};

// Throws std::invalid_argument with the byte offset on malformed input.
Value parse(std::string_view text);

std::string quote(std::string_view text);
// Shortest text that parses back to the same double and always reads as a non-integer.
std::string formatDouble(double value);

std::string readFile(const std::string& path, const char* what);

}  // namespace dli::json
