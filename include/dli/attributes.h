#pragma once

// Typed node attributes of a dli.graph.v1 node.
// Interface kept identical to include/dli/attributes.h:12-45 of the reference so that
// operator plugins compiled against either header agree on the variant layout.

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

namespace dli {

// Alternative order is part of the plugin ABI (utils attrDouble tests index 0 == int64).
using AttributeValue =
    std::variant<std::int64_t, double, bool, std::string, std::vector<std::int64_t>,
                 std::vector<double>, std::vector<std::string>>;

class Attributes {
 public:
  void set(std::string name, AttributeValue value);
  bool contains(const std::string& name) const;

  template <typename T>
  const T& require(const std::string& name) const {
    const AttributeValue& value = lookup(name);
    const T* typed = std::get_if<T>(&value);
    if (typed == nullptr) throw std::invalid_argument("attribute has unexpected type: " + name);
    return *typed;
  }

  template <typename T>
  T value_or(const std::string& name, T fallback) const {
    auto it = values_.find(name);
    if (it == values_.end()) return fallback;
    const T* typed = std::get_if<T>(&it->second);
    if (typed == nullptr) throw std::invalid_argument("attribute has unexpected type: " + name);
    return *typed;
  }

  const std::map<std::string, AttributeValue>& values() const { return values_; }

 private:
  const AttributeValue& lookup(const std::string& name) const;

  std::map<std::string, AttributeValue> values_;
};

}  // namespace dli
