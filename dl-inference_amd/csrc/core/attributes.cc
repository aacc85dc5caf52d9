// Attribute map storage (reference: src/attributes.cc:5-11).
#include "dli/attributes.h"

#include <utility>

namespace dli {

void Attributes::set(std::string name, AttributeValue value) {
  values_.insert_or_assign(std::move(name), std::move(value));
}

bool Attributes::contains(const std::string& name) const { return values_.count(name) != 0; }

const AttributeValue& Attributes::lookup(const std::string& name) const {
  auto it = values_.find(name);
  if (it == values_.end()) throw std::invalid_argument("missing required attribute: " + name);
  return it->second;
}

}  // namespace dli
