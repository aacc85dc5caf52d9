// String-keyed operator factories and the plugin loader (reference: src/operator_registry.cc:9-41).
// loadLibrary keeps the reference contract: dlopen(RTLD_NOW|RTLD_LOCAL), resolve
// "dli_register_operators", call it with this registry, dlclose and throw if the symbol is
// missing or registration reports failure; a loaded library is never unloaded. A later
// registration of the same name replaces the earlier one.
#include <dlfcn.h>

#include <stdexcept>

#include "dli/operator.h"

namespace dli {

void OperatorRegistry::registerFactory(std::string type, Factory factory) {
  factories_.insert_or_assign(std::move(type), std::move(factory));
  ++version_;
}

bool OperatorRegistry::contains(const std::string& type) const {
  return factories_.find(type) != factories_.end();
}

std::unique_ptr<Operator> OperatorRegistry::create(const std::string& type) const {
  auto it = factories_.find(type);
  if (it == factories_.end()) throw std::invalid_argument("operator is not registered: " + type);
  return it->second();
}

std::vector<std::string> OperatorRegistry::names() const {
  std::vector<std::string> out;
  out.reserve(factories_.size());
  for (const auto& entry : factories_) out.push_back(entry.first);
  return out;
}

void OperatorRegistry::loadLibrary(const std::string& path) {
  dlerror();
  void* handle = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
  if (handle == nullptr) {
    const char* why = dlerror();
    throw std::runtime_error("failed to load operator library: " + path + ": " +
                             (why ? why : "unknown error"));
  }
  auto register_fn = reinterpret_cast<RegisterOperatorsFn>(dlsym(handle, "dli_register_operators"));
  if (register_fn == nullptr) {
    dlclose(handle);
    throw std::runtime_error("operator library is missing dli_register_operators: " + path);
  }
  bool ok = false;
  try {
    ok = register_fn(this);
  } catch (...) {
    ok = false;
  }
  if (!ok) {
    dlclose(handle);
    throw std::runtime_error("operator library registration failed: " + path);
  }
  library_handles_.push_back(handle);
}

}  // namespace dli
