#pragma once

// Operator interface, registry and plugin entry point.
// Same contract as include/dli/operator.h:15-41 of the reference: a plugin .so exports
//   extern "C" bool dli_register_operators(dli::OperatorRegistry*);
// and registers string-keyed factories. ExecutionContext keeps kv_cache as its first member;
// new fields are appended after it so that plugins built against the reference still read
// kv_cache at the same offset.

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "dli/attributes.h"
#include "dli/kv_cache.h"
#include "dli/tensor.h"

namespace dli {

class ProfileSession;

struct ExecutionContext {
  KVCache* kv_cache = nullptr;
  // HIP stream (hipStream_t) on which operators enqueue their kernels; nullptr = null stream.
  void* stream = nullptr;
  // The run's profiling session, or nullptr (include/dli/profiler.h); operators may read it.
  ProfileSession* profiler = nullptr;
};

class Operator {
 public:
  virtual ~Operator() = default;
  virtual std::string type() const = 0;
  virtual void compute(const std::vector<const Tensor*>& inputs,
                       const std::vector<Tensor*>& outputs, const Attributes& attrs,
                       ExecutionContext& context) const = 0;
};

class OperatorRegistry {
 public:
  using Factory = std::function<std::unique_ptr<Operator>()>;
  void registerFactory(std::string type, Factory factory);
  bool contains(const std::string& type) const;
  std::unique_ptr<Operator> create(const std::string& type) const;
  void loadLibrary(const std::string& path);

  // Registered operator names, sorted.
  std::vector<std::string> names() const;
  // Incremented on every registration; lets callers cache created operators.
  std::uint64_t version() const { return version_; }

 private:
  std::map<std::string, Factory> factories_;
  std::vector<void*> library_handles_;
  std::uint64_t version_ = 0;
};

using RegisterOperatorsFn = bool (*)(OperatorRegistry*);

}  // namespace dli
