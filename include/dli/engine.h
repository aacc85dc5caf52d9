#pragma once

// Sequential graph executor. Contract as include/dli/engine.h:12-28 / src/engine.cc:13-52 of the
// reference: nodes run in file order, inputs are looked up by name, outputs are moved into the
// tensor map, and the result is graph.outputs (or every tensor when that list is empty).
//
// Differences in mechanism: operators are created once per op type and reused (operators are
// stateless: compute() is const), debug logging is formatted only when enabled, and the kernels
// of every node go on one caller-chosen HIP stream. Inputs are looked up by name in the run's
// tensor map for every node, as in the reference.

#include <map>
#include <memory>
#include <string>
#include <unordered_map>

#include "dli/graph.h"
#include "dli/operator.h"
#include "dli/profiler.h"
#include "dli/tensor.h"

namespace dli {

using TensorMap = std::map<std::string, Tensor>;

class Engine {
 public:
  Engine();
  Engine(const Engine&) = delete;
  Engine& operator=(const Engine&) = delete;

  OperatorRegistry& registry() { return registry_; }
  const OperatorRegistry& registry() const { return registry_; }
  KVCache& kvCache() { return kv_cache_; }
  const KVCache& kvCache() const { return kv_cache_; }

  TensorMap run(const Graph& graph, TensorMap inputs);
  // With options.profiler, every node is timed into that session (include/dli/profiler.h).
  TensorMap run(const Graph& graph, TensorMap inputs, const RunOptions& options);

  // Stream for subsequent run() calls (hipStream_t as void*; nullptr = null stream).
  void setStream(void* stream);
  void* stream() const { return stream_; }

 private:
  Operator& operatorFor(const std::string& type);

  OperatorRegistry registry_;
  KVCache kv_cache_;
  void* stream_ = nullptr;
  std::unordered_map<std::string, std::unique_ptr<Operator>> op_cache_;
  std::uint64_t op_cache_version_ = 0;
};

}  // namespace dli
