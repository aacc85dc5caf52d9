// Graph executor (reference behaviour: src/engine.cc:11-52).
#include "dli/engine.h"

#include <stdexcept>

#include "dli/aten_operator.h"
#include "dli/logging.h"
#include "dli/utils.h"
#include "dli_hip.h"

namespace dli {

Engine::Engine() { registerAtenOperator(registry_); }

void Engine::setStream(void* stream) {
  stream_ = stream;
  kv_cache_.setStream(stream);
}

Operator& Engine::operatorFor(const std::string& type) {
  if (op_cache_version_ != registry_.version()) {
    op_cache_.clear();
    op_cache_version_ = registry_.version();
  }
  auto it = op_cache_.find(type);
  if (it == op_cache_.end()) it = op_cache_.emplace(type, registry_.create(type)).first;
  return *it->second;
}

TensorMap Engine::run(const Graph& graph, TensorMap tensors) {
  return run(graph, std::move(tensors), RunOptions{});
}

TensorMap Engine::run(const Graph& graph, TensorMap tensors, const RunOptions& options) {
  ExecutionContext context;
  context.kv_cache = &kv_cache_;
  context.stream = stream_;
  context.profiler = options.profiler;
  kv_cache_.setStream(stream_);
  ProfileSession* const profiler = options.profiler;
  std::int64_t run_id = -1;
  if (profiler != nullptr) {
    int capturing = 0;
    if (profiler->config().gpu && dli_hip_available() != 0 &&
        dli_hip_stream_is_capturing(stream_, &capturing) != 0)
      capturing = 1;  // cannot tell: no device timing for this run
    run_id = profiler->beginRun(stream_, capturing != 0);
  }
  // Ends the run record on every exit path (error status while unwinding).
  struct RunEnd {
    ProfileSession* p;
    std::int64_t id;
    bool ok = false;
    ~RunEnd() {
      if (p != nullptr) p->endRun(id, ok);
    }
  } run_end{profiler, run_id};

  std::vector<const Tensor*> inputs;
  std::vector<Tensor> produced;
  std::vector<Tensor*> outputs;
  for (const Node& node : graph.nodes) {
    inputs.clear();
    for (const std::string& name : node.inputs) {
      auto it = tensors.find(name);
      if (it == tensors.end())
        throw std::invalid_argument("node '" + node.name + "' missing input tensor: " + name);
      inputs.push_back(&it->second);
      LOG_DEBUG << "node '" << node.name << "' input " << name << ' '
                << formatShape(it->second.shape());
    }
    produced.assign(node.outputs.size(), Tensor());
    outputs.clear();
    for (Tensor& slot : produced) outputs.push_back(&slot);

    Operator& op = operatorFor(node.op_type);
    LOG_DEBUG << "node '" << node.name << "' op " << node.op_type;
    if (profiler != nullptr) {
      ProfileSession::Scope scope = profiler->beginOperator(
          run_id, static_cast<std::int64_t>(&node - graph.nodes.data()), node, inputs);
      op.compute(inputs, outputs, node.attributes, context);
      scope.finish(true, &outputs);
    } else {
      op.compute(inputs, outputs, node.attributes, context);
    }

    for (std::size_t i = 0; i < node.outputs.size(); ++i) {
      LOG_DEBUG << "node '" << node.name << "' output " << node.outputs[i] << ' '
                << formatShape(produced[i].shape());
      tensors.insert_or_assign(node.outputs[i], std::move(produced[i]));
    }
  }

  run_end.ok = true;
  if (graph.outputs.empty()) return tensors;
  TensorMap result;
  for (const std::string& name : graph.outputs) {
    auto it = tensors.find(name);
    if (it == tensors.end())
      throw std::invalid_argument("graph output tensor was not produced: " + name);
    result.emplace(name, it->second);
  }
  return result;
}

}  // namespace dli
