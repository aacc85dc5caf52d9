// Greedy decode driver (include/dli/greedy.h): the C++ counterpart of
// python/dli_qwen2/session.py's DecodeSession.generate, with the step captured into a HIP graph
// through ATen's graph capture.
#include "dli/greedy.h"

#include <ATen/ATen.h>
#include <ATen/hip/HIPGraph.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace dli {

struct GreedyDecoder::Impl {
  Engine& engine;
  Graph graph;
  TensorMap inputs;
  std::int64_t batch = 0;
  GreedyOptions options;
  bool on_device = false;
  int device_id = 0;
  bool has_status = false;  // the graph lists a "status" output (decoder_stack launch status)
  Tensor ids;               // static step inputs (the captured graph reads these buffers)
  Tensor positions;
  Tensor status;            // the status output of the last run (a persistent device word)
  std::unique_ptr<at::cuda::CUDAGraph> hip_graph;
  std::optional<c10::hip::HIPStream> capture_stream;
  TensorMap captured_out;

  Impl(Engine& e, Graph g, TensorMap w, std::int64_t b, GreedyOptions o)
      : engine(e), graph(std::move(g)), inputs(std::move(w)), batch(b), options(o) {}

  void* currentStream() const {
    return on_device ? static_cast<void*>(c10::hip::getCurrentHIPStream(device_id).stream())
                     : nullptr;
  }

  TensorMap keepStatus(TensorMap out) {
    if (has_status) status = out.at("status");
    return out;
  }

  TensorMap runEager() {
    engine.setStream(currentStream());
    return keepStatus(engine.run(graph, inputs));
  }

  // The first step on a device with capture on: the step runs eagerly on the capture stream
  // with the real ids and positions (so operators are created and every lazily allocated cache
  // and workspace exists, and nothing but this step's own tokens is written to the KV cache),
  // then the same step is recorded into a HIP graph that later steps replay.
  TensorMap runThenCapture() {
    // the static inputs were written on the current stream
    c10::hip::getCurrentHIPStream(device_id).synchronize();
    c10::hip::HIPStream stream = c10::hip::getStreamFromPool(false, device_id);
    c10::hip::HIPStreamGuard guard(stream);
    void* const previous = engine.stream();
    engine.setStream(stream.stream());
    TensorMap first;
    try {
      first = keepStatus(engine.run(graph, inputs));
      stream.synchronize();
      auto g = std::make_unique<at::cuda::CUDAGraph>();
      g->capture_begin();
      try {
        captured_out = engine.run(graph, inputs);
      } catch (...) {
        try {
          g->capture_end();
        } catch (...) {
        }
        throw;
      }
      g->capture_end();
      hip_graph = std::move(g);
    } catch (...) {
      engine.setStream(previous);
      throw;
    }
    engine.setStream(previous);
    return first;
  }

  // One step on the static inputs (already copied in).
  TensorMap run() {
    if (hip_graph) {
      hip_graph->replay();
      if (has_status) status = captured_out.at("status");
      return captured_out;
    }
    if (on_device && options.capture) return runThenCapture();
    return runEager();
  }

  // Raises if a step since the last check reported a failed launch (the graph's status output,
  // non-zero when a decoder_stack wait gave up and its outputs are invalid), clearing the word.
  // Synchronizes with the device: called where the caller synchronizes anyway.
  void checkStatus() {
    if (!has_status || !status.defined()) return;
    at::Tensor& word = status.torchTensor();
    if (word.item<std::int32_t>() == 0) return;
    word.zero_();
    throw std::runtime_error(
        "decode step failed: a decoder_stack workgroup gave up waiting (its outputs are invalid)");
  }
};

namespace {

void requireIds(const Tensor& t, std::int64_t batch, const char* what) {
  if (!t.defined() || t.dtype() != DType::Int64 || t.rank() != 1 || t.dim(0) != batch)
    throw std::invalid_argument(std::string(what) + " must be int64 [" + std::to_string(batch) +
                                "]");
}

bool listed(const std::vector<std::string>& names, const std::string& name) {
  return std::find(names.begin(), names.end(), name) != names.end();
}

}  // namespace

GreedyDecoder::GreedyDecoder(Engine& engine, Graph graph, TensorMap weights, std::int64_t batch,
                             GreedyOptions options) {
  if (batch <= 0) throw std::invalid_argument("batch must be positive");
  if (options.block_size <= 0 || options.max_seq_len <= 0)
    throw std::invalid_argument("block_size and max_seq_len must be positive");
  for (const char* name : {"input_ids", "positions"}) {
    if (!listed(graph.inputs, name))
      throw std::invalid_argument(std::string("decode graph has no input ") + name);
    if (weights.count(name) != 0)
      throw std::invalid_argument(std::string(name) + " is a step input, not a weight");
  }
  if (!listed(graph.outputs, "next_ids"))
    throw std::invalid_argument("decode graph has no output next_ids");
  impl_ = std::make_unique<Impl>(engine, std::move(graph), std::move(weights), batch, options);
  Impl& s = *impl_;
  for (const auto& [name, t] : s.inputs) {
    if (t.isCuda()) {
      s.on_device = true;
      s.device_id = t.deviceId();
      break;
    }
  }
  s.ids = s.on_device ? Tensor::cuda(DType::Int64, {batch}, s.device_id)
                      : Tensor::zeros(DType::Int64, {batch});
  s.positions = s.on_device ? Tensor::cuda(DType::Int64, {batch}, s.device_id)
                            : Tensor::zeros(DType::Int64, {batch});
  if (s.on_device) {
    s.ids.torchTensor().zero_();
    s.positions.torchTensor().zero_();
  }
  s.inputs["input_ids"] = s.ids;
  s.inputs["positions"] = s.positions;
  s.has_status = listed(s.graph.outputs, "status");
  engine.kvCache().configure(options.block_size, options.max_seq_len);
}

GreedyDecoder::~GreedyDecoder() = default;

std::int64_t GreedyDecoder::batch() const { return impl_->batch; }

bool GreedyDecoder::captured() const { return impl_->hip_graph != nullptr; }

TensorMap GreedyDecoder::step(const Tensor& ids, const Tensor& positions) {
  Impl& s = *impl_;
  requireIds(ids, s.batch, "ids");
  requireIds(positions, s.batch, "positions");
  const at::Tensor& pos = positions.torchTensor();
  const std::int64_t lo = pos.min().item<std::int64_t>();
  const std::int64_t hi = pos.max().item<std::int64_t>();
  if (lo < 0 || hi >= s.options.max_seq_len)
    throw std::out_of_range("position outside the KV cache capacity [0, " +
                            std::to_string(s.options.max_seq_len) + ")");
  s.checkStatus();  // a failure of an earlier step (the reads above synchronized)
  s.ids.torchTensor().copy_(ids.torchTensor());
  s.positions.torchTensor().copy_(pos);
  return s.run();
}

void GreedyDecoder::checkStatus() { impl_->checkStatus(); }

Tensor GreedyDecoder::generate(const Tensor& prompt, std::int64_t steps, std::int64_t start) {
  Impl& s = *impl_;
  if (!prompt.defined() || prompt.dtype() != DType::Int64 || prompt.rank() != 2 ||
      prompt.dim(0) != s.batch || prompt.dim(1) < 1)
    throw std::invalid_argument("prompt must be int64 [" + std::to_string(s.batch) +
                                ", S] with S >= 1");
  if (steps < 1 || start < 0) throw std::invalid_argument("steps must be >= 1 and start >= 0");
  const std::int64_t length = prompt.dim(1);
  // the last step to run feeds the (steps - 1)-th generated token
  if (start + length + steps - 2 >= s.options.max_seq_len)
    throw std::out_of_range("prompt plus generated tokens exceed max_seq_len");
  s.checkStatus();
  const at::Device device = s.ids.torchTensor().device();
  const at::Tensor tokens = prompt.torchTensor().to(device).contiguous();
  at::Tensor& pos = s.positions.torchTensor();
  pos.fill_(start);
  at::Tensor next;
  // positions are checked above for the whole run, so no step synchronizes with the host
  auto advance = [&](const at::Tensor& in) {
    s.ids.torchTensor().copy_(in);
    TensorMap out = s.run();
    next = out.at("next_ids").torchTensor().clone();
    pos.add_(1);
  };
  for (std::int64_t t = 0; t < length; ++t) advance(tokens.select(1, t));
  std::vector<at::Tensor> generated;
  generated.reserve(static_cast<std::size_t>(steps));
  for (std::int64_t i = 0; i < steps; ++i) {
    generated.push_back(next);
    if (i + 1 < steps) advance(next);
  }
  Tensor result(at::stack(generated, 1).cpu());  // synchronizes
  s.checkStatus();
  return result;
}

}  // namespace dli
