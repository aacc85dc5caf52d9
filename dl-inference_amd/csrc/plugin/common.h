#pragma once

// Shared helpers for the gfx950 operator plugin: dtype mapping to the device C ABI, error
// translation (device status -> std::runtime_error, as the reference's CUDA wrappers throw),
// and operator registration.

#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "dli/operator.h"
#include "dli/utils.h"
#include "dli_hip.h"

namespace dli::plugin {

inline int hipDtype(DType dtype) {
  switch (dtype) {
    case DType::Float32: return DLI_F32;
    case DType::Int64: return DLI_I64;
    case DType::BFloat16: return DLI_BF16;
    case DType::Float16: return DLI_F16;
    case DType::Int32: return DLI_I32;
  }
  throw std::invalid_argument("unknown dtype");
}

inline void check(int rc, const std::string& op) {
  if (rc == DLI_HIP_EINVAL) throw std::invalid_argument(op + ": " + dli_hip_last_error());
  if (rc != 0) throw std::runtime_error(op + ": " + dli_hip_last_error());
}

inline void requireArity(const std::vector<const Tensor*>& inputs,
                         const std::vector<Tensor*>& outputs, std::size_t min_in,
                         std::size_t max_in, std::size_t n_out, const std::string& op) {
  if (inputs.size() < min_in || inputs.size() > max_in || outputs.size() != n_out)
    throw std::invalid_argument(op + " arity");
  for (const Tensor* t : inputs)
    if (t == nullptr) throw std::invalid_argument(op + " received a null input");
  for (Tensor* t : outputs)
    if (t == nullptr) throw std::invalid_argument(op + " received a null output");
}

inline void requireIndex(const Tensor& t, const std::string& op, const std::string& what) {
  if (t.dtype() != DType::Int64 && t.dtype() != DType::Int32)
    throw std::invalid_argument(op + " " + what + " must be int64 or int32");
}

inline std::vector<std::int64_t> withLast(std::vector<std::int64_t> shape, std::int64_t last) {
  shape.back() = last;
  return shape;
}

// Zero-initialised device scratch kept across calls of one operator instance (split-K partials,
// attention partials and the arrival counters that kernels leave at zero; the nodes of one
// operator instance run in stream order). Allocated on first use, outside any captured region
// in a decode session, and replaced by a larger zeroed buffer when a node needs more. A replaced
// buffer is kept alive with the operator (the engine caches one operator per type, so a HIP
// graph captured earlier may still point at it), and the device is synchronized after the
// zero fill, which runs on torch's current stream, before any kernel on another stream uses it.
class PersistentWorkspace {
 public:
  // The node's buffer of at least `bytes`, zero-filled when first made (or grown). Making it
  // allocates and synchronizes the device, which a stream under capture cannot do: such a call
  // is refused with std::runtime_error (run the graph once eagerly before capturing it, as
  // DecodeSession and GreedyDecoder do, so every node has its buffer).
  void* get(std::size_t bytes, int device_id, void* stream) {
    if (bytes == 0) return nullptr;
    std::lock_guard<std::mutex> lock(mutex_);
    if (!buffer_.defined() || buffer_.nbytes() < bytes || buffer_.deviceId() != device_id) {
      int capturing = 0;
      if (int rc = dli_hip_stream_is_capturing(stream, &capturing))
        throw std::runtime_error(std::string("workspace: ") + dli_hip_last_error() + " (" +
                                 std::to_string(rc) + ")");
      if (capturing != 0)
        throw std::runtime_error(
            "workspace: the first use of this node's scratch buffer is inside a stream capture; "
            "run the graph once without capture first (the buffer is allocated and zero-filled "
            "then, and reused by the captured graph)");
      const auto words = static_cast<std::int64_t>((bytes + 3) / 4);
      if (buffer_.defined()) retired_.push_back(buffer_);
      buffer_ = Tensor(at::zeros({words}, at::TensorOptions().dtype(at::kInt).device(at::kCUDA, device_id)));
      if (int rc = dli_hip_device_synchronize())
        throw std::runtime_error(std::string("workspace zero fill: ") + dli_hip_last_error() +
                                 " (" + std::to_string(rc) + ")");
    }
    return buffer_.deviceData();
  }

  // The current buffer (int32 words); undefined before the first get().
  Tensor tensor() const {
    std::lock_guard<std::mutex> lock(mutex_);
    return buffer_;
  }

 private:
  mutable std::mutex mutex_;
  Tensor buffer_;
  std::vector<Tensor> retired_;
};

template <typename Op>
void add(OperatorRegistry* registry) {
  registry->registerFactory(Op().type(), [] { return std::make_unique<Op>(); });
}

// Registration hooks of the plugin's source files.
void registerReferenceOps(OperatorRegistry* registry);
void registerFusedOps(OperatorRegistry* registry);

}  // namespace dli::plugin
