// Plugin helper functions (reference: src/utils.cc:8-76).
#include "dli/utils.h"

#include <stdexcept>

namespace dli {

std::int64_t product(const std::vector<std::int64_t>& shape, std::size_t begin, std::size_t end) {
  if (end == static_cast<std::size_t>(-1) || end > shape.size()) end = shape.size();
  std::int64_t result = 1;
  for (std::size_t i = begin; i < end; ++i) result *= shape[i];
  return result;
}

unsigned ceilDiv(std::int64_t a, std::int64_t b) {
  return static_cast<unsigned>(a / b + (a % b != 0 ? 1 : 0));
}

std::string formatShape(const std::vector<std::int64_t>& shape) {
  std::string text = "[";
  for (std::size_t i = 0; i < shape.size(); ++i) {
    if (i > 0) text += ',';
    text += std::to_string(shape[i]);
  }
  text += ']';
  return text;
}

void requireCudaInputs(const std::vector<const Tensor*>& inputs, const std::string& op) {
  for (const Tensor* tensor : inputs) {
    if (tensor == nullptr || !tensor->isCuda())
      throw std::invalid_argument(op + " expects CUDA tensors");
  }
}

void requireFloat(const Tensor& tensor, const std::string& op) {
  if (tensor.dtype() != DType::Float32) throw std::invalid_argument(op + " expects float32");
}

void requireFloating(const Tensor& tensor, const std::string& op) {
  if (!isFloating(tensor.dtype()))
    throw std::invalid_argument(op + " expects float32, bfloat16 or float16");
}

void requireSameDType(const Tensor& a, const Tensor& b, const std::string& op) {
  if (a.dtype() != b.dtype())
    throw std::invalid_argument(op + " dtype mismatch: " + toString(a.dtype()) + " vs " +
                                toString(b.dtype()));
}

double attrDouble(const Attributes& attrs, const std::string& name, double fallback) {
  if (!attrs.contains(name)) return fallback;
  const auto& value = attrs.values().at(name);
  if (const auto* as_int = std::get_if<std::int64_t>(&value)) return static_cast<double>(*as_int);
  return attrs.require<double>(name);
}

std::vector<std::int64_t> attrInts(const Attributes& attrs, const std::string& name,
                                   std::vector<std::int64_t> fallback) {
  if (!attrs.contains(name)) return fallback;
  return attrs.require<std::vector<std::int64_t>>(name);
}

void* ptr(const Tensor& tensor) { return const_cast<void*>(tensor.deviceData()); }

std::vector<std::int64_t> reshapeShape(const std::vector<std::int64_t>& input,
                                       std::vector<std::int64_t> target) {
  std::size_t inferred = target.size();
  std::int64_t fixed = 1;
  for (std::size_t i = 0; i < target.size(); ++i) {
    const std::int64_t d = target[i];
    if (d == -1) {
      if (inferred != target.size())
        throw std::invalid_argument("reshape has multiple inferred dimensions");
      inferred = i;
      continue;
    }
    if (d <= 0) throw std::invalid_argument("reshape dimension must be positive or -1");
    fixed *= d;
  }
  const std::int64_t total = product(input);
  if (inferred != target.size()) {
    if (total % fixed != 0)
      throw std::invalid_argument("reshape inferred dimension is not integral");
    target[inferred] = total / fixed;
  }
  if (product(target) != total) throw std::invalid_argument("reshape changes element count");
  return target;
}

}  // namespace dli
