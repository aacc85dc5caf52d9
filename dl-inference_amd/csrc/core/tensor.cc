// dli::Tensor over ATen storage (reference behaviour: src/tensor.cc:52-248).
#include "dli/tensor.h"

#include <limits>
#include <utility>

namespace dli {

struct Tensor::Impl {
  explicit Impl(at::Tensor t) : tensor(std::move(t)) {}
  at::Tensor tensor;
};

at::ScalarType toTorchDType(DType dtype) {
  switch (dtype) {
    case DType::Float32: return at::kFloat;
    case DType::Int64: return at::kLong;
    case DType::BFloat16: return at::kBFloat16;
    case DType::Float16: return at::kHalf;
    case DType::Int32: return at::kInt;
  }
  throw std::invalid_argument("unknown dtype");
}

DType fromTorchDType(at::ScalarType dtype) {
  switch (dtype) {
    case at::kFloat: return DType::Float32;
    case at::kLong: return DType::Int64;
    case at::kBFloat16: return DType::BFloat16;
    case at::kHalf: return DType::Float16;
    case at::kInt: return DType::Int32;
    default: break;
  }
  throw std::invalid_argument(std::string("unsupported torch tensor dtype: ") +
                              c10::toString(dtype));
}

namespace {

DeviceType deviceOf(const at::Tensor& t) {
  if (t.device().is_cpu()) return DeviceType::Cpu;
  if (t.device().is_cuda()) return DeviceType::Cuda;
  throw std::invalid_argument("unsupported torch tensor device: " + t.device().str());
}

at::TensorOptions optionsFor(DType dtype, DeviceType device, int device_id) {
  auto options = at::TensorOptions().dtype(toTorchDType(dtype));
  return device == DeviceType::Cpu ? options.device(at::kCPU)
                                   : options.device(at::Device(at::kCUDA, device_id));
}

void validateShape(std::vector<std::int64_t>& shape) {
  if (shape.empty()) shape.push_back(1);
  for (std::int64_t d : shape)
    if (d < 0) throw std::invalid_argument("negative tensor dimension");
}

template <typename T>
DType dtypeOf();
template <>
DType dtypeOf<float>() { return DType::Float32; }
template <>
DType dtypeOf<std::int64_t>() { return DType::Int64; }
template <>
DType dtypeOf<std::int32_t>() { return DType::Int32; }
template <>
DType dtypeOf<at::BFloat16>() { return DType::BFloat16; }
template <>
DType dtypeOf<at::Half>() { return DType::Float16; }

}  // namespace

std::string toString(DeviceType device) {
  switch (device) {
    case DeviceType::Cpu: return "cpu";
    case DeviceType::Cuda: return "cuda";
  }
  throw std::invalid_argument("unknown device type");
}

DeviceType deviceFromString(const std::string& device) {
  if (device == "cpu") return DeviceType::Cpu;
  if (device == "cuda" || device == "gpu" || device == "hip") return DeviceType::Cuda;
  throw std::invalid_argument("unsupported device type: " + device);
}

std::string toString(DType dtype) {
  switch (dtype) {
    case DType::Float32: return "float32";
    case DType::Int64: return "int64";
    case DType::BFloat16: return "bfloat16";
    case DType::Float16: return "float16";
    case DType::Int32: return "int32";
  }
  throw std::invalid_argument("unknown dtype");
}

DType dtypeFromString(const std::string& dtype) {
  if (dtype == "float32" || dtype == "f32") return DType::Float32;
  if (dtype == "int64" || dtype == "i64") return DType::Int64;
  if (dtype == "bfloat16" || dtype == "bf16") return DType::BFloat16;
  if (dtype == "float16" || dtype == "f16") return DType::Float16;
  if (dtype == "int32" || dtype == "i32") return DType::Int32;
  throw std::invalid_argument("unsupported dtype: " + dtype);
}

std::size_t byteSize(DType dtype) {
  switch (dtype) {
    case DType::Float32: return 4;
    case DType::Int64: return 8;
    case DType::BFloat16: return 2;
    case DType::Float16: return 2;
    case DType::Int32: return 4;
  }
  throw std::invalid_argument("unknown dtype");
}

bool isFloating(DType dtype) {
  return dtype == DType::Float32 || dtype == DType::BFloat16 || dtype == DType::Float16;
}

Tensor::Tensor(std::shared_ptr<Impl> impl) : impl_(std::move(impl)) {
  const at::Tensor& t = impl_->tensor;
  dtype_ = fromTorchDType(t.scalar_type());
  device_ = deviceOf(t);
  device_id_ = t.device().is_cuda() ? static_cast<int>(t.device().index()) : 0;
  shape_.assign(t.sizes().begin(), t.sizes().end());
  if (shape_.empty()) shape_.push_back(1);
}

Tensor::Tensor(at::Tensor tensor)
    : Tensor(std::make_shared<Impl>(tensor.is_contiguous() ? std::move(tensor)
                                                           : tensor.contiguous())) {}

Tensor::Tensor(DType dtype, std::vector<std::int64_t> shape) {
  validateShape(shape);
  *this = Tensor(std::make_shared<Impl>(at::zeros(shape, optionsFor(dtype, DeviceType::Cpu, 0))));
}

const Tensor::Impl& Tensor::impl() const {
  if (!impl_) throw std::logic_error("tensor is uninitialized");
  return *impl_;
}

Tensor::Impl& Tensor::impl() {
  if (!impl_) throw std::logic_error("tensor is uninitialized");
  return *impl_;
}

Tensor Tensor::zeros(DType dtype, std::vector<std::int64_t> shape) {
  return Tensor(dtype, std::move(shape));
}

Tensor Tensor::cuda(DType dtype, std::vector<std::int64_t> shape, int device_id) {
  validateShape(shape);
  return Tensor(
      std::make_shared<Impl>(at::empty(shape, optionsFor(dtype, DeviceType::Cuda, device_id))));
}

Tensor Tensor::externalCuda(DType dtype, std::vector<std::int64_t> shape, void* data,
                            int device_id) {
  if (data == nullptr) throw std::invalid_argument("external CUDA tensor pointer is null");
  validateShape(shape);
  Tensor tensor;
  tensor.dtype_ = dtype;
  tensor.device_ = DeviceType::Cuda;
  tensor.device_id_ = device_id;
  tensor.shape_ = std::move(shape);
  tensor.external_device_ptr_ = data;
  return tensor;
}

std::int64_t Tensor::dim(std::size_t index) const {
  if (index >= shape_.size()) throw std::out_of_range("tensor dimension out of range");
  return shape_[index];
}

std::size_t Tensor::numel() const {
  if (impl_) return static_cast<std::size_t>(impl_->tensor.numel());
  std::size_t count = 1;
  for (std::int64_t d : shape_) {
    if (d == 0) return 0;
    const auto ud = static_cast<std::size_t>(d);
    if (count > std::numeric_limits<std::size_t>::max() / ud)
      throw std::overflow_error("tensor shape is too large");
    count *= ud;
  }
  return count;
}

std::size_t Tensor::nbytes() const { return numel() * byteSize(dtype_); }

void* Tensor::deviceData() {
  if (device_ != DeviceType::Cuda) throw std::logic_error("tensor is not on CUDA");
  return impl_ ? impl_->tensor.data_ptr() : external_device_ptr_;
}

const void* Tensor::deviceData() const {
  if (device_ != DeviceType::Cuda) throw std::logic_error("tensor is not on CUDA");
  return impl_ ? impl_->tensor.data_ptr() : external_device_ptr_;
}

Tensor Tensor::withShape(std::vector<std::int64_t> shape) const {
  validateShape(shape);
  std::size_t count = 1;
  for (std::int64_t d : shape) count *= static_cast<std::size_t>(d);
  if (count != numel()) throw std::invalid_argument("tensor view changes element count");
  if (!impl_) {
    Tensor view = *this;
    view.shape_ = std::move(shape);
    return view;
  }
  return Tensor(std::make_shared<Impl>(impl_->tensor.view(shape)));
}

at::Tensor& Tensor::torchTensor() { return impl().tensor; }
const at::Tensor& Tensor::torchTensor() const { return impl().tensor; }

template <typename T>
T* Tensor::data() {
  if (!isCpu()) throw std::logic_error("host data access requested for non-CPU tensor");
  if (dtype_ != dtypeOf<T>()) throw std::logic_error("tensor dtype does not match requested host type");
  return static_cast<T*>(impl().tensor.data_ptr());
}

template <typename T>
const T* Tensor::data() const {
  if (!isCpu()) throw std::logic_error("host data access requested for non-CPU tensor");
  if (dtype_ != dtypeOf<T>()) throw std::logic_error("tensor dtype does not match requested host type");
  return static_cast<const T*>(impl().tensor.data_ptr());
}

template float* Tensor::data<float>();
template const float* Tensor::data<float>() const;
template std::int64_t* Tensor::data<std::int64_t>();
template const std::int64_t* Tensor::data<std::int64_t>() const;
template std::int32_t* Tensor::data<std::int32_t>();
template const std::int32_t* Tensor::data<std::int32_t>() const;
template at::BFloat16* Tensor::data<at::BFloat16>();
template const at::BFloat16* Tensor::data<at::BFloat16>() const;
template at::Half* Tensor::data<at::Half>();
template const at::Half* Tensor::data<at::Half>() const;

bool sameShape(const Tensor& lhs, const Tensor& rhs) { return lhs.shape() == rhs.shape(); }

std::size_t contiguousOffset(const std::vector<std::int64_t>& shape,
                             const std::vector<std::int64_t>& indices) {
  if (shape.size() != indices.size())
    throw std::invalid_argument("rank mismatch in contiguousOffset");
  std::size_t offset = 0;
  for (std::size_t i = 0; i < shape.size(); ++i) {
    if (indices[i] < 0 || indices[i] >= shape[i])
      throw std::out_of_range("tensor index out of range");
    offset = offset * static_cast<std::size_t>(shape[i]) + static_cast<std::size_t>(indices[i]);
  }
  return offset;
}

}  // namespace dli
