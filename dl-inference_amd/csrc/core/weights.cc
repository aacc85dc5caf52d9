// dli.weights.v1 loader: a JSON manifest {format, data, tensors{name: {dtype, shape, offset,
// nbytes}}} plus one binary blob (reference: src/weights.cc:242-272, written by
// python/dli_export/weights.py:18-62). The blob is read once, straight into each tensor's
// host storage; device tensors are then copied over in one transfer each.
#include "dli/weights.h"

#include <cstdio>
#include <filesystem>
#include <memory>
#include <stdexcept>

#include "json.h"

namespace dli {
namespace {

struct FileCloser {
  void operator()(std::FILE* f) const {
    if (f) std::fclose(f);
  }
};

std::int64_t intField(const json::Value& v, const std::string& field) {
  if (v.kind != json::Value::Kind::Int)
    throw std::invalid_argument("JSON field must be integer: " + field);
  return v.i;
}

}  // namespace

TensorMap loadWeights(const std::string& manifest_path, DeviceType device, int device_id) {
  const std::filesystem::path manifest(manifest_path);
  const json::Value root = json::parse(json::readFile(manifest_path, "weights manifest"));
  if (!root.isObject()) throw std::invalid_argument("weights manifest root must be an object");
  const json::Value& format = root.at("format");
  if (!format.isString()) throw std::invalid_argument("JSON field must be string: format");
  if (format.s != "dli.weights.v1")
    throw std::invalid_argument("unsupported weights format: " + format.s);
  const json::Value& data_field = root.at("data");
  if (!data_field.isString()) throw std::invalid_argument("JSON field must be string: data");
  std::filesystem::path data_path(data_field.s);
  if (data_path.is_relative()) data_path = manifest.parent_path() / data_path;
  const json::Value& tensors = root.at("tensors");
  if (!tensors.isObject()) throw std::invalid_argument("weights tensors must be an object");

  std::unique_ptr<std::FILE, FileCloser> file(std::fopen(data_path.c_str(), "rb"));
  if (!file) throw std::runtime_error("failed to open weights data: " + data_path.string());
  std::error_code ec;
  const auto file_size = static_cast<std::size_t>(std::filesystem::file_size(data_path, ec));
  if (ec) throw std::runtime_error("failed to stat weights data: " + data_path.string());

  TensorMap result;
  for (const auto& [name, meta] : tensors.fields) {
    if (!meta.isObject())
      throw std::invalid_argument("weights tensor metadata must be an object: " + name);
    const json::Value& dtype_field = meta.at("dtype");
    if (!dtype_field.isString()) throw std::invalid_argument("JSON field must be string: dtype");
    const DType dtype = dtypeFromString(dtype_field.s);
    const json::Value& shape_field = meta.at("shape");
    if (!shape_field.isArray()) throw std::invalid_argument("JSON field must be integer array: shape");
    std::vector<std::int64_t> shape;
    for (const auto& d : shape_field.items) shape.push_back(intField(d, "shape"));
    const auto offset = static_cast<std::size_t>(intField(meta.at("offset"), "offset"));
    const auto nbytes = static_cast<std::size_t>(intField(meta.at("nbytes"), "nbytes"));
    if (offset > file_size || nbytes > file_size - offset)
      throw std::invalid_argument("weights tensor range exceeds data file: " + name);

    at::Tensor host = at::empty(shape, at::TensorOptions().dtype(toTorchDType(dtype)));
    if (static_cast<std::size_t>(host.numel()) * byteSize(dtype) != nbytes)
      throw std::invalid_argument("weights tensor byte count does not match dtype and shape: " + name);
    if (nbytes > 0) {
      if (std::fseek(file.get(), static_cast<long>(offset), SEEK_SET) != 0 ||
          std::fread(host.data_ptr(), 1, nbytes, file.get()) != nbytes)
        throw std::runtime_error("failed to read weights tensor: " + name);
    }
    if (device == DeviceType::Cpu) {
      result.emplace(name, Tensor(std::move(host)));
    } else {
      result.emplace(name, Tensor(host.to(at::Device(at::kCUDA, device_id))));
    }
  }
  return result;
}

}  // namespace dli
