// dli_operator_engine_runner: one dli.graph.v1 graph through the C++ Engine and a plugin, with
// no Python anywhere (the reference's tests/operator_engine_runner.cc:114-137 drives its
// per-operator tests the same way).
//
//   dli_operator_engine_runner --graph g.json --inputs x.dli.weights.json --plugin lib.so
//                              --output-dir DIR [--device cuda|cpu]
//
// The inputs are a dli.weights.v1 manifest (loaded to the device, like the reference's runner),
// the plugin is dlopen'd through OperatorRegistry::loadLibrary, and every graph output is written
// to DIR/<name>.bin (raw little-endian elements, row-major) and listed in DIR/outputs.json:
//   {"format": "dli.outputs.v1", "tensors": {"<name>": {"dtype": ..., "shape": [...],
//    "file": "<name>.bin"}, ...}}
// Exit status 0 on success; 1 with "operator engine runner failed: <reason>" on stderr.
#include <ATen/ATen.h>

#include <cctype>
#include <cstdio>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "dli/engine.h"
#include "dli/graph.h"
#include "dli/tensor.h"
#include "dli/weights.h"

namespace fs = std::filesystem;

namespace {

struct Options {
  std::map<std::string, std::string> values{{"--device", "cuda"}};

  const std::string& operator[](const std::string& key) const { return values.at(key); }
};

Options parse(int argc, char** argv) {
  static const char* kUsage =
      "usage: dli_operator_engine_runner --graph path --inputs path --plugin path "
      "--output-dir path [--device cuda|cpu]";
  Options opt;
  for (int i = 1; i < argc; i += 2) {
    const std::string key = argv[i];
    const bool known = key == "--graph" || key == "--inputs" || key == "--plugin" ||
                       key == "--output-dir" || key == "--device";
    if (!known || i + 1 >= argc) throw std::invalid_argument(kUsage);
    opt.values[key] = argv[i + 1];
  }
  for (const char* key : {"--graph", "--inputs", "--plugin", "--output-dir"})
    if (opt.values.count(key) == 0 || opt.values.at(key).empty())
      throw std::invalid_argument(std::string("missing ") + key + "; " + kUsage);
  const std::string& device = opt["--device"];
  if (device != "cuda" && device != "cpu") throw std::invalid_argument(kUsage);
  return opt;
}

// Output names become file names: letters, digits, '_', '-' and '.' only, not starting with '.'.
std::string fileFor(const std::string& name) {
  bool ok = !name.empty() && name.front() != '.';
  for (char c : name)
    ok = ok && (std::isalnum(static_cast<unsigned char>(c)) || c == '_' || c == '-' || c == '.');
  if (!ok) throw std::invalid_argument("output name cannot be a file name: " + name);
  return name + ".bin";
}

std::string jsonString(const std::string& s) {
  std::string out = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') out += '\\';
    out += c;
  }
  return out + "\"";
}

// The tensor's elements on the host, contiguous (a device tensor is copied back through ATen).
at::Tensor hostCopy(const dli::Tensor& t) {
  return t.torchTensor().to(at::kCPU).contiguous();
}

void writeOutputs(const fs::path& dir, const dli::Graph& graph, const dli::TensorMap& result) {
  std::string manifest = "{\n  \"format\": \"dli.outputs.v1\",\n  \"tensors\": {";
  const char* sep = "\n";
  for (const std::string& name : graph.outputs) {
    auto it = result.find(name);
    if (it == result.end()) throw std::runtime_error("graph output was not produced: " + name);
    const dli::Tensor& t = it->second;
    const std::string file = fileFor(name);
    const at::Tensor host = hostCopy(t);
    std::ofstream out(dir / file, std::ios::binary);
    if (!out) throw std::runtime_error("cannot write " + (dir / file).string());
    out.write(static_cast<const char*>(host.data_ptr()), static_cast<std::streamsize>(host.nbytes()));
    if (!out) throw std::runtime_error("short write to " + (dir / file).string());
    std::string shape;
    for (std::size_t i = 0; i < t.shape().size(); ++i)
      shape += (i ? ", " : "") + std::to_string(t.shape()[i]);
    manifest += sep;
    manifest += "    " + jsonString(name) + ": {\"dtype\": " + jsonString(dli::toString(t.dtype())) +
                ", \"shape\": [" + shape + "], \"file\": " + jsonString(file) + "}";
    sep = ",\n";
  }
  manifest += "\n  }\n}\n";
  std::ofstream out(dir / "outputs.json");
  if (!out || !(out << manifest)) throw std::runtime_error("cannot write outputs.json");
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const Options opt = parse(argc, argv);
    const fs::path dir(opt["--output-dir"]);
    fs::create_directories(dir);
    const dli::Graph graph = dli::Graph::fromJsonFile(opt["--graph"]);
    const auto device = opt["--device"] == "cuda" ? dli::DeviceType::Cuda : dli::DeviceType::Cpu;
    dli::TensorMap inputs = dli::loadWeights(opt["--inputs"], device);
    dli::Engine engine;
    engine.registry().loadLibrary(opt["--plugin"]);
    const dli::TensorMap result = engine.run(graph, std::move(inputs));
    writeOutputs(dir, graph, result);
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "operator engine runner failed: " << e.what() << "\n";
    return 1;
  }
}
