// Python module _dli_native (reference surface: src/python_bindings.cc:49-85): Graph,
// Engine.load_library / run, load_weights. Additions: Engine.run(..., stream=, profile=)
// (hipStream_t as int, so kernels join torch's current stream; a ProfileSession, the
// reference's .codex/profiling_design.md), registry and KV-cache controls, and
// load_weights(device_id=), and the C++ greedy decode driver (GreedyDecoder).
#include <ATen/ATen.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/csrc/utils/pybind.h>

#include <cstdint>
#include <utility>

#include "dli/engine.h"
#include "dli/graph.h"
#include "dli/greedy.h"
#include "dli/logging.h"
#include "dli/profiler.h"
#include "dli/tensor.h"
#include "dli/weights.h"

namespace py = pybind11;

namespace {

dli::TensorMap toTensorMap(const py::dict& tensors) {
  dli::TensorMap map;
  for (const auto& item : tensors)
    map.emplace(py::cast<std::string>(item.first), dli::Tensor(py::cast<at::Tensor>(item.second)));
  return map;
}

py::dict toDict(const dli::TensorMap& tensors) {
  py::dict out;
  for (const auto& [name, tensor] : tensors) out[py::str(name)] = py::cast(tensor.torchTensor());
  return out;
}

void* streamFrom(std::uintptr_t value) { return reinterpret_cast<void*>(value); }

}  // namespace

PYBIND11_MODULE(_dli_native, m) {
  m.doc() = "dl-inference C++ graph engine with the gfx950 operator plugin ABI";

  py::class_<dli::Node>(m, "Node")
      .def_readonly("name", &dli::Node::name)
      .def_readonly("op_type", &dli::Node::op_type)
      .def_readonly("inputs", &dli::Node::inputs)
      .def_readonly("outputs", &dli::Node::outputs);

  py::class_<dli::Graph>(m, "Graph")
      .def(py::init<>())
      .def_static("from_json", &dli::Graph::fromJson, py::arg("json"))
      .def_static("from_json_file", &dli::Graph::fromJsonFile, py::arg("path"))
      .def("to_json", &dli::Graph::toJson)
      .def_readwrite("format", &dli::Graph::format)
      .def_readwrite("model_type", &dli::Graph::model_type)
      .def_readwrite("weights", &dli::Graph::weights)
      .def_readwrite("inputs", &dli::Graph::inputs)
      .def_readwrite("outputs", &dli::Graph::outputs)
      .def_property_readonly("nodes", [](const dli::Graph& g) { return g.nodes; });

  py::class_<dli::ProfileSession>(m, "ProfileSession")
      .def(py::init([](bool cpu, bool gpu, bool record_shapes, std::size_t max_events) {
             dli::ProfileConfig config;
             config.cpu = cpu;
             config.gpu = gpu;
             config.record_shapes = record_shapes;
             config.max_events = max_events;
             return new dli::ProfileSession(config);
           }),
           py::arg("cpu") = true, py::arg("gpu") = true, py::arg("record_shapes") = false,
           py::arg("max_events") = 1000000)
      .def(
          "finalize",
          [](dli::ProfileSession& s) {
            py::gil_scoped_release release;
            s.finalize();
          })
      .def_property_readonly("finalized", &dli::ProfileSession::finalized)
      .def("to_json", &dli::ProfileSession::toJson)
      .def("write_json", &dli::ProfileSession::writeJson, py::arg("path"));

  py::class_<dli::Engine>(m, "Engine")
      .def(py::init<>())
      .def(
          "load_library",
          [](dli::Engine& engine, const std::string& path) -> dli::Engine& {
            engine.registry().loadLibrary(path);
            return engine;
          },
          py::arg("path"), py::return_value_policy::reference_internal)
      .def(
          "run",
          [](dli::Engine& engine, const dli::Graph& graph, const py::dict& inputs,
             std::uintptr_t stream, dli::ProfileSession* profile) {
            auto tensors = toTensorMap(inputs);
            dli::TensorMap result;
            {
              py::gil_scoped_release release;
              engine.setStream(streamFrom(stream));
              result = engine.run(graph, std::move(tensors), dli::RunOptions{profile});
            }
            return toDict(result);
          },
          py::arg("graph"), py::arg("inputs"), py::arg("stream") = 0,
          py::arg("profile") = nullptr)
      .def("has_operator",
           [](const dli::Engine& e, const std::string& name) { return e.registry().contains(name); })
      .def("operator_names", [](const dli::Engine& e) { return e.registry().names(); })
      .def(
          "configure_kv_cache",
          [](dli::Engine& e, std::int64_t block_size, std::int64_t max_seq_len) {
            e.kvCache().configure(block_size, max_seq_len);
          },
          py::arg("block_size") = 64, py::arg("max_seq_len") = 4096)
      .def("clear_kv_cache", [](dli::Engine& e) { e.kvCache().clear(); })
      .def("kv_cache_size", [](const dli::Engine& e) { return e.kvCache().size(); })
      .def("set_kv_cache_length",
           [](dli::Engine& e, std::int64_t length) { e.kvCache().setLength(length); })
      .def(
          "kv_cache_entry",
          [](dli::Engine& e, const std::string& name) -> py::object {
            const dli::KVCacheEntry* entry = e.kvCache().get(name);
            if (entry == nullptr) return py::none();
            py::dict d;
            d["key_pool"] = py::cast(entry->key_pool.torchTensor());
            d["value_pool"] = py::cast(entry->value_pool.torchTensor());
            d["block_table"] = py::cast(entry->block_table.torchTensor());
            d["block_size"] = entry->block_size;
            d["max_blocks"] = entry->max_blocks;
            d["length"] = entry->length;
            return d;
          },
          py::arg("name"))
      .def(
          "reserve_kv_cache",
          [](dli::Engine& e, const std::string& name, const std::string& dtype, std::int64_t batch,
             std::int64_t heads, std::int64_t head_dim, int device_id) {
            e.kvCache().reserve(name, dli::dtypeFromString(dtype), batch, heads, head_dim,
                                device_id);
          },
          py::arg("name"), py::arg("dtype"), py::arg("batch"), py::arg("heads"),
          py::arg("head_dim"), py::arg("device_id") = 0);

  py::class_<dli::GreedyDecoder>(m, "GreedyDecoder")
      .def(py::init([](dli::Engine& engine, const dli::Graph& graph, const py::dict& weights,
                       std::int64_t batch, std::int64_t block_size, std::int64_t max_seq_len,
                       bool capture) {
             auto tensors = toTensorMap(weights);
             py::gil_scoped_release release;
             return std::make_unique<dli::GreedyDecoder>(
                 engine, graph, std::move(tensors), batch,
                 dli::GreedyOptions{block_size, max_seq_len, capture});
           }),
           py::arg("engine"), py::arg("graph"), py::arg("weights"), py::arg("batch"),
           py::arg("block_size") = 64, py::arg("max_seq_len") = 4096, py::arg("capture") = true,
           py::keep_alive<1, 2>())
      .def_property_readonly("batch", &dli::GreedyDecoder::batch)
      .def_property_readonly("captured", &dli::GreedyDecoder::captured)
      .def(
          "step",
          [](dli::GreedyDecoder& d, const at::Tensor& ids, const at::Tensor& positions) {
            dli::TensorMap out;
            {
              py::gil_scoped_release release;
              out = d.step(dli::Tensor(ids), dli::Tensor(positions));
            }
            return toDict(out);
          },
          py::arg("ids"), py::arg("positions"))
      .def(
          "generate",
          [](dli::GreedyDecoder& d, const at::Tensor& prompt, std::int64_t steps,
             std::int64_t start) {
            dli::Tensor out;
            {
              py::gil_scoped_release release;
              out = d.generate(dli::Tensor(prompt), steps, start);
            }
            return out.torchTensor();
          },
          py::arg("prompt"), py::arg("steps"), py::arg("start") = 0)
      .def("check_status", &dli::GreedyDecoder::checkStatus,
           py::call_guard<py::gil_scoped_release>());

  m.def(
      "load_weights",
      [](const std::string& path, const std::string& device, int device_id) {
        return toDict(dli::loadWeights(path, dli::deviceFromString(device), device_id));
      },
      py::arg("path"), py::arg("device") = "cpu", py::arg("device_id") = 0);

  m.def("set_log_level", [](const std::string& level) {
    if (level == "debug") dli::setLogLevel(dli::LogSeverity::Debug);
    else if (level == "info") dli::setLogLevel(dli::LogSeverity::Info);
    else if (level == "warn") dli::setLogLevel(dli::LogSeverity::Warn);
    else if (level == "error") dli::setLogLevel(dli::LogSeverity::Error);
    else throw std::invalid_argument("unknown log level: " + level);
  });
}
