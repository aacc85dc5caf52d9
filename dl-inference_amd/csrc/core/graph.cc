// dli.graph.v1 reader/writer.
// Format and attribute typing follow src/graph.cc:230-273 and 327-409 of the reference:
//  - a node names its operator with "op" or, failing that, "op_type";
//  - attrs: bool -> bool, integer literal -> int64, other number -> double, string -> string,
//    arrays are homogeneous: all strings -> [string], all integers -> [int64], any mix of
//    numbers -> [double]; an empty array is [int64].
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <type_traits>

#include "dli/graph.h"
#include "json.h"

namespace dli {
namespace {

std::string stringField(const json::Value& v, const std::string& field) {
  if (!v.isString()) throw std::invalid_argument("JSON field must be string: " + field);
  return v.s;
}

std::vector<std::string> stringList(const json::Value& v, const std::string& field) {
  if (!v.isArray()) throw std::invalid_argument("JSON field must be string array: " + field);
  std::vector<std::string> out;
  out.reserve(v.items.size());
  for (const auto& item : v.items) out.push_back(stringField(item, field));
  return out;
}

AttributeValue attributeFrom(const json::Value& v, const std::string& name) {
  using K = json::Value::Kind;
  switch (v.kind) {
    case K::Bool: return v.b;
    case K::Int: return v.i;
    case K::Double: return v.d;
    case K::String: return v.s;
    case K::Array: {
      bool strings = true, ints = true, numbers = true;
      for (const auto& item : v.items) {
        strings &= item.kind == K::String;
        ints &= item.kind == K::Int;
        numbers &= item.isNumber();
      }
      if (v.items.empty() || ints) {
        std::vector<std::int64_t> out;
        for (const auto& item : v.items) out.push_back(item.i);
        return out;
      }
      if (strings) {
        std::vector<std::string> out;
        for (const auto& item : v.items) out.push_back(item.s);
        return out;
      }
      if (numbers) {
        std::vector<double> out;
        for (const auto& item : v.items)
          out.push_back(item.kind == K::Int ? static_cast<double>(item.i) : item.d);
        return out;
      }
      break;
    }
    default: break;
  }
  throw std::invalid_argument("unsupported attribute JSON value: " + name);
}

void writeStrings(std::ostringstream& out, const std::vector<std::string>& items) {
  out << '[';
  for (std::size_t i = 0; i < items.size(); ++i) out << (i ? "," : "") << json::quote(items[i]);
  out << ']';
}

void writeAttribute(std::ostringstream& out, const AttributeValue& value) {
  std::visit(
      [&out](const auto& v) {
        using T = std::decay_t<decltype(v)>;
        if constexpr (std::is_same_v<T, bool>) {
          out << (v ? "true" : "false");
        } else if constexpr (std::is_same_v<T, std::int64_t>) {
          out << v;
        } else if constexpr (std::is_same_v<T, double>) {
          out << json::formatDouble(v);
        } else if constexpr (std::is_same_v<T, std::string>) {
          out << json::quote(v);
        } else if constexpr (std::is_same_v<T, std::vector<std::string>>) {
          writeStrings(out, v);
        } else if constexpr (std::is_same_v<T, std::vector<double>>) {
          out << '[';
          for (std::size_t i = 0; i < v.size(); ++i) out << (i ? "," : "") << json::formatDouble(v[i]);
          out << ']';
        } else {
          out << '[';
          for (std::size_t i = 0; i < v.size(); ++i) out << (i ? "," : "") << v[i];
          out << ']';
        }
      },
      value);
}

}  // namespace

Graph Graph::fromJson(const std::string& text) {
  const json::Value root = json::parse(text);
  if (!root.isObject()) throw std::invalid_argument("graph JSON root must be an object");
  Graph graph;
  if (const auto* v = root.find("format")) graph.format = stringField(*v, "format");
  if (graph.format != "dli.graph.v1")
    throw std::invalid_argument("unsupported graph format: " + graph.format);
  if (const auto* v = root.find("model_type")) graph.model_type = stringField(*v, "model_type");
  if (const auto* v = root.find("weights")) graph.weights = stringField(*v, "weights");
  if (const auto* v = root.find("inputs")) graph.inputs = stringList(*v, "inputs");
  if (const auto* v = root.find("outputs")) graph.outputs = stringList(*v, "outputs");

  const json::Value& nodes = root.at("nodes");
  if (!nodes.isArray()) throw std::invalid_argument("graph nodes must be an array");
  graph.nodes.reserve(nodes.items.size());
  for (const auto& item : nodes.items) {
    if (!item.isObject()) throw std::invalid_argument("graph node must be an object");
    Node node;
    node.name = stringField(item.at("name"), "name");
    const json::Value* op = item.find("op");
    node.op_type = op ? stringField(*op, "op") : stringField(item.at("op_type"), "op_type");
    node.inputs = stringList(item.at("inputs"), "inputs");
    node.outputs = stringList(item.at("outputs"), "outputs");
    if (const auto* attrs = item.find("attrs")) {
      if (!attrs->isObject()) throw std::invalid_argument("node attrs must be an object");
      for (const auto& [key, value] : attrs->fields) node.attributes.set(key, attributeFrom(value, key));
    }
    graph.nodes.push_back(std::move(node));
  }
  return graph;
}

Graph Graph::fromJsonFile(const std::string& path) {
  std::ifstream probe(path);
  if (!probe) throw std::runtime_error("failed to open graph file: " + path);
  return fromJson(json::readFile(path, "graph file"));
}

std::string Graph::toJson() const {
  std::ostringstream out;
  out << "{\n  \"format\":" << json::quote(format) << ",\n  \"model_type\":" << json::quote(model_type)
      << ",\n";
  if (!weights.empty()) out << "  \"weights\":" << json::quote(weights) << ",\n";
  out << "  \"inputs\":";
  writeStrings(out, inputs);
  out << ",\n  \"outputs\":";
  writeStrings(out, outputs);
  out << ",\n  \"nodes\":[";
  for (std::size_t n = 0; n < nodes.size(); ++n) {
    const Node& node = nodes[n];
    out << (n ? ",\n    " : "\n    ") << "{\"name\":" << json::quote(node.name)
        << ",\"op\":" << json::quote(node.op_type) << ",\"inputs\":";
    writeStrings(out, node.inputs);
    out << ",\"outputs\":";
    writeStrings(out, node.outputs);
    out << ",\"attrs\":{";
    bool first = true;
    for (const auto& [key, value] : node.attributes.values()) {
      out << (first ? "" : ",") << json::quote(key) << ':';
      writeAttribute(out, value);
      first = false;
    }
    out << "}}";
  }
  out << "\n  ]\n}\n";
  return out.str();
}

}  // namespace dli
