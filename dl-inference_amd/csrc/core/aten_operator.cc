// The "aten" operator (reference behaviour: src/aten_operator.cc:61-113).
// attrs: name (e.g. "aten::add"), overload (default ""), attr_order (names of further attrs
// pushed after the tensor inputs, in schema order). Returns are a Tensor, a TensorList or a
// tuple of Tensors and must match the node's output count.
#include "dli/aten_operator.h"

#include <ATen/core/dispatch/Dispatcher.h>
#include <ATen/core/ivalue.h>

#include <stdexcept>

namespace dli {
namespace {

c10::IValue toIValue(const AttributeValue& value) {
  return std::visit([](const auto& v) { return c10::IValue(v); }, value);
}

void flattenReturn(const c10::IValue& value, std::vector<at::Tensor>& out) {
  if (value.isTensor()) {
    out.push_back(value.toTensor());
  } else if (value.isTensorList()) {
    for (const at::Tensor& t : value.toTensorVector()) out.push_back(t);
  } else if (value.isTuple()) {
    for (const c10::IValue& item : value.toTupleRef().elements()) {
      if (!item.isTensor()) throw std::invalid_argument("aten tuple output contains non-tensor value");
      out.push_back(item.toTensor());
    }
  } else {
    throw std::invalid_argument(
        "aten operator output is not a tensor, tensor list, or tensor tuple");
  }
}

class AtenOperator final : public Operator {
 public:
  std::string type() const override { return "aten"; }

  void compute(const std::vector<const Tensor*>& inputs, const std::vector<Tensor*>& outputs,
               const Attributes& attrs, ExecutionContext&) const override {
    const std::string& name = attrs.require<std::string>("name");
    const std::string overload = attrs.value_or<std::string>("overload", "");
    const auto order = attrs.value_or<std::vector<std::string>>("attr_order", {});

    c10::Stack stack;
    stack.reserve(inputs.size() + order.size());
    for (const Tensor* input : inputs) {
      if (input == nullptr) throw std::invalid_argument("aten operator received null input tensor");
      stack.emplace_back(input->torchTensor());
    }
    for (const std::string& key : order) {
      if (key == "name" || key == "overload" || key == "attr_order")
        throw std::invalid_argument("aten attr_order contains reserved attribute: " + key);
      auto it = attrs.values().find(key);
      if (it == attrs.values().end())
        throw std::invalid_argument("aten operator missing ordered attr: " + key);
      stack.push_back(toIValue(it->second));
    }

    auto op = c10::Dispatcher::singleton().findSchemaOrThrow(name.c_str(), overload.c_str());
    op.callBoxed(&stack);
    if (stack.empty()) throw std::runtime_error("aten operator produced no boxed return value");

    std::vector<at::Tensor> returned;
    flattenReturn(stack.back(), returned);
    if (returned.size() != outputs.size())
      throw std::invalid_argument("aten operator output count mismatch");
    for (std::size_t i = 0; i < returned.size(); ++i) {
      if (outputs[i] == nullptr) throw std::invalid_argument("aten operator received null output tensor");
      *outputs[i] = Tensor(std::move(returned[i]));
    }
  }
};

}  // namespace

void registerAtenOperator(OperatorRegistry& registry) {
  registry.registerFactory("aten", [] { return std::make_unique<AtenOperator>(); });
}

}  // namespace dli
