#pragma once

// The built-in "aten" operator: calls any ATen schema through the c10 dispatcher
// (src/aten_operator.cc:61-113 of the reference).

#include "dli/operator.h"

namespace dli {

void registerAtenOperator(OperatorRegistry& registry);

}  // namespace dli
