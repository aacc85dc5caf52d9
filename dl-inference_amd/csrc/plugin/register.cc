// Plugin entry point: the C symbol OperatorRegistry::loadLibrary resolves
// (reference: the generated dli_register_operators, tools/build_triton_aot_ops.py:404-407;
// typedef RegisterOperatorsFn, include/dli/operator.h:41).
#include "common.h"

extern "C" __attribute__((visibility("default"))) bool dli_register_operators(
    dli::OperatorRegistry* registry) {
  if (registry == nullptr) return false;
  try {
    dli::plugin::registerReferenceOps(registry);
    dli::plugin::registerFusedOps(registry);
    return true;
  } catch (...) {
    return false;
  }
}
