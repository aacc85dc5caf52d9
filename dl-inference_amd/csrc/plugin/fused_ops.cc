// Fused decode operators (registered next to the reference operators).
#include "common.h"

namespace dli::plugin {

void registerFusedOps(OperatorRegistry*) {}

}  // namespace dli::plugin
