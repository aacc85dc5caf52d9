#pragma once

// dli.weights.v1 loader (manifest JSON + one binary blob), as include/dli/weights.h:10-11 of
// the reference, with "bfloat16", "float16" and "int32" accepted as dtypes.

#include <string>

#include "dli/engine.h"
#include "dli/tensor.h"

namespace dli {

TensorMap loadWeights(const std::string& manifest_path, DeviceType device = DeviceType::Cpu,
                      int device_id = 0);

}  // namespace dli
