#pragma once

// Size of the static device scratch of dli_hip_lm_head_argmax_norm_noalloc, shared by the
// kernel module that defines the array (decode.hip) and the host entry point that checks call
// sizes against it (csrc/hip/decode_ops.cc).
#include <stddef.h>

namespace dli_scratch {

// lm_head argmax partials: (fp32 value, int32 index) per row and lm_head workgroup, laid out
// within the room of one per row and 32-row vocab tile (there are never more workgroups than
// tiles), i.e. 8 * m * ceil(vocab / 32) bytes. 4 MiB holds m = 64 rows at vocab 262,144 (Qwen2's
// 151,936-row vocabulary at 64 rows needs 2.3 MiB).
constexpr size_t kLmHeadBytes = size_t{4} << 20;

}  // namespace dli_scratch
