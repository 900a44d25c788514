// Drop-in of quantize_int8 (include/quixicore_cpu/quantization.h:40-42 of the
// reference): dynamic symmetric int8 over contiguous groups of each row;
// group_size 0 means one group per row; scales is [rows, dim/group_size].
// Synchronous; codes and scales are bit-identical to the reference.
#pragma once

#include <cstdint>

#include "quixicore_cpu/status.h"

namespace quixicore_cpu {

Status quantize_int8(const float* x, std::int8_t* codes, float* scales, long long rows,
                     long long dim, long long group_size = 0);

}  // namespace quixicore_cpu
