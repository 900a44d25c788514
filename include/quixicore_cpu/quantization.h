// Drop-in of the reference's activation quantizers on the W8A8 path
// (include/quixicore_cpu/quantization.h): quantize_int8 (40-42) is dynamic
// symmetric int8 over contiguous groups of each row; group_size 0 means one
// group per row; scales is [rows, dim/group_size].  Synchronous; codes and
// scales are bit-identical to the reference.
#pragma once

#include <cstdint>

#include "quixicore_cpu/status.h"

namespace quixicore_cpu {

Status quantize_int8(const float* x, std::int8_t* codes, float* scales, long long rows,
                     long long dim, long long group_size = 0);

// Per-row asymmetric int8 (reference quantization.h:49-54): reconstruct with
// scale[row] * (code - zero_point[row]).  Bit-identical to the reference.
Status quantize_int8_asymmetric(const float* x, std::int8_t* codes, float* scales,
                                int* zero_points, long long rows, long long dim);
Status dequantize_int8_asymmetric(const std::int8_t* codes, const float* scales,
                                  const int* zero_points, float* out, long long rows,
                                  long long dim);

// Residual add + RMSNorm + dynamic int8 quantization (reference
// quantization.h:110-116): residual_out = x + residual, codes / scales of
// RMSNorm(residual_out) * weight per group (group_size 0: per row).  A group
// whose normalized values are not finite keeps its scale and codes unwritten
// and the call returns kInvalidArgument after writing everything else.
// Bit-identical to the reference.
Status rms_norm_add_quant_int8(const float* x, const float* residual, const float* weight,
                               std::int8_t* codes, float* residual_out, float* scales,
                               long long rows, long long hidden, float eps = 1e-5f,
                               long long group_size = 0);

}  // namespace quixicore_cpu
