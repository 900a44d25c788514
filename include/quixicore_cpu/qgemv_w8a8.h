// Drop-in of the activation-quantizing GEMV (include/quixicore_cpu/qgemv_w8a8.h
// of the reference) on gfx950.  Same names, argument order and Status
// semantics; every call is synchronous.  Pointers may be host or device
// memory (host buffers are staged through device memory).
//
// y = dequant(W) @ dequant(blockwise_int8(x)): x is quantized per 32-element
// block to int8 (scale = max|x_b| / 127), each block dot is exact, and each
// row is summed in block order -- outputs are bit-identical to the
// reference's.
#pragma once

#include "quixicore_cpu/qgemv.h"

namespace quixicore_cpu {

Status qgemv_w8a8(QuantFormat format, const void* packed_weights, const float* x, float* y,
                  long long n, long long k);

// Packed size / pack for the w8a8 weight formats (the q8_0 / q4_0 layouts of
// qgemv).  k must be a multiple of 32.
Status qgemv_w8a8_packed_size(QuantFormat format, long long n, long long k, long long* bytes);
Status qgemv_w8a8_pack(QuantFormat format, const float* weights, long long n, long long k,
                       void* packed);

// Name of the route taken for a weight format.
const char* qgemv_w8a8_variant(QuantFormat format);

}  // namespace quixicore_cpu
