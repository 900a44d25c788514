// Drop-in of the hot-path entries of include/quixicore_cpu/qgemm.h of the
// reference.  Synchronous; host or device pointers (see qgemv.h).
#pragma once

#include <cstdint>

#include "quixicore_cpu/packed_weights.h"
#include "quixicore_cpu/qgemv.h"
#include "quixicore_cpu/workspace.h"

namespace quixicore_cpu {

// qgemm.h:19 -- Y[M,N] = X[M,K] @ dequantize(W[N,K])^T, f32.
Status qgemm(QuantFormat format, const void* packed_weights, const float* x, float* y,
             long long m, long long n, long long k);
// qgemm.h:26 -- prepared equivalent of qgemm, reading the device mirror.
Status qgemm_prepacked(const CpuPackedWeights& weights, const float* x, float* y, long long m,
                       Workspace* workspace = nullptr);
// qgemm.h:42
Status qgemv_prepacked(const CpuPackedWeights& weights, const float* x, float* y,
                       Workspace* workspace = nullptr);

// qgemm.h:235 -- prequantized integer GEMM, X token-major [M,K], W [N,K].
Status int8_gemm(const std::int8_t* weights, const std::int8_t* x, const float* weight_scale,
                 const float* activation_scale, const std::int32_t* weight_row_sum,
                 const int* activation_zero_point, float* y, long long m, long long n,
                 long long k, bool asymmetric = false);
// qgemm.h:240
const char* int8_gemm_variant();
// qgemm.h:250
Status qgemm_w8a8(const std::int8_t* weights, const std::int8_t* x, const float* weight_scale,
                  const float* activation_scale, float* y, long long m, long long n,
                  long long k);
// qgemm.h:253-257
Status qgemm_w8a8_azp(const std::int8_t* weights, const std::int8_t* x,
                      const float* weight_scale, const float* activation_scale,
                      const std::int32_t* weight_row_sum, const int* activation_zero_point,
                      float* y, long long m, long long n, long long k);

}  // namespace quixicore_cpu
