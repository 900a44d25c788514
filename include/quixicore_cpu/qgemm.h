// Drop-in of the hot-path entries of include/quixicore_cpu/qgemm.h of the
// reference.  Synchronous; host or device pointers (see qgemv.h).
#pragma once

#include <cstdint>

#include "quixicore_cpu/float_storage.h"
#include "quixicore_cpu/ops.h"
#include "quixicore_cpu/packed_weights.h"
#include "quixicore_cpu/qgemv.h"
#include "quixicore_cpu/quant_import.h"
#include "quixicore_cpu/workspace.h"

namespace quixicore_cpu {

// qgemm.h:19 -- Y[M,N] = X[M,K] @ dequantize(W[N,K])^T, f32.
Status qgemm(QuantFormat format, const void* packed_weights, const float* x, float* y,
             long long m, long long n, long long k);
// qgemm.h:26 -- prepared equivalent of qgemm, reading the device mirror.
Status qgemm_prepacked(const CpuPackedWeights& weights, const float* x, float* y, long long m,
                       Workspace* workspace = nullptr);
// qgemm.h:42 -- the M = 1 storage projection with f32 x and y (as in the
// reference, weights prepared from GGUF bytes return kUnsupportedFormat here;
// qgemm_prepacked takes them).
Status qgemv_prepacked(const CpuPackedWeights& weights, const float* x, float* y,
                       Workspace* workspace = nullptr);

// Prepared storage projections (qgemm.h:32-101).  Weights prepared from a
// CanonicalQuantTensor; GGUF-prepared weights return kUnsupportedFormat, as in
// the reference (kernels/quantization/qgemm_canonical.cpp:4275-4291).  This
// GPU route computes the int8 canonical layouts (kInt8Symmetric,
// kInt8Affine; row, channel or group scales); other canonical layouts return
// kUnsupportedFormat after the reference's validation.
Status qgemm_prepacked_storage(const CpuPackedWeights& weights, FloatStorageInput x,
                               FloatStorageOutput y, long long m,
                               Workspace* workspace = nullptr);
Status qgemm_prepacked_epilogue_storage(const CpuPackedWeights& weights, FloatStorageInput x,
                                        const float* bias, FloatStorageOutput y, long long m,
                                        LinearActivation activation,
                                        Workspace* workspace = nullptr);
Status qgemv_prepacked_storage(const CpuPackedWeights& weights, FloatStorageInput x,
                               FloatStorageOutput y, Workspace* workspace = nullptr);
Status qgemm_prepacked_gate_up_storage(const CpuPackedWeights& gate_weights,
                                       const CpuPackedWeights& up_weights, FloatStorageInput x,
                                       FloatStorageOutput gate_output,
                                       FloatStorageOutput up_output, long long m,
                                       Workspace* workspace = nullptr);
Status qgemv_prepacked_gate_up_storage(const CpuPackedWeights& gate_weights,
                                       const CpuPackedWeights& up_weights, FloatStorageInput x,
                                       FloatStorageOutput gate_output,
                                       FloatStorageOutput up_output,
                                       Workspace* workspace = nullptr);
Status qgemm_prepacked_qkv_storage(const CpuPackedWeights& q_weights,
                                   const CpuPackedWeights& k_weights,
                                   const CpuPackedWeights& v_weights, FloatStorageInput x,
                                   FloatStorageOutput q_output, FloatStorageOutput k_output,
                                   FloatStorageOutput v_output, long long m,
                                   Workspace* workspace = nullptr);
Status qgemv_prepacked_qkv_storage(const CpuPackedWeights& q_weights,
                                   const CpuPackedWeights& k_weights,
                                   const CpuPackedWeights& v_weights, FloatStorageInput x,
                                   FloatStorageOutput q_output, FloatStorageOutput k_output,
                                   FloatStorageOutput v_output, Workspace* workspace = nullptr);
// Q / K get split-half RoPE at `position` (cosine / sine [max_position]
// [head_dim / 2]); K and V go to slot `slot` of [slots][kv_heads][head_dim]
// caches (slot -1: Q only).
Status qgemv_prepacked_qkv_rope_kv_storage(
    const CpuPackedWeights& q_weights, const CpuPackedWeights& k_weights,
    const CpuPackedWeights& v_weights, FloatStorageInput x, const float* cosine,
    const float* sine, FloatStorageOutput q_output, FloatStorageOutput key_cache,
    FloatStorageOutput value_cache, long long query_heads, long long kv_heads,
    long long head_dim, long long slots, long long max_position, int position, int slot,
    Workspace* workspace = nullptr);
// output = SiLU(gate) * up; neither projection is stored.
Status qgemm_prepacked_swiglu_storage(const CpuPackedWeights& gate_weights,
                                      const CpuPackedWeights& up_weights, FloatStorageInput x,
                                      FloatStorageOutput output, long long m,
                                      Workspace* workspace = nullptr);
Status qgemv_prepacked_swiglu_storage(const CpuPackedWeights& gate_weights,
                                      const CpuPackedWeights& up_weights, FloatStorageInput x,
                                      FloatStorageOutput output, Workspace* workspace = nullptr);

// qgemm.h:118-127 -- canonical activations (e.g. from quantize_canonical)
// projected against canonical prepared weights: activation [M, K] codes,
// f32 y [M, N] (host or device memory).  Computed on the GPU for int8
// weights x int8 activations (kInt8Symmetric / kInt8Affine, row or group
// scales); other pairs return kUnsupportedFormat after the reference's
// validation.  qgemv_prepacked_quantized requires M = 1.
Status qgemm_prepacked_quantized(const CpuPackedWeights& weights,
                                 const CanonicalQuantTensor& activation, float* y,
                                 Workspace* workspace = nullptr);
Status qgemv_prepacked_quantized(const CpuPackedWeights& weights,
                                 const CanonicalQuantTensor& activation, float* y,
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
