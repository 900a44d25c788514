// Drop-in of the qgemv family (include/quixicore_cpu/qgemv.h of the
// reference), for q8_0 and q4_0 on gfx950.  Same names, argument order and
// Status semantics; every call is synchronous (outputs are ready on return).
// Pointers may be host or device memory: device pointers are used in place,
// host buffers are staged through device memory.
#pragma once

#include <cstddef>
#include <cstdint>

#include "quixicore_cpu/status.h"

namespace quixicore_cpu {

// Numbering kept from include/quixicore_cpu/qgemv.h:10-47 of the reference so
// stored format ids stay valid; only kQ8_0 and kQ4_0 have kernels here.
enum class QuantFormat {
  kQ8_0,  // GGUF q8_0: 32-element blocks, fp16 scale + 32 int8 values
  kQ4_0,  // GGUF q4_0: 32-element blocks, fp16 scale + 16 packed nibbles (-8 offset)
  kQ4_1,
  kQ5_0,
  kQ5_1,
  kU4B8,
  kU4,
  kHQQ,
  kFP8E4M3,
  kFP8E5M2,
  kFP8Block,
  kFP8Raw,
  kFP4E2M1,
  kMXFP8,
  kNVFP4,
  kMXFP4,
  kMXFP6E3M2,
  kMXFP6E2M3,
  kBitnet,
  kQ2_K,
  kQ3_K,
  kQ4_K,
  kQ5_K,
  kQ6_K,
  kIQ4_NL,
  kIQ4_XS,
  kIQ2_XXS,
  kIQ2_XS,
  kIQ3_XXS,
  kIQ1_S,
  kTQ2_0,
  kQ1_0,
  kQ2_0,
  kIQ3_S,
  kIQ2_S,
  kIQ1_M,
  kTQ1_0,
};

// include/quixicore_cpu/qgemv.h:70
Status qgemv_packed_size(QuantFormat format, long long n, long long k, size_t* size);
// include/quixicore_cpu/qgemv.h:77 (bit-identical blocks, packed on the GPU)
Status qgemv_pack(QuantFormat format, const float* weights, long long n, long long k,
                  void* packed);
// include/quixicore_cpu/qgemv.h:89
Status qgemv_unpack(QuantFormat format, const void* packed, long long n, long long k,
                    float* weights);
// include/quixicore_cpu/qgemv.h:108: y = dequantize(wq) @ x, f32 accumulation.
Status qgemv(QuantFormat format, const void* packed, const float* x, float* y, long long n,
             long long k);
// include/quixicore_cpu/qgemv.h:166
const char* qgemv_variant(QuantFormat format);

// Fused decode projections over one x (include/quixicore_cpu/qgemv.h:143-163
// of the reference), one GPU launch: up/gate [n][k] each; the activation form
// stores out = activation(gate) * up (GELU-tanh or SiLU) without storing either
// projection; Q [query_dim][input_dim], K and V [kv_dim][input_dim].  q8_0 and
// q4_0 only (other formats return kUnsupportedFormat).
Status qgemv_up_gate(QuantFormat format, const void* packed_up, const void* packed_gate,
                     const float* x, float* up, float* gate, long long n, long long k);
Status qgemv_up_gate_activation(QuantFormat format, const void* packed_up,
                                const void* packed_gate, const float* x, float* out,
                                long long n, long long k, bool gelu_tanh = true);
Status qgemv_qkv(QuantFormat format, const void* packed_q, const void* packed_k,
                 const void* packed_v, const float* x, float* q, float* k_out, float* v_out,
                 long long query_dim, long long kv_dim, long long input_dim);
// include/quixicore_cpu/qgemv.h:157-163: one decode token's Q/K/V with
// split-half RoPE on Q and K at `position` (cosine / sine are
// [max_position][head_dim / 2]) and K/V stored into slot `slot` of the
// [slots][kv_heads][head_dim] caches (slot -1: Q only).
Status qgemv_qkv_rope_kv(QuantFormat format, const void* packed_q, const void* packed_k,
                         const void* packed_v, const float* x, const float* cosine,
                         const float* sine, float* q, float* key_cache, float* value_cache,
                         long long query_heads, long long kv_heads, long long head_dim,
                         long long input_dim, long long slots, long long max_position,
                         int position, int slot);

}  // namespace quixicore_cpu
