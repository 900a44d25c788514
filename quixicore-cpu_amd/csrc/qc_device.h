// Device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qc {

// Canonical GGUF block sizes (kernels/quantization/gguf_ref.cpp:509-510).
constexpr int kBlock = 32;
constexpr int kQ8Bytes = 34;
constexpr int kQ4Bytes = 18;
enum Format { kQ8_0 = 0, kQ4_0 = 1 };

template <int FMT>
struct Fmt;
template <>
struct Fmt<kQ8_0> {
  static constexpr int block_bytes = kQ8Bytes;
  static constexpr int pair_dwords = 17;  // two blocks = 68 B
};
template <>
struct Fmt<kQ4_0> {
  static constexpr int block_bytes = kQ4Bytes;
  static constexpr int pair_dwords = 9;  // two blocks = 36 B
};

// Exact binary16 -> binary32 (v_cvt_f32_f16; subnormals, inf and NaN kept).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
  const uint16_t h = static_cast<uint16_t>(bits16);
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Signed byte `b` of a dword as float (one SDWA-selected convert on gfx9).
template <int B>
__device__ __forceinline__ float sbyte(uint32_t w) {
  return static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(w >> (8 * B))));
}

// Unsigned byte `b` of a dword as float (v_cvt_f32_ubyteN).
template <int B>
__device__ __forceinline__ float ubyte(uint32_t w) {
  return static_cast<float>(static_cast<uint8_t>(w >> (8 * B)));
}

// Butterfly sum over the 64 lanes of a wavefront; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset >= 1; offset >>= 1) v += __shfl_xor(v, offset, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset >= 1; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
  return v;
}

// 4-byte-aligned 128-bit load (global_load_dwordx4 accepts dword alignment).
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

}  // namespace qc
