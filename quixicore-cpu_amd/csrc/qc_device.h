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

// Cross-lane moves with DPP (no LDS traffic).  Control words of the gfx9 DPP
// encoding: row_shr:n = 0x110 + n, row_bcast:15 = 0x142, row_bcast:31 = 0x143,
// quad_perm [1,0,3,2] = 0xB1.  Lanes whose source is out of range, or that
// the row/bank masks leave out, receive `old` (0 here).
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF, bool BOUND_ZERO = true>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK,
                                                    BANK_MASK, BOUND_ZERO));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}

// Value of the neighbouring lane l ^ 1.
__device__ __forceinline__ float xor1_f32(float v) { return dpp_f32<0xB1>(v); }
__device__ __forceinline__ int xor1_i32(int v) { return dpp_i32<0xB1>(v); }

// Reductions over each aligned group of 8 lanes, returned to all 8 (quad
// perms [1,0,3,2] = 0xB1 and [2,3,0,1] = 0x4E, then row_half_mirror = 0x141,
// which pairs lane i of a group with lane 7 - i, in the other quad).
__device__ __forceinline__ float group8_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  return fmaxf(v, dpp_f32<0x141>(v));
}
__device__ __forceinline__ int group8_sum(int v) {
  v += dpp_i32<0xB1>(v);
  v += dpp_i32<0x4E>(v);
  return v + dpp_i32<0x141>(v);
}
__device__ __forceinline__ int group8_and(int v) {
  v &= dpp_i32<0xB1>(v);
  v &= dpp_i32<0x4E>(v);
  return v & dpp_i32<0x141>(v);
}

// Sum over the 64 lanes of a wavefront, valid in lane 63 only (the AMD DPP
// reduction: partial sums within each 16-lane row, then row broadcasts).
// Summation order is fixed, so results are deterministic.
__device__ __forceinline__ float wave_sum_lane63(float v) {
  float t = v + dpp_f32<0x111>(v);       // + v[l-1]
  t = t + dpp_f32<0x112>(v);             // + v[l-2]
  t = t + dpp_f32<0x113>(v);             // + v[l-3]: sum of 4 lanes
  t = t + dpp_f32<0x114, 0xF, 0xE, false>(t);   // lanes 4..15 of each row: sum of 8
  t = t + dpp_f32<0x118, 0xF, 0xC, false>(t);   // lanes 8..15: lane 15 = row sum
  t = t + dpp_f32<0x142, 0xA, 0xF, false>(t);   // rows 1, 3 += lane 15 of rows 0, 2
  t = t + dpp_f32<0x143, 0xC, 0xF, false>(t);   // rows 2, 3 += lane 31: lane 63 = total
  return t;
}

// Sum over the wavefront, returned to every lane.
__device__ __forceinline__ float wave_sum(float v) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_lane63(v)), 63));
}

// Max over the wavefront of non-negative values (disabled DPP lanes read 0),
// returned to every lane.
__device__ __forceinline__ float wave_max_nonneg(float v) {
  float t = fmaxf(v, dpp_f32<0x111>(v));
  t = fmaxf(t, dpp_f32<0x112>(v));
  t = fmaxf(t, dpp_f32<0x113>(v));
  t = fmaxf(t, dpp_f32<0x114, 0xF, 0xE, false>(t));
  t = fmaxf(t, dpp_f32<0x118, 0xF, 0xC, false>(t));
  t = fmaxf(t, dpp_f32<0x142, 0xA, 0xF, false>(t));
  t = fmaxf(t, dpp_f32<0x143, 0xC, 0xF, false>(t));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 63));
}

// 4-byte-aligned 128-bit load (global_load_dwordx4 accepts dword alignment).
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

}  // namespace qc
