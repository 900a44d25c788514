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
// 16-byte vector for the non-temporal loads of the streaming kernels.
typedef uint32_t u32x4nt __attribute__((ext_vector_type(4)));

// The f32 dot of block h (0 / 1) of a pair (its bytes at `wp` in global
// memory) with the block's 32 values of x, summed in element order
// (kernels/quantization/qgemv_ref.cpp:70-76).
template <int FMT>
__device__ __forceinline__ float block_f32(const uint8_t* wp, int h, const float* xb) {
  float s = 0.0f;
#pragma unroll 1
  for (int j = 0; j < 32; ++j) {
    int q;
    if constexpr (FMT == kQ8_0) {
      q = static_cast<int8_t>(wp[(h == 0 ? 2 : 36) + j]);   // codes follow each fp16 scale
    } else {
      const uint8_t b = wp[(h == 0 ? 2 : 20) + (j & 15)];   // code j low, j + 16 high nibble
      q = static_cast<int>(j < 16 ? (b & 0xF) : (b >> 4)) - 8;
    }
    s += static_cast<float>(q) * xb[j];
  }
  return s;
}

// For an activation row x holding NaN or +-inf: the sum over blocks
// [b0, b1) of W row `wrow` of d_b * sum_j q_j x_j in f32, taken over the
// blocks whose 32 values of x hold NaN or +-inf only.  Each such block gives
// +-inf or NaN (the reference's class: +-inf by the signs of its products,
// NaN where a zero weight or scale meets an infinity, opposite infinities
// meet, or x holds NaN), and the finite blocks the reference adds to them do
// not change the result, so this is the reference's value of a K range in
// which x is not finite; ranges added together keep that class.  A rare
// path: callers reach it from one rolled loop after their main work.
template <int FMT>
__device__ __forceinline__ float nonfinite_blocks_f32(const uint8_t* wrow, const float* xr, int b0,
                                                   int b1) {
  constexpr int BB = Fmt<FMT>::block_bytes;
  float acc = 0.0f;
  for (int b = b0; b < b1; ++b) {
    const float* xb = xr + 32LL * b;
    bool special = false;
    for (int j = 0; j < 32; ++j) special = special || !(fabsf(xb[j]) <= 3.402823466e38f);
    if (!special) continue;
    const uint8_t* wp = wrow + static_cast<long long>(b >> 1) * (2 * BB);
    const uint16_t d = *reinterpret_cast<const uint16_t*>(wp + (b & 1) * BB);
    acc += half_bits_to_float(d) * block_f32<FMT>(wp, b & 1, xb);
  }
  return acc;
}

}  // namespace qc
