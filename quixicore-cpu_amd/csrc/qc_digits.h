// Exact-digit encoding of f32 activations for int8 dot products, shared by
// the q8_0 / q4_0 GEMV kernels and the canonical int8 projections.
//
// For every 32-element block b of x: the power of two 2^e_b with max|x_b| <
// 2^(e_b + 21) (e_b = frexp exponent - 21) and the integers q_j = rint(x_j *
// 2^-e_b), clamped to [-2^21, 2^21 - 1], split into three int8 digits (floor
// division): q_j = 2^14 d0_j + 2^7 d1_j + d2_j, d0 in [-128, 127], d1, d2 in
// [0, 127].  A block dot with int8 codes c is then three exact int32 sums
// S_t = sum_j c_j d_t,j (v_dot4_i32_i8) combined as 2^e_b (2^14 S0 + 2^7 S1 +
// S2); x_j is held to within max|x_b| 2^-21.  A block holding NaN or +-inf is
// given zero digits and gate NaN.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qc_device.h"
#include "qc_internal.h"

namespace qc {

constexpr int kRec = 208;  // LDS bytes per pair: 3 digit planes x 64 + 16 pad

__device__ __forceinline__ int first_pair(int pbeg, int lane) {
  return pbeg + ((lane - pbeg) & 63);
}

// Barrier that orders LDS traffic only: global loads already issued stay in
// flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders one wavefront's LDS accesses across lanes (stores of some lanes
// before loads of them by others, or loads before later stores): a fence at
// wavefront scope plus a wave barrier.  The hardware already runs a wave's
// LDS operations in order, so this emits no instruction; it keeps the
// compiler from reordering the accesses.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// LDS layout of one chunk of kc elements (kc a multiple of 64):
//   [kc/64 pair records of kRec bytes][kc/32 int32 exponents e_b]
//   [kc/32 f32 gates: 1, or NaN for a non-finite block][3 x kc/32 int32 digit sums]
__host__ __device__ constexpr size_t exp_off(int kc) { return static_cast<size_t>(kc / 64) * kRec; }
__host__ __device__ constexpr size_t gate_off(int kc) { return exp_off(kc) + 4 * static_cast<size_t>(kc / 32); }
__host__ __device__ constexpr size_t dsum_off(int kc) { return gate_off(kc) + 4 * static_cast<size_t>(kc / 32); }
__host__ __device__ constexpr size_t lds_size(int kc) { return dsum_off(kc) + 12 * static_cast<size_t>(kc / 32); }

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | (static_cast<uint32_t>(d) << 24);
}

// Digits of half-block h (16 values v) of one row of x into that row's LDS
// chunk; the two halves of a block sit in lanes t and t^1 (both call this
// together: the block maximum is exchanged between them).
template <bool WITH_SUMS>
__device__ __forceinline__ void build_half(uint8_t* lds, const float* v, int h, int kc) {
  float m = 0.f;
  bool finite = true;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    m = fmaxf(m, fabsf(v[i]));
    finite = finite && isfinite(v[i]);
  }
  m = fmaxf(m, xor1_f32(m));
  finite = finite && (xor1_i32(finite ? 1 : 0) != 0);
  int ex = 0;
  (void)frexpf(m, &ex);                            // m < 2^ex
  const int e = finite ? ex - 21 : 0;
  int d0[16], d1[16], d2[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    int q = finite ? __float2int_rn(ldexpf(v[i], -e)) : 0;   // |x * 2^-e| <= 2^21
    q = q > 2097151 ? 2097151 : q;
    d0[i] = q >> 14;                               // [-128, 127]
    d1[i] = (q >> 7) & 127;                        // [0, 127]
    d2[i] = q & 127;                               // [0, 127]
  }
  const int pair = h >> 2;
  uint8_t* rec = lds + pair * kRec + (h & 3) * 16;
  uint4 p0, p1, p2;
  p0.x = pack4(d0[0], d0[1], d0[2], d0[3]);    p0.y = pack4(d0[4], d0[5], d0[6], d0[7]);
  p0.z = pack4(d0[8], d0[9], d0[10], d0[11]);  p0.w = pack4(d0[12], d0[13], d0[14], d0[15]);
  p1.x = pack4(d1[0], d1[1], d1[2], d1[3]);    p1.y = pack4(d1[4], d1[5], d1[6], d1[7]);
  p1.z = pack4(d1[8], d1[9], d1[10], d1[11]);  p1.w = pack4(d1[12], d1[13], d1[14], d1[15]);
  p2.x = pack4(d2[0], d2[1], d2[2], d2[3]);    p2.y = pack4(d2[4], d2[5], d2[6], d2[7]);
  p2.z = pack4(d2[8], d2[9], d2[10], d2[11]);  p2.w = pack4(d2[12], d2[13], d2[14], d2[15]);
  *reinterpret_cast<uint4*>(rec) = p0;
  *reinterpret_cast<uint4*>(rec + 64) = p1;
  *reinterpret_cast<uint4*>(rec + 128) = p2;
  const int blk = h >> 1;
  if constexpr (WITH_SUMS) {
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s0 += d0[i];
      s1 += d1[i];
      s2 += d2[i];
    }
    s0 += xor1_i32(s0);
    s1 += xor1_i32(s1);
    s2 += xor1_i32(s2);
    if ((h & 1) == 0) {
      int* sums = reinterpret_cast<int*>(lds + dsum_off(kc));
      sums[blk] = s0;
      sums[(kc >> 5) + blk] = s1;
      sums[2 * (kc >> 5) + blk] = s2;
    }
  }
  if ((h & 1) == 0) {
    reinterpret_cast<int*>(lds + exp_off(kc))[blk] = e;
    reinterpret_cast<float*>(lds + gate_off(kc))[blk] = finite ? 1.0f : __builtin_nanf("");
  }
}

// The digits of one pair as seen by its owning lane.
struct PairDigits {
  uint32_t d[3][16];  // plane t, dword i = elements 4i..4i+3 of the pair
  int e[2];           // block exponents e_b
  float gate[2];      // 1, or NaN for a block of x holding a non-finite value
  int off[2][3];      // q4_0: -8 * sum of plane t over block b
};

template <int FMT>
__device__ __forceinline__ void read_digits(PairDigits& g, const uint8_t* lds, int pl, int kc) {
  const uint8_t* rec = lds + pl * kRec;
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(rec + 64 * t + 16 * i);
      g.d[t][4 * i] = v.x; g.d[t][4 * i + 1] = v.y; g.d[t][4 * i + 2] = v.z; g.d[t][4 * i + 3] = v.w;
    }
  const int2 ev = *reinterpret_cast<const int2*>(lds + exp_off(kc) + 8 * pl);
  const float2 gv = *reinterpret_cast<const float2*>(lds + gate_off(kc) + 8 * pl);
  g.e[0] = ev.x;
  g.e[1] = ev.y;
  g.gate[0] = gv.x;
  g.gate[1] = gv.y;
  if constexpr (FMT == kQ4_0) {
    const int* sums = reinterpret_cast<const int*>(lds + dsum_off(kc));
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      const int2 v = *reinterpret_cast<const int2*>(sums + t * (kc >> 5) + 2 * pl);
      g.off[0][t] = -8 * v.x;
      g.off[1][t] = -8 * v.y;
    }
  }
}

__device__ __forceinline__ float combine(int s0, int s1, int s2) {
  return fmaf(static_cast<float>(s0), 16384.f, fmaf(static_cast<float>(s1), 128.f, static_cast<float>(s2)));
}

// An integral zero point z with |z| <= 2^16, as an int (false otherwise: NaN,
// fractional or larger zero points keep the f32 form f - z * xs).
__device__ __forceinline__ bool integral_zero(float z, int& zi) {
  zi = __float2int_rn(z);   // saturates; NaN gives 0, which then differs from z
  return static_cast<float>(zi) == z && zi >= -65536 && zi <= 65536;
}

// The affine block dot sum_j (c_j - z) x_j for an integral zero point, from
// the code-digit sums sd[t] = sum_j c_j d_t,j and the digit-plane sums
// ds[t] = sum_j d_t,j: each plane's sum_j (c_j - z) d_t,j = sd[t] - z ds[t] is
// an exact int32 (|sd| <= 2^19, |z ds| <= 2^28), so a row or group whose codes
// all equal z gives exactly 0, as the reference's per-element decode
// scale * (code - zero) does.
__device__ __forceinline__ float affine_block(const int (&sd)[3], const int (&ds)[3], int zi, int e) {
  return ldexpf(combine(sd[0] - zi * ds[0], sd[1] - zi * ds[1], sd[2] - zi * ds[2]), e);
}

// The digit-plane sums of pair pl's two blocks: s[b][t] = sum_j d_t,j.
__device__ __forceinline__ void read_digit_sums(int (&s)[2][3], const uint8_t* lds, int pl, int kc) {
  const int* sums = reinterpret_cast<const int*>(lds + dsum_off(kc));
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const int2 v = *reinterpret_cast<const int2*>(sums + t * (kc >> 5) + 2 * pl);
    s[0][t] = v.x;
    s[1][t] = v.y;
  }
}

}  // namespace qc
