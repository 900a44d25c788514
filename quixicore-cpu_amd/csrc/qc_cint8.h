// Shared by the canonical int8 projection kernels: canonical_int8.hip (the
// digit-dot, f32 multiply-add and generic kernels, and the routing) and
// canonical_planes.hip (the row-plane route on the int8 MFMA GEMM).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "qc_internal.h"

namespace qc {

// The launch's row space: segments of logical rows over up to three
// matrices.  mode 0: plain rows (segment s, row r -> y[s][m * ld + r]), with
// bias and activation on segment 0 when given.  mode 1: one segment whose
// logical rows 2i / 2i + 1 are gate / up row i (w[0] / w[1]); out[m * ld + i]
// = SiLU(gate) * up.  mode 2 (m = 1): segments below nrope hold RoPE pairs:
// logical rows 2j / 2j + 1 are rows d / d + half of head j / half.
struct CSegs {
  const int8_t* w[3];
  const float* scale[3];
  const float* zero[3];
  void* y[3];
  long long ld[3];     // elements between activation rows of y[s]
  int ytype[3];
  int start[4];        // start[nseg] = logical rows
  int nseg;
  int mode;
  int groups;          // scale groups per row (1: one scale per row)
  int gshift;          // log2(group size) when groups > 1 (power of two >= 16), else 0
  int gsize;
  const float* bias;
  int act;
  int half, nrope;
  const float* rc;
  const float* rs;
};

// Row-plane route limits (canonical_planes.hip): K, and the fewest
// activation rows it takes (N = 14336, K = 4096 at M = 2: row scales 22.9 us
// on the digit-dot kernel, 18.8 there; groups of 128 22.0 on the digit-dot
// kernel, 26.5 there; M = 3 with groups of 128 or 64: 34 against 26 / 34;
// groups of 32 at M = 4: 40 against 44.5, at M = 5-8: 62-79 against 46).
constexpr int kPlanesMaxK = 16384;
constexpr int kPlanesMinM = 2;
constexpr int kPlanesMinMGrouped = 3;
constexpr int kPlanesMinMGroups32 = 5;

// The projections of L over the row-plane route (all checks done by the
// caller: 16-byte aligned codes, K % 32 == 0, K <= kPlanesMaxK, not the RoPE
// mode; grouped: K % 128 == 0 and group sizes of 32, 64 or a multiple of 128
// columns).
hipError_t launch_cint8_planes(const CSegs& sg, const CInt8Launch& L, int m, int k, bool grouped,
                               hipStream_t s);

// The call's scratch: buffer 0 of its stream's cache entry, whose call lock
// `hold` keeps until the caller's last launch.
hipError_t call_scratch(hipStream_t s, size_t bytes, std::unique_lock<std::mutex>& hold,
                        void** out);

namespace {   // device helpers: one copy per file

__device__ __forceinline__ float load_x(const void* x, long long i, int type) {
  if (type == QC_STORAGE_F32) return static_cast<const float*>(x)[i];
  const uint16_t b = static_cast<const uint16_t*>(x)[i];
  if (type == QC_STORAGE_F16) return static_cast<float>(__builtin_bit_cast(_Float16, b));
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// float_to_bf16 of kernels/utils/float_storage_ref.cpp:184-193 (round to
// nearest even; NaNs stay NaN) and IEEE binary16 round to nearest even.
__device__ __forceinline__ void store_y(void* y, long long i, int type, float v) {
  if (type == QC_STORAGE_F32) {
    static_cast<float*>(y)[i] = v;
  } else if (type == QC_STORAGE_F16) {
    asm volatile("" : "+v"(v));   // keep the conversion a plain v_cvt_f16_f32
    static_cast<uint16_t*>(y)[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  } else {
    const uint32_t bits = __float_as_uint(v);
    uint16_t out;
    if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x007fffffu) != 0)
      out = static_cast<uint16_t>((bits >> 16) | 0x0040u);
    else
      out = static_cast<uint16_t>((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
    static_cast<uint16_t*>(y)[i] = out;
  }
}

// projection_activation of kernels/quantization/qgemm_canonical.cpp:361-379
// (LinearActivation: 0 none, 1 GELU-erf, 2 GELU-tanh, 3 SiLU, 4 ReLU^2).
__device__ __forceinline__ float linear_activation(float v, int act) {
  constexpr float kInvSqrt2 = 0.7071067811865475f;
  constexpr float kSqrt2OverPi = 0.7978845608028654f;
  switch (act) {
    case 1: return 0.5f * v * (1.0f + erff(v * kInvSqrt2));
    case 2: return 0.5f * v * (1.0f + tanhf(kSqrt2OverPi * (v + 0.044715f * v * v * v)));
    case 3: return v / (1.0f + expf(-v));
    case 4: return v > 0.0f ? v * v : 0.0f;
    default: return v;
  }
}

// sum_j (code_j - z) * x_j in f32, element order, over the 32 codes at
// `codes` and x[xi ..]: the rare form for a block of x that holds NaN or
// +-inf, whose per-element products give the reference's inf / NaN classes
// (the split into sum q x - z sum x could turn +-inf into NaN).
__device__ __noinline__ float cint8_block_f32(const int8_t* codes, const void* x, long long xi,
                                              int xtype, float z) {
  float s = 0.0f;
#pragma unroll 1
  for (int j = 0; j < 32; ++j) s += (static_cast<float>(codes[j]) - z) * load_x(x, xi + j, xtype);
  return s;
}

}  // namespace
}  // namespace qc
