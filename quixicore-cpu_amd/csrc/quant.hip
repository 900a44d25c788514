// Dynamic per-row (per-group) int8 quantization of activations, the
// non-finite pre-scan, and q8_0/q4_0 weight pack/unpack on gfx950.
//
// quantize_int8 restates kernels/quantization/quantization_ref.cpp:143-168 of
// the reference bit for bit: scale = max|x| / 127 (IEEE division),
// inv = scale > 0 ? 1/scale : 0 (IEEE division), code =
// clamp(rint(x * inv), -127, 127) with round-half-even.  hipcc's default
// float division is correctly rounded and this file is compiled with
// -ffp-contract=off, so no step is fused or approximated.
#include "qc_device.h"
#include "qc_internal.h"

namespace qc {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int8_t quant_code(float v, float inv) {
  int q = static_cast<int>(rintf(v * inv));
  q = q < -127 ? -127 : (q > 127 ? 127 : q);
  return static_cast<int8_t>(q);
}

__device__ __forceinline__ uint32_t quant4(float4 v, float inv) {
  const uint32_t a = static_cast<uint8_t>(quant_code(v.x, inv));
  const uint32_t b = static_cast<uint8_t>(quant_code(v.y, inv));
  const uint32_t c = static_cast<uint8_t>(quant_code(v.z, inv));
  const uint32_t d = static_cast<uint8_t>(quant_code(v.w, inv));
  return a | (b << 8) | (c << 16) | (d << 24);
}

__device__ __forceinline__ bool finite4(float4 v) {
  return isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w);
}

__device__ __forceinline__ float abs_max4(float4 v, float m) {
  return fmaxf(fmaxf(fmaxf(m, fabsf(v.x)), fmaxf(fabsf(v.y), fabsf(v.z))), fabsf(v.w));
}

// Workgroup-wide (NT threads) max of a per-thread value and OR of a per-thread flag.
template <int NT>
__device__ __forceinline__ void block_max_or(float& m, int& bad) {
  __shared__ float smax[NT / 64];
  __shared__ int sbad[NT / 64];
  m = wave_max_nonneg(m);
  bad = __any(bad) ? 1 : 0;
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    smax[wave] = m;
    sbad[wave] = bad;
  }
  __syncthreads();
  m = smax[0];
  bad = sbad[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) {
    m = fmaxf(m, smax[w]);
    bad |= sbad[w];
  }
}

// One workgroup of NT threads per row, the row held in registers: V float4
// per thread.  Requires dim % 4 == 0, 4 <= dim <= 4 * NT * V, x 16-byte
// aligned and codes 4-byte aligned.
template <int V, int NT>
__global__ __launch_bounds__(NT) void quantize_rows_regs(const float* __restrict__ x,
                                                               int8_t* __restrict__ codes,
                                                               float* __restrict__ scales,
                                                               int dim, int* status) {
  const long long row = blockIdx.x;
  const float4* xr = reinterpret_cast<const float4*>(x + row * dim);
  uint32_t* cr = reinterpret_cast<uint32_t*>(codes + row * dim);
  const int n4 = dim >> 2;
  float4 v[V];
  float m = 0.f;
  int bad = 0;
  // Every lane issues all V loads (a lane past the row re-reads its last
  // float4 and ignores it), so they are in flight together: a load inside
  // `if (idx < n4)` was waited for before the next one was issued.  x is read
  // once and the codes written once: non-temporal loads and stores measured
  // 5.5% faster at M=2048 K=4096 (9.52-9.68 -> 8.97-9.04 us).
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * NT;
    const u32x4nt t = __builtin_nontemporal_load(reinterpret_cast<const u32x4nt*>(xr) +
                                                 (idx < n4 ? idx : n4 - 1));
    v[i] = make_float4(__uint_as_float(t.x), __uint_as_float(t.y), __uint_as_float(t.z), __uint_as_float(t.w));
  }
#pragma unroll
  for (int i = 0; i < V; ++i) {
    if (static_cast<int>(threadIdx.x) + i * NT < n4) {
      bad |= !finite4(v[i]);
      m = abs_max4(v[i], m);
    }
  }
  block_max_or<NT>(m, bad);
  if (bad && status != nullptr) {
    if (threadIdx.x == 0) *status = 3;
    return;
  }
  const float scale = m / 127.0f;
  const float inv = scale > 0.f ? 1.0f / scale : 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * NT;
    if (idx < n4) __builtin_nontemporal_store(quant4(v[i], inv), cr + idx);
  }
  if (threadIdx.x == 0) scales[row] = scale;
}

// Any dim / group size: one wavefront per group, two passes over the group.
__global__ __launch_bounds__(kThreads) void quantize_groups_generic(
    const float* __restrict__ x, int8_t* __restrict__ codes, float* __restrict__ scales,
    long long ngroups, long long group, int* status) {
  const long long g = static_cast<long long>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  if (g >= ngroups) return;
  const int lane = threadIdx.x & 63;
  const float* xg = x + g * group;
  float m = 0.f;
  int bad = 0;
  for (long long i = lane; i < group; i += 64) {
    const float v = xg[i];
    bad |= !isfinite(v);
    m = fmaxf(m, fabsf(v));
  }
  m = wave_max_nonneg(m);
  if (__any(bad)) {
    if (status != nullptr) {
      if (lane == 0) *status = 3;
      return;
    }
  }
  const float scale = m / 127.0f;
  const float inv = scale > 0.f ? 1.0f / scale : 0.f;
  for (long long i = lane; i < group; i += 64) codes[g * group + i] = quant_code(xg[i], inv);
  if (lane == 0) scales[g] = scale;
}

__global__ __launch_bounds__(kThreads) void nonfinite_scan(const float* __restrict__ x,
                                                           long long count, int* flag) {
  int bad = 0;
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  const long long n4 = (reinterpret_cast<uintptr_t>(x) % 16 == 0) ? count / 4 : 0;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride)
    bad |= !finite4(x4[i]);
  for (long long i = n4 * 4 + static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += stride)
    bad |= !isfinite(x[i]);
  if (__any(bad) && (threadIdx.x & 63) == 0) *flag = 1;
}

// ------------------------------------------------------- weight packing --

// f32 -> f16 bits, round to nearest even (v_cvt_f16_f32).  The empty asm keeps
// the compiler from fusing the conversion with the producing multiply into
// v_fma_mix*_f16 with a +0 addend, which turns a -0 scale (all-zero q4_0
// block, d = 0 / -8) into +0.
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  asm volatile("" : "+v"(f));
  const _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

// One thread per 32-element block.  q8_0: kernels/quantization/qgemv_ref.cpp:14-41;
// q4_0: kernels/quantization/qgemv_w8a8_ref.cpp:45-77 (lround = half away from zero).
template <int FMT>
__global__ __launch_bounds__(kThreads) void pack_blocks(const float* __restrict__ w,
                                                        uint8_t* __restrict__ out,
                                                        long long nblocks, int* status) {
  const long long b = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (b >= nblocks) return;
  const float* src = w + b * 32;
  float v[32];
  bool ok = true;
  float amax = 0.f, vmax = 0.f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    v[j] = src[j];
    ok = ok && isfinite(v[j]);
    if constexpr (FMT == kQ8_0) {
      amax = fmaxf(amax, fabsf(v[j]));
    } else if (fabsf(v[j]) > amax) {
      amax = fabsf(v[j]);
      vmax = v[j];
    }
  }
  if (!ok) {
    *status = 3;
    return;
  }
  if constexpr (FMT == kQ8_0) {
    uint8_t* blk = out + b * kQ8Bytes;
    const float d = amax / 127.0f;
    const float id = d != 0.f ? 1.0f / d : 0.f;
    const uint16_t dh = float_to_half_bits(d);
    blk[0] = dh & 0xFF;
    blk[1] = dh >> 8;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      float q = rintf(v[j] * id);
      q = q < -127.f ? -127.f : (q > 127.f ? 127.f : q);
      blk[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(q));
    }
  } else {
    uint8_t* blk = out + b * kQ4Bytes;
    const float d = vmax / -8.0f;
    const float id = d != 0.f ? 1.0f / d : 0.f;
    const uint16_t dh = float_to_half_bits(d);
    blk[0] = dh & 0xFF;
    blk[1] = dh >> 8;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      int lo = static_cast<int>(roundf(v[j] * id)) + 8;
      int hi = static_cast<int>(roundf(v[j + 16] * id)) + 8;
      lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
      hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
      blk[2 + j] = static_cast<uint8_t>(lo | (hi << 4));
    }
  }
}

template <int FMT>
__global__ __launch_bounds__(kThreads) void unpack_blocks(const uint8_t* __restrict__ in,
                                                          float* __restrict__ w,
                                                          long long nblocks) {
  const long long b = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (b >= nblocks) return;
  constexpr int BB = Fmt<FMT>::block_bytes;
  const uint8_t* blk = in + b * BB;
  const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
  float* dst = w + b * 32;
  if constexpr (FMT == kQ8_0) {
#pragma unroll
    for (int j = 0; j < 32; ++j) dst[j] = d * static_cast<float>(static_cast<int8_t>(blk[2 + j]));
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      dst[j] = static_cast<float>((blk[2 + j] & 15) - 8) * d;
      dst[j + 16] = static_cast<float>((blk[2 + j] >> 4) - 8) * d;
    }
  }
}

unsigned grid_for(long long items) {
  return static_cast<unsigned>((items + kThreads - 1) / kThreads);
}

}  // namespace

hipError_t launch_quantize_int8(const float* x, int8_t* codes, float* scales, long long rows,
                                long long dim, long long group, int* status, hipStream_t s) {
  const bool per_row = group == dim;
  const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(codes) % 4 == 0 && dim % 4 == 0;
  if (per_row && aligned && dim >= 4 && dim <= 32768 && rows <= 0x7FFFFFFFLL) {
    const unsigned grid = static_cast<unsigned>(rows);
    if (dim <= 1024)
      quantize_rows_regs<1, 256><<<grid, 256, 0, s>>>(x, codes, scales, (int)dim, status);
    else if (dim <= 2048)
      quantize_rows_regs<2, 256><<<grid, 256, 0, s>>>(x, codes, scales, (int)dim, status);
    else if (dim <= 4096)
      quantize_rows_regs<4, 256><<<grid, 256, 0, s>>>(x, codes, scales, (int)dim, status);
    else if (dim <= 8192)
      quantize_rows_regs<8, 256><<<grid, 256, 0, s>>>(x, codes, scales, (int)dim, status);
    else if (dim <= 16384)
      quantize_rows_regs<8, 512><<<grid, 512, 0, s>>>(x, codes, scales, (int)dim, status);
    else
      quantize_rows_regs<8, 1024><<<grid, 1024, 0, s>>>(x, codes, scales, (int)dim, status);
    return hipGetLastError();
  }
  const long long ngroups = rows * (dim / group);
  const long long grid = (ngroups + (kThreads / 64) - 1) / (kThreads / 64);
  quantize_groups_generic<<<static_cast<unsigned>(grid), kThreads, 0, s>>>(x, codes, scales,
                                                                           ngroups, group, status);
  return hipGetLastError();
}

hipError_t launch_nonfinite_scan(const float* x, long long count, int* flag, hipStream_t s) {
  long long blocks = (count / 4 + kThreads - 1) / kThreads;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  nonfinite_scan<<<static_cast<unsigned>(blocks), kThreads, 0, s>>>(x, count, flag);
  return hipGetLastError();
}

hipError_t launch_pack(int fmt, const float* w, void* packed, long long n, long long k,
                       int* status, hipStream_t s) {
  const long long nblocks = n * (k / 32);
  auto* out = static_cast<uint8_t*>(packed);
  if (fmt == kQ8_0)
    pack_blocks<kQ8_0><<<grid_for(nblocks), kThreads, 0, s>>>(w, out, nblocks, status);
  else
    pack_blocks<kQ4_0><<<grid_for(nblocks), kThreads, 0, s>>>(w, out, nblocks, status);
  return hipGetLastError();
}

hipError_t launch_unpack(int fmt, const void* packed, float* w, long long n, long long k,
                         hipStream_t s) {
  const long long nblocks = n * (k / 32);
  const auto* in = static_cast<const uint8_t*>(packed);
  if (fmt == kQ8_0)
    unpack_blocks<kQ8_0><<<grid_for(nblocks), kThreads, 0, s>>>(in, w, nblocks);
  else
    unpack_blocks<kQ4_0><<<grid_for(nblocks), kThreads, 0, s>>>(in, w, nblocks);
  return hipGetLastError();
}

// Streaming-read ceiling: reads `bytes` (a multiple of 16) with 16-byte loads,
// all sixteen of a 64 KB slab in flight per thread, the workgroups taking
// interleaved slabs; each thread stores the XOR of what it read (so nothing
// is optimised away).  A measurement seam: the GEMV's HBM efficiency is
// judged against it.  The loads carry the non-temporal hint, which measured
// 6-11% faster for this whole-line pattern on MI355X (256 MB: 47-48 ->
// 42.4 us).
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, long long n16,
                                                          uint32_t* __restrict__ out) {
  constexpr long long kSlab = 4096;                // 16-byte units per slab (64 KB)
  uint32_t x = 0;
  for (long long base = static_cast<long long>(blockIdx.x) * kSlab; base < n16;
       base += static_cast<long long>(gridDim.x) * kSlab) {
    uint4 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const long long i = base + threadIdx.x + 256LL * u;
      const u32x4nt t = i < n16 ? __builtin_nontemporal_load(reinterpret_cast<const u32x4nt*>(p) + i)
                                : u32x4nt{0, 0, 0, 0};
      v[u] = make_uint4(t.x, t.y, t.z, t.w);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  out[static_cast<long long>(blockIdx.x) * 256 + threadIdx.x] = x;
}

hipError_t launch_stream_read(const void* p, long long bytes, uint32_t* out, int grid,
                              hipStream_t s) {
  stream_read_kernel<<<grid, 256, 0, s>>>(static_cast<const uint4*>(p), bytes / 16, out);
  return hipGetLastError();
}

}  // namespace qc
