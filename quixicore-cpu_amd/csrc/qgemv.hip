// q8_0 / q4_0 block-dequant GEMV (decode, M=1) and small-batch GEMM (M>1)
// over the canonical GGUF bytes, for gfx950.
//
// Semantics: y[m][n] = sum_k dequant(W)[n][k] * x[m][k] with f32 activations
// and f32 accumulation (include/quixicore_cpu/qgemv.h:100-108 of the
// reference; qgemm is one qgemv per activation row, kernels/quantization/
// qgemm_ref.cpp:156-162).  Deterministic: every output is reduced in a fixed
// order that does not depend on timing.
//
// Layout in HBM: W is row-major [N][K/32] canonical blocks (34 B q8_0, 18 B
// q4_0).  Two consecutive blocks form a "pair" of 68 B / 36 B -- a whole
// number of dwords -- so when K/32 is even every row and every pair starts on
// a 4-byte boundary and a lane can fetch its pair with dword-aligned 128-bit
// loads.  Lane l of a wavefront owns pairs l, l+64, ... of a row: one
// load instruction of the wave covers a contiguous span of the row.
//
// M = 1 goes to the exact-int8-dot kernel of qgemv_dot.hip.  For M > 1, x is
// staged per workgroup into LDS (padded by 16 B every 64 floats so the per-
// lane 256-B slices of consecutive lanes fall into different banks) and every
// decoded weight is reused for up to 8 activation rows.
#include "qc_device.h"
#include "qc_internal.h"

namespace qc {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsBudget = 64 * 1024;

__device__ __forceinline__ int xpad(int j) { return j + ((j >> 6) << 2); }

// Lane l always owns the pairs p with p % 64 == l, whatever the K chunking,
// so every row is summed in the same order by the M = 1 and M > 1 kernels
// (qgemm row m is bit-identical to qgemv of x[m], as in the reference).
__device__ __forceinline__ int first_pair(int pbeg, int lane) {
  return pbeg + ((lane - pbeg) & 63);
}

// Stage x[c0 : c0+clen] (clen a multiple of 64) of `mt` activation rows into
// LDS; for q4_0 also the per-block sums used to fold the -8 nibble offset.
template <int FMT>
__device__ __forceinline__ void stage_x(float* xs, const float* __restrict__ x, long long ldx,
                                        int mt, int c0, int clen, int kc, bool vec_ok) {
  const int row_stride = xpad(kc);
  for (int mi = 0; mi < mt; ++mi) {
    const float* src = x + mi * ldx + c0;
    float* dst = xs + mi * row_stride;
    if (vec_ok) {
      for (int i = threadIdx.x * 4; i < clen; i += kThreads * 4)
        *reinterpret_cast<float4*>(dst + xpad(i)) = *reinterpret_cast<const float4*>(src + i);
    } else {
      for (int i = threadIdx.x; i < clen; i += kThreads) dst[xpad(i)] = src[i];
    }
  }
  if constexpr (FMT == kQ4_0) {
    __syncthreads();
    float* sums = xs + mt * row_stride;
    const int nblk = clen >> 5;
    for (int t = threadIdx.x; t < mt * nblk; t += kThreads) {
      const int mi = t / nblk, b = t - mi * nblk;
      const float* v = xs + mi * row_stride + xpad(b * 32);
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 32; ++j) s += v[j];
      sums[mi * (kc >> 5) + b] = s;
    }
  }
}

template <int FMT>
__device__ __forceinline__ void load_pair(uint32_t (&d)[Fmt<FMT>::pair_dwords], const uint8_t* p) {
  const u32x4_a4* v = reinterpret_cast<const u32x4_a4*>(p);
  if constexpr (FMT == kQ8_0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_a4 t = __builtin_nontemporal_load(v + i);
      d[4 * i] = t.x; d[4 * i + 1] = t.y; d[4 * i + 2] = t.z; d[4 * i + 3] = t.w;
    }
    d[16] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p) + 16);
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const u32x4_a4 t = __builtin_nontemporal_load(v + i);
      d[4 * i] = t.x; d[4 * i + 1] = t.y; d[4 * i + 2] = t.z; d[4 * i + 3] = t.w;
    }
    d[8] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p) + 8);
  }
}

// Sum of 4 signed codes (bytes of w) times x[0..3].
__device__ __forceinline__ float dot4_s8(uint32_t w, const float* xv, float s) {
  s = fmaf(sbyte<0>(w), xv[0], s);
  s = fmaf(sbyte<1>(w), xv[1], s);
  s = fmaf(sbyte<2>(w), xv[2], s);
  s = fmaf(sbyte<3>(w), xv[3], s);
  return s;
}

// q4_0: 4 nibble bytes -> elements e..e+3 (low) and e+16..e+19 (high) as
// unsigned 0..15; the -8 offset is folded in by the caller via block sums.
__device__ __forceinline__ float dot8_u4(uint32_t q, const float* xlo, const float* xhi, float s) {
  const uint32_t lo = q & 0x0F0F0F0Fu;
  const uint32_t hi = (q >> 4) & 0x0F0F0F0Fu;
  s = fmaf(ubyte<0>(lo), xlo[0], s);
  s = fmaf(ubyte<1>(lo), xlo[1], s);
  s = fmaf(ubyte<2>(lo), xlo[2], s);
  s = fmaf(ubyte<3>(lo), xlo[3], s);
  s = fmaf(ubyte<0>(hi), xhi[0], s);
  s = fmaf(ubyte<1>(hi), xhi[1], s);
  s = fmaf(ubyte<2>(hi), xhi[2], s);
  s = fmaf(ubyte<3>(hi), xhi[3], s);
  return s;
}

// Contribution of one pair (two blocks) against the 64 x values xv
// (xv[0..31] block 0, xv[32..63] block 1).  xsum: the two block sums (q4_0).
template <int FMT>
__device__ __forceinline__ float pair_dot(const uint32_t (&d)[Fmt<FMT>::pair_dwords],
                                          const float* xv, const float* xsum, float acc) {
  if constexpr (FMT == kQ8_0) {
    // block 0: scale in bytes 0-1, codes in bytes 2..33
    float s0 = 0.f;
    s0 = fmaf(sbyte<2>(d[0]), xv[0], s0);
    s0 = fmaf(sbyte<3>(d[0]), xv[1], s0);
#pragma unroll
    for (int i = 1; i < 8; ++i) s0 = dot4_s8(d[i], xv + 2 + 4 * (i - 1), s0);
    s0 = fmaf(sbyte<0>(d[8]), xv[30], s0);
    s0 = fmaf(sbyte<1>(d[8]), xv[31], s0);
    // block 1: scale in bytes 34-35 (upper half of dword 8), codes dwords 9..16
    float s1 = 0.f;
#pragma unroll
    for (int i = 9; i < 17; ++i) s1 = dot4_s8(d[i], xv + 32 + 4 * (i - 9), s1);
    acc = fmaf(half_bits_to_float(d[0] & 0xFFFFu), s0, acc);
    acc = fmaf(half_bits_to_float(d[8] >> 16), s1, acc);
  } else {
    // block 0: scale bytes 0-1, nibble bytes 2..17 (realign by 2 bytes)
    float s0 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = __builtin_amdgcn_alignbyte(d[i + 1], d[i], 2);
      s0 = dot8_u4(q, xv + 4 * i, xv + 16 + 4 * i, s0);
    }
    float s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) s1 = dot8_u4(d[5 + i], xv + 32 + 4 * i, xv + 48 + 4 * i, s1);
    s0 = fmaf(-8.f, xsum[0], s0);
    s1 = fmaf(-8.f, xsum[1], s1);
    acc = fmaf(half_bits_to_float(d[0] & 0xFFFFu), s0, acc);
    acc = fmaf(half_bits_to_float(d[4] >> 16), s1, acc);
  }
  return acc;
}

// Small-batch path: MT activation rows per launch share every weight decode.
template <int FMT, int MT>
__global__ __launch_bounds__(kThreads) void qgemm_pairs_kernel(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ y, int m,
    int n, int k, int kc, int vec_ok) {
  extern __shared__ float xs[];
  constexpr int BB = Fmt<FMT>::block_bytes;
  constexpr int PD = Fmt<FMT>::pair_dwords;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long row_bytes = static_cast<long long>(k >> 5) * BB;
  const int row = blockIdx.x * kWaves + wave;
  const int mt = min(MT, m);
  float acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = 0.f;
  const int row_stride = xpad(kc);

  for (int c0 = 0; c0 < k; c0 += kc) {
    const int clen = min(kc, k - c0);
    if (c0) __syncthreads();
    stage_x<FMT>(xs, x, k, mt, c0, clen, kc, vec_ok != 0);
    __syncthreads();
    const int pbeg = c0 >> 6, pend = (c0 + clen) >> 6;
    const float* sums = xs + mt * row_stride;
    for (int p = first_pair(pbeg, lane); p < pend; p += 64) {
      uint32_t d[PD];
      load_pair<FMT>(d, W + min(row, n - 1) * row_bytes + static_cast<long long>(p) * (2 * BB));
#pragma unroll
      for (int mi = 0; mi < MT; ++mi) {
        if (mi < mt) {
          float xv[64];
          const float* xsrc = xs + mi * row_stride + xpad((p - pbeg) * 64);
#pragma unroll
          for (int j = 0; j < 64; j += 4)
            *reinterpret_cast<float4*>(xv + j) = *reinterpret_cast<const float4*>(xsrc + j);
          float xsum[2] = {0.f, 0.f};
          if constexpr (FMT == kQ4_0) {
            xsum[0] = sums[mi * (kc >> 5) + 2 * (p - pbeg)];
            xsum[1] = sums[mi * (kc >> 5) + 2 * (p - pbeg) + 1];
          }
          acc[mi] = pair_dot<FMT>(d, xv, xsum, acc[mi]);
        }
      }
    }
  }
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    if (mi < mt) {
      const float t = wave_sum(acc[mi]);
      if (lane == 0 && row < n) y[static_cast<long long>(mi) * n + row] = t;
    }
  }
}

// Any K % 32 == 0 and any byte alignment: one wave per output row, lane per
// block, byte loads.  Used when K/32 is odd or W is not 4-byte aligned.
template <int FMT>
__global__ __launch_bounds__(kThreads) void qgemm_generic_kernel(
    const uint8_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ y, int m,
    int n, int k) {
  constexpr int BB = Fmt<FMT>::block_bytes;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= n) return;
  const int nb = k >> 5;
  const uint8_t* wrow = W + static_cast<long long>(row) * nb * BB;
  for (int mi = 0; mi < m; ++mi) {
    const float* xr = x + static_cast<long long>(mi) * k;
    float acc = 0.f;
    for (int b = lane; b < nb; b += 64) {
      const uint8_t* blk = wrow + static_cast<long long>(b) * BB;
      const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
      float s = 0.f;
      if constexpr (FMT == kQ8_0) {
        for (int j = 0; j < 32; ++j) s = fmaf(static_cast<float>(static_cast<int8_t>(blk[2 + j])), xr[b * 32 + j], s);
      } else {
        for (int j = 0; j < 16; ++j) {
          s = fmaf(static_cast<float>((blk[2 + j] & 15) - 8), xr[b * 32 + j], s);
          s = fmaf(static_cast<float>((blk[2 + j] >> 4) - 8), xr[b * 32 + 16 + j], s);
        }
      }
      acc = fmaf(d, s, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[static_cast<long long>(mi) * n + row] = acc;
  }
}

// Largest multiple of 64 elements whose padded x rows (and q4_0 block sums)
// for `mt` activation rows fit the LDS budget, capped at k.
int chunk_for(int fmt, int mt, int k) {
  const int per64 = 68 + (fmt == kQ4_0 ? 2 : 0);  // floats per 64 elements
  int kc = (kLdsBudget / (4 * mt * per64)) * 64;
  const int kr = (k + 63) / 64 * 64;
  return kc < kr ? kc : kr;
}

size_t lds_bytes(int fmt, int mt, int kc) {
  return sizeof(float) * (static_cast<size_t>(mt) * (kc + (kc >> 6) * 4) +
                          (fmt == kQ4_0 ? static_cast<size_t>(mt) * (kc >> 5) : 0));
}

template <int FMT>
hipError_t launch_fmt(const uint8_t* W, const float* x, float* y, int m, int n, int k,
                      hipStream_t s, const GemvTuning& t, bool noalloc) {
  const bool fast = ((k >> 5) % 2 == 0) && (reinterpret_cast<uintptr_t>(W) % 4 == 0);
  if (!fast) {
    qgemm_generic_kernel<FMT><<<(n + kWaves - 1) / kWaves, kThreads, 0, s>>>(W, x, y, m, n, k);
    return hipGetLastError();
  }
  const int vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (k % 4 == 0);
  if (m == 1) return launch_qgemv_dot(FMT, W, x, y, n, k, t.rows_per_wave, s);
  // The exact-digit rows kernel (one pass over W, no scratch, no prep launch;
  // every row bit-identical to the GEMV of that row) where it measured faster
  // than the MFMA kernels on MI355X: m = 2 with K in one 4096-column chunk,
  // and m = 3, 4 when N is also small enough that the MFMA grid leaves CUs
  // idle (q8_0 / q4_0, K = 4096: m = 2 N = 4096 8.2 / 7.4 us vs 11.8 / 11.3;
  // m = 4 N = 4096 11.3 / 10.1 vs 11.3 / 11.5; m = 4 N = 14336 23.4 vs 18.8).
  const bool rows_pays = k <= 4096 && (m == 2 || (m <= 4 && n <= 8192));
  if (m <= 8 && k % 64 == 0 && t.qgemm_rows >= 0 && (t.qgemm_rows > 0 || rows_pays)) {
    int rb = t.rows_per_wave == 1 || t.rows_per_wave == 2 || t.rows_per_wave == 4 ? t.rows_per_wave : 0;
    if (rb == 0) rb = m == 2 ? 1 : 2;
    return launch_qgemm_rows(FMT, W, x, y, n, k, m, rb, s);
  }
  // The MFMA path addresses W with 32-bit offsets from its base (plus up to
  // one stage of row overrun).
  const long long w_bytes = static_cast<long long>(n) * (k / 32) * Fmt<FMT>::block_bytes;
  if (k % 64 == 0 && w_bytes + 4096 < (1LL << 32))
    return noalloc ? launch_qgemm_mfma_noalloc(FMT, W, x, y, m, n, k, s)
                   : launch_qgemm_mfma(FMT, W, x, y, m, n, k, s, t.qgemm_waves, t.qgemm_stages,
                                       t.qgemm_panel, t.qgemm_fold);
  const int grid = (n + kWaves - 1) / kWaves;
  for (int m0 = 0; m0 < m; m0 += 8) {
    const int mt = m - m0 < 8 ? m - m0 : 8;
    const int kc = chunk_for(FMT, mt, k);
    const size_t lds = lds_bytes(FMT, mt, kc);
    const float* xm = x + static_cast<long long>(m0) * k;
    float* ym = y + static_cast<long long>(m0) * n;
    const int v = vec;
    if (mt <= 2)
      qgemm_pairs_kernel<FMT, 2><<<grid, kThreads, lds, s>>>(W, xm, ym, mt, n, k, kc, v);
    else if (mt <= 4)
      qgemm_pairs_kernel<FMT, 4><<<grid, kThreads, lds, s>>>(W, xm, ym, mt, n, k, kc, v);
    else
      qgemm_pairs_kernel<FMT, 8><<<grid, kThreads, lds, s>>>(W, xm, ym, mt, n, k, kc, v);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_qgemm(int fmt, const void* W, const float* x, float* y, long long m,
                        long long n, long long k, hipStream_t s, const GemvTuning& t,
                        bool noalloc) {
  const auto* w = static_cast<const uint8_t*>(W);
  return fmt == kQ8_0 ? launch_fmt<kQ8_0>(w, x, y, (int)m, (int)n, (int)k, s, t, noalloc)
                      : launch_fmt<kQ4_0>(w, x, y, (int)m, (int)n, (int)k, s, t, noalloc);
}

// Compute units of the current device (256 on a full MI355X; fewer under a
// compute partition).  The tile and split planners size their grids by it.
int device_cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  return cus;
}

}  // namespace qc
