// W8A8 int8 GEMM on gfx950 int8 MFMA (v_mfma_i32_16x16x64_i8) with exact
// int32 accumulation and the reference's f32 epilogue.
//
// Semantics (src/dispatch/int8_gemm.cpp:67-94, kernels/quantization/
// int8_gemm_ref.cpp:9-32 of the reference):
//   dot[m][n] = sum_k W[n][k] * X[m][k]         (exact integer)
//   dot      -= zp[m] * row_sum[n]               (asymmetric only, int64)
//   y[m][n]   = (float(dot) * ws[n]) * as[m]     (two IEEE multiplies, no FMA)
// W is [N][K] and X is token-major [M][K]: both operands are K-contiguous.
//
// Tiling: a 256-thread workgroup owns a 128(n) x 128(m) output tile; its
// four wavefronts each own 64 x 64 as 4 x 4 MFMA tiles of 16 x 16.  Per
// K step of 64 the workgroup stages W[128][64] and X[128][64] (8 KB each) in
// LDS; a lane's 16-byte operand fragment is one row's 16-byte chunk, stored
// with the chunk index XOR-swizzled by (row >> 2) & 3 so the 16 rows read by
// one quarter-wave hit 16 distinct bank groups.  The next K step's global
// loads are issued before the current step's MFMAs.
//
// The MFMA's "A" operand is the W tile, "B" the X tile, so each lane's four
// accumulators are 4 consecutive n of one m: the epilogue stores 16 bytes.
#include "qc_device.h"
#include "qc_internal.h"

namespace qc {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kTileN = 128;
constexpr int kTileM = 128;
constexpr int kStepK = 64;
// Largest K for which an int32 accumulator cannot overflow:
// 131071 * 128 * 128 < 2^31.
constexpr long long kMaxK32 = 131071;

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * kStepK + ((chunk ^ ((row >> 2) & 3)) << 4);
}

__device__ __forceinline__ v4i load16(const int8_t* base, long long rows, long long row,
                                      long long ld, long long col, long long k) {
  v4i v = {0, 0, 0, 0};
  if (row < rows && col < k) v = *reinterpret_cast<const v4i*>(base + row * ld + col);
  return v;
}

__device__ __forceinline__ float epilogue(int32_t acc, long long m, long long n, const float* ws,
                                          const float* as, const int32_t* row_sum, const int* zp,
                                          bool asym) {
  if (asym) {
    const long long dot = static_cast<long long>(acc) - static_cast<long long>(zp[m]) * row_sum[n];
    return (static_cast<float>(dot) * ws[n]) * as[m];
  }
  return (static_cast<float>(acc) * ws[n]) * as[m];
}

__global__ __launch_bounds__(kThreads) void int8_gemm_mfma(
    const int8_t* __restrict__ W, const int8_t* __restrict__ X, const float* __restrict__ ws,
    const float* __restrict__ as, const int32_t* __restrict__ row_sum, const int* __restrict__ zp,
    float* __restrict__ y, int32_t* __restrict__ acc_out, int M, int N, int K, int asym,
    int* status) {
  __shared__ __attribute__((aligned(16))) int8_t sW[kTileN * kStepK];
  __shared__ __attribute__((aligned(16))) int8_t sX[kTileM * kStepK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const long long n0 = static_cast<long long>(blockIdx.x) * kTileN;
  const long long m0 = static_cast<long long>(blockIdx.y) * kTileM;

  // global -> LDS mapping: two 16-byte chunks per thread per operand
  const int lrow = tid >> 2;  // 0..63 (and +64)
  const int lchunk = tid & 3;

  v4i gw[2], gx[2];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      gw[h] = load16(W, N, n0 + lrow + 64 * h, K, k0 + 16 * lchunk, K);
      gx[h] = load16(X, M, m0 + lrow + 64 * h, K, k0 + 16 * lchunk, K);
    }
  };

  v4i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  const int wn = (wave >> 1) * 64;  // wave's n offset inside the tile
  const int wm = (wave & 1) * 64;   // wave's m offset inside the tile
  const int frow = lane & 15;
  const int fchunk = lane >> 4;

  fetch(0);
  for (int k0 = 0; k0 < K; k0 += kStepK) {
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      *reinterpret_cast<v4i*>(sW + swz(lrow + 64 * h, lchunk)) = gw[h];
      *reinterpret_cast<v4i*>(sX + swz(lrow + 64 * h, lchunk)) = gx[h];
    }
    __syncthreads();
    if (k0 + kStepK < K) fetch(k0 + kStepK);
    v4i a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const v4i*>(sW + swz(wn + 16 * i + frow, fchunk));
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const v4i*>(sX + swz(wm + 16 * j + frow, fchunk));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
  }

  // C layout of a 16x16 tile: lane holds rows 4*(lane>>4)+e (n), column lane&15 (m).
  if (acc_out != nullptr) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long long m = m0 + wm + 16 * j + (lane & 15);
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const long long nb = n0 + wn + 16 * i + 4 * (lane >> 4);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (nb + e < N) acc_out[m * N + nb + e] = acc[i][j][e];
      }
    }
    return;
  }
  bool bad = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const long long m = m0 + wm + 16 * j + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const long long nb = n0 + wn + 16 * i + 4 * (lane >> 4);
      float out[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const long long n = nb + e < N ? nb + e : N - 1;
        out[e] = epilogue(acc[i][j][e], m, n, ws, as, row_sum, zp, asym != 0);
        bad |= !isfinite(ws[n]);
      }
      bad |= !isfinite(as[m]);
      float* dst = y + m * N + nb;
      if (nb + 3 < N && (N & 3) == 0) {
        *reinterpret_cast<float4*>(dst) = float4{out[0], out[1], out[2], out[3]};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (nb + e < N) dst[e] = out[e];
      }
    }
  }
  if (status != nullptr && __any(bad) && lane == 0) *status = 3;
}

// Exact fallback for any shape/alignment and for K beyond the int32 bound:
// one thread per output, int64 accumulation.
__global__ __launch_bounds__(kThreads) void int8_gemm_simple(
    const int8_t* __restrict__ W, const int8_t* __restrict__ X, const float* __restrict__ ws,
    const float* __restrict__ as, const int32_t* __restrict__ row_sum, const int* __restrict__ zp,
    float* __restrict__ y, int32_t* __restrict__ acc_out, long long M, long long N, long long K,
    int asym, int* status) {
  const long long item = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (item >= M * N) return;
  const long long m = item / N, n = item - m * N;
  long long dot = 0;
  const int8_t* w = W + n * K;
  const int8_t* x = X + m * K;
  for (long long i = 0; i < K; ++i) dot += static_cast<int>(w[i]) * static_cast<int>(x[i]);
  if (acc_out != nullptr) {
    acc_out[item] = static_cast<int32_t>(dot);
    return;
  }
  if (asym) dot -= static_cast<long long>(zp[m]) * row_sum[n];
  y[item] = (static_cast<float>(dot) * ws[n]) * as[m];
  if (status != nullptr && !(isfinite(ws[n]) && isfinite(as[m]))) *status = 3;
}

}  // namespace

hipError_t launch_int8_gemm(const int8_t* W, const int8_t* X, const float* ws, const float* as,
                            const int32_t* row_sum, const int* zp, float* y, int32_t* acc_out,
                            long long m, long long n, long long k, bool asymmetric, int* status,
                            hipStream_t s) {
  const bool aligned = reinterpret_cast<uintptr_t>(W) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(X) % 16 == 0 && k % 16 == 0;
  const bool fits = m <= 0x7FFFFFFFLL && n <= 0x7FFFFFFFLL && k <= kMaxK32;
  if (aligned && fits) {
    const dim3 grid(static_cast<unsigned>((n + kTileN - 1) / kTileN),
                    static_cast<unsigned>((m + kTileM - 1) / kTileM));
    int8_gemm_mfma<<<grid, kThreads, 0, s>>>(W, X, ws, as, row_sum, zp, y, acc_out, (int)m,
                                             (int)n, (int)k, asymmetric ? 1 : 0, status);
    return hipGetLastError();
  }
  const long long items = m * n;
  int8_gemm_simple<<<static_cast<unsigned>((items + kThreads - 1) / kThreads), kThreads, 0, s>>>(
      W, X, ws, as, row_sum, zp, y, acc_out, m, n, k, asymmetric ? 1 : 0, status);
  return hipGetLastError();
}

}  // namespace qc
