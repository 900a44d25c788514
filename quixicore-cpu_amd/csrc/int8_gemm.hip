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
// Tiling: a 256-thread workgroup owns a TN(n) x TM(m) output tile; its four
// wavefronts form a 2 x 2 grid of (TN/2) x (TM/2) wave tiles made of 16 x 16
// MFMA tiles.  The MFMA "A" operand is the W tile and "B" the X tile, so each
// lane's four accumulators are 4 consecutive n of one m and the epilogue
// stores 16 bytes.  Per K step of 64 the workgroup stages W[TN][64] and
// X[TM][64] in LDS; a lane's 16-byte operand fragment is one row's 16-byte
// chunk, stored with the chunk index XOR-swizzled by (row >> 2) & 3 so the 16
// rows read by one quarter-wave hit 16 distinct bank groups.
//
// Pipeline: two LDS buffers and one register stage.  Iteration k stores the
// registers holding step k+1 into the idle LDS buffer, issues the global loads
// of step k+2, computes step k from the other buffer, then meets the
// workgroup at a single barrier.
#include "qc_device.h"
#include "qc_internal.h"

namespace qc {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kStepK = 64;
// Largest K for which an int32 accumulator cannot overflow:
// 131071 * 128 * 128 < 2^31.
constexpr long long kMaxK32 = 131071;

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * kStepK + ((chunk ^ ((row >> 2) & 3)) << 4);
}

// Branch-free guarded 16-byte load: an out-of-range row or K chunk reads a
// clamped in-range address; the caller zeroes it when it is staged into LDS
// (one step later), so neither a branch nor the select forces a wait on the
// load before the MFMAs of the current step.
__device__ __forceinline__ v4i load16(const int8_t* base, long long rows, long long row,
                                      long long ld, long long col, long long k, bool& ok) {
  ok = row < rows && col < k;
  const long long r = row < rows ? row : rows - 1;
  const long long c = col < k ? col : k - 16;
  return *reinterpret_cast<const v4i*>(base + r * ld + c);
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

template <int TN, int TM>
__global__ __launch_bounds__(kThreads) void int8_gemm_mfma(
    const int8_t* __restrict__ W, const int8_t* __restrict__ X, const float* __restrict__ ws,
    const float* __restrict__ as, const int32_t* __restrict__ row_sum, const int* __restrict__ zp,
    float* __restrict__ y, int32_t* __restrict__ acc_out, int M, int N, int K, int tiles_n,
    int asym, int* status) {
  constexpr int WN = TN / 2, WM = TM / 2;        // wave tile
  constexpr int FN = WN / 16, FM = WM / 16;      // MFMA tiles per wave
  constexpr int LW = TN * 4 / kThreads;          // 16-byte W chunks per thread per step
  constexpr int LX = TM * 4 / kThreads;          // 16-byte X chunks per thread per step
  __shared__ __attribute__((aligned(16))) int8_t sW[2][TN * kStepK];
  __shared__ __attribute__((aligned(16))) int8_t sX[2][TM * kStepK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const long long n0 = static_cast<long long>(blockIdx.x % tiles_n) * TN;
  const long long m0 = static_cast<long long>(blockIdx.x / tiles_n) * TM;

  // global -> LDS mapping: thread t moves chunk (t & 3) of rows (t >> 2) + 64 j
  const int lrow = tid >> 2;
  const int lchunk = tid & 3;
  v4i gw[LW], gx[LX];
  bool okw[LW], okx[LX];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int j = 0; j < LW; ++j)
      gw[j] = load16(W, N, n0 + lrow + 64 * j, K, k0 + 16 * lchunk, K, okw[j]);
#pragma unroll
    for (int j = 0; j < LX; ++j)
      gx[j] = load16(X, M, m0 + lrow + 64 * j, K, k0 + 16 * lchunk, K, okx[j]);
  };
  const v4i zero = {0, 0, 0, 0};
  auto stage = [&](int buf) {
#pragma unroll
    for (int j = 0; j < LW; ++j)
      *reinterpret_cast<v4i*>(&sW[buf][swz(lrow + 64 * j, lchunk)]) = okw[j] ? gw[j] : zero;
#pragma unroll
    for (int j = 0; j < LX; ++j)
      *reinterpret_cast<v4i*>(&sX[buf][swz(lrow + 64 * j, lchunk)]) = okx[j] ? gx[j] : zero;
  };

  v4i acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  const int wn = (wave >> 1) * WN;
  const int wm = (wave & 1) * WM;
  const int frow = lane & 15;
  const int fchunk = lane >> 4;
  const int nk = (K + kStepK - 1) / kStepK;

  fetch(0);
  stage(0);
  if (nk > 1) fetch(kStepK);
  __syncthreads();
  for (int k = 0; k < nk; ++k) {
    const int buf = k & 1;
    if (k + 1 < nk) stage(buf ^ 1);
    if (k + 2 < nk) fetch((k + 2) * kStepK);
    v4i a[FN], b[FM];
#pragma unroll
    for (int i = 0; i < FN; ++i) a[i] = *reinterpret_cast<const v4i*>(&sW[buf][swz(wn + 16 * i + frow, fchunk)]);
#pragma unroll
    for (int j = 0; j < FM; ++j) b[j] = *reinterpret_cast<const v4i*>(&sX[buf][swz(wm + 16 * j + frow, fchunk)]);
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }

  // C layout of a 16x16 tile: lane holds rows 4*(lane>>4)+e (n), column lane&15 (m).
  if (acc_out != nullptr) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const long long m = m0 + wm + 16 * j + (lane & 15);
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < FN; ++i) {
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
  for (int j = 0; j < FM; ++j) {
    const long long m = m0 + wm + 16 * j + (lane & 15);
    if (m >= M) continue;
    const float am = as[m];
    bad |= !isfinite(am);
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const long long nb = n0 + wn + 16 * i + 4 * (lane >> 4);
      float out[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const long long n = nb + e < N ? nb + e : N - 1;
        out[e] = epilogue(acc[i][j][e], m, n, ws, as, row_sum, zp, asym != 0);
        bad |= !isfinite(ws[n]);
      }
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

template <int TN, int TM>
hipError_t launch_tile(const int8_t* W, const int8_t* X, const float* ws, const float* as,
                       const int32_t* row_sum, const int* zp, float* y, int32_t* acc_out,
                       long long m, long long n, long long k, bool asymmetric, int* status,
                       hipStream_t s) {
  const long long tiles_n = (n + TN - 1) / TN;
  const long long tiles_m = (m + TM - 1) / TM;
  int8_gemm_mfma<TN, TM><<<static_cast<unsigned>(tiles_n * tiles_m), kThreads, 0, s>>>(
      W, X, ws, as, row_sum, zp, y, acc_out, (int)m, (int)n, (int)k, (int)tiles_n,
      asymmetric ? 1 : 0, status);
  return hipGetLastError();
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
    if (m >= 256)
      return launch_tile<128, 256>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k, asymmetric,
                                   status, s);
    return launch_tile<128, 128>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k, asymmetric,
                                 status, s);
  }
  const long long items = m * n;
  int8_gemm_simple<<<static_cast<unsigned>((items + kThreads - 1) / kThreads), kThreads, 0, s>>>(
      W, X, ws, as, row_sum, zp, y, acc_out, m, n, k, asymmetric ? 1 : 0, status);
  return hipGetLastError();
}

}  // namespace qc
