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
#include "qc_int8_ring.h"
#include "qc_internal.h"

namespace qc {
namespace {

// 16-byte store that only assumes the 4-byte alignment of a float pointer
// (global_store_dwordx4 accepts dword-aligned addresses).
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

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

// Writes one wavefront's FN x FM grid of 16 x 16 accumulator tiles whose
// origin is (mw, nw).  C layout of a 16x16 tile: the lane holds n rows
// 4*(lane>>4)+e and m column lane&15.
template <int FN, int FM>
__device__ __forceinline__ void write_tile(const v4i (&acc)[FN][FM], long long mw, long long nw,
                                           int lane, int M, int N, const float* ws,
                                           const float* as, const int32_t* row_sum,
                                           const int* zp, float* y, int32_t* acc_out, int asym,
                                           int* status) {
  if (acc_out != nullptr) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const long long m = mw + 16 * j + (lane & 15);
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const long long nb = nw + 16 * i + 4 * (lane >> 4);
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
    const long long m = mw + 16 * j + (lane & 15);
    if (m >= M) continue;
    const float am = as[m];
    bad |= !isfinite(am);
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const long long nb = nw + 16 * i + 4 * (lane >> 4);
      float out[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const long long n = nb + e < N ? nb + e : N - 1;
        out[e] = epilogue(acc[i][j][e], m, n, ws, as, row_sum, zp, asym != 0);
        bad |= !isfinite(ws[n]);
      }
      float* dst = y + m * N + nb;
      if (nb + 3 < N && (N & 3) == 0) {
        *reinterpret_cast<f32x4_a4*>(dst) = f32x4_a4{out[0], out[1], out[2], out[3]};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (nb + e < N) dst[e] = out[e];
      }
    }
  }
  if (status != nullptr && __any(bad) && lane == 0) *status = 3;
}

// Waits until at most G * min(D, ahead) loads are outstanding: the loads of
// the `ahead` steps issued after the one needed now (at most D of them).
template <int G, int D>
__device__ __forceinline__ void wait_step(int ahead) {
  if constexpr (D <= 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= D) wait_vmcnt<G * D>();
    else wait_step<G, D - 1>(ahead);
  }
}

// Direct-to-LDS pipelined kernel (K % 64 == 0).  An S-deep ring of LDS stages,
// each holding W[TN][64] and X[TM][64] as 1 KB groups of 16 rows, is filled
// with global_load_lds_dwordx4: one instruction moves a group, lane l writing
// LDS bytes [16l, 16l+16) of it, i.e. row l>>2 at position l&3.  The lane
// fetches logical chunk (l&3) ^ (l>>4), which realises the same XOR swizzle
// as swz() for the fragment reads.  Loads run S-1 steps ahead of the MFMAs;
// rows beyond M or N load a clamped in-range row whose products are never
// stored.
template <int TN, int TM, int S>
__global__ __launch_bounds__(kThreads) void int8_gemm_dma(
    const int8_t* __restrict__ W, const int8_t* __restrict__ X, const float* __restrict__ ws,
    const float* __restrict__ as, const int32_t* __restrict__ row_sum, const int* __restrict__ zp,
    float* __restrict__ y, int32_t* __restrict__ acc_out, int M, int N, int K, int tiles_n,
    int tiles_m, int asym, int* status) {
  constexpr int WN = TN / 2, WM = TM / 2;
  constexpr int FN = WN / 16, FM = WM / 16;
  constexpr int GW = TN / 16 / 4, GX = TM / 16 / 4;  // 1 KB groups per wave per step
  constexpr int G = GW + GX;
  constexpr int kStage = (TN + TM) * kStepK;
  static_assert(GW >= 1 && GX >= 1 && S >= 2, "tile shape");
  static_assert(G * (S - 2) < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) int8_t ring[S * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tn, tm;
  tile_of(blockIdx.x, tiles_n * tiles_m, tiles_n, tiles_m, tn, tm);
  const long long n0 = static_cast<long long>(tn) * TN;
  const long long m0 = static_cast<long long>(tm) * TM;

  // Source row pointers of this lane's groups, at logical chunk (l&3)^(l>>4).
  const int chunk = ((lane & 3) ^ (lane >> 4)) * 16;
  const int8_t* src[G];
#pragma unroll
  for (int j = 0; j < GW; ++j) {
    long long r = n0 + 16 * (wave * GW + j) + (lane >> 2);
    r = r < N ? r : N - 1;
    src[j] = W + r * K + chunk;
  }
#pragma unroll
  for (int j = 0; j < GX; ++j) {
    long long r = m0 + 16 * (wave * GX + j) + (lane >> 2);
    r = r < M ? r : M - 1;
    src[GW + j] = X + r * K + chunk;
  }
  auto issue = [&](int step) {
    int8_t* base = ring + (step % S) * kStage;
    const int k0 = step * kStepK;
#pragma unroll
    for (int j = 0; j < GW; ++j) load_lds16(src[j] + k0, base + (wave * GW + j) * 1024);
#pragma unroll
    for (int j = 0; j < GX; ++j)
      load_lds16(src[GW + j] + k0, base + TN * kStepK + (wave * GX + j) * 1024);
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
  const int nk = K / kStepK;

#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) issue(s);
  for (int k = 0; k < nk; ++k) {
    // Step k must have landed: the loads of the min(S-2, nk-1-k) later steps
    // already issued may stay in flight.
    wait_step<G, S - 2>(nk - 1 - k);
    wait_lgkmcnt0();
    // All waves' loads of step k are visible, and every wave is done reading
    // the stage that the loads issued next will overwrite.
    ring_barrier();
    if (k + S - 1 < nk) issue(k + S - 1);
    const int8_t* sw = ring + (k % S) * kStage;
    const int8_t* sx = sw + TN * kStepK;
    v4i a[FN], b[FM];
#pragma unroll
    for (int i = 0; i < FN; ++i) a[i] = *reinterpret_cast<const v4i*>(&sw[swz(wn + 16 * i + frow, fchunk)]);
#pragma unroll
    for (int j = 0; j < FM; ++j) b[j] = *reinterpret_cast<const v4i*>(&sx[swz(wm + 16 * j + frow, fchunk)]);
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
  }
  write_tile<FN, FM>(acc, m0 + wm, n0 + wn, lane, M, N, ws, as, row_sum, zp, y, acc_out, asym,
                     status);
}

// Epilogue for 32 x 32 accumulator tiles (v_mfma_i32_32x32x32_i8 C layout:
// the lane holds m column lane&31 and, in register e, n row
// 8*(e>>2) + 4*(lane>>5) + (e&3): four runs of 4 consecutive n).  Every
// scale (and zero-point term) the lane needs is loaded up front, so the
// whole epilogue waits on memory once instead of once per output group.
template <int FN, int FM>
__device__ __forceinline__ void write_tile32(const v16i (&acc)[FN][FM], long long mw,
                                             long long nw, int lane, int M, int N,
                                             const float* ws, const float* as,
                                             const int32_t* row_sum, const int* zp, float* y,
                                             int32_t* acc_out, int asym, int* status) {
  if (acc_out != nullptr) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const long long m = mw + 32 * j + (lane & 31);
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const long long nb = nw + 32 * i + 8 * g + 4 * (lane >> 5);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (nb + e < N) acc_out[m * N + nb + e] = acc[i][j][4 * g + e];
        }
    }
    return;
  }
  float wsv[FN][16], asv[FM];
  int32_t rsv[FN][16], zpv[FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      long long n = nw + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      n = n < N ? n : N - 1;
      wsv[i][r] = ws[n];
      rsv[i][r] = asym ? row_sum[n] : 0;
    }
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    long long m = mw + 32 * j + (lane & 31);
    m = m < M ? m : M - 1;
    asv[j] = as[m];
    zpv[j] = asym ? zp[m] : 0;
  }
  bool bad = false;
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const long long m = mw + 32 * j + (lane & 31);
    if (m >= M) continue;
    bad |= !isfinite(asv[j]);
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const long long nb = nw + 32 * i + 8 * g + 4 * (lane >> 5);
        float out[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          float d;
          if (asym)
            d = static_cast<float>(static_cast<long long>(acc[i][j][r]) -
                                   static_cast<long long>(zpv[j]) * rsv[i][r]);
          else
            d = static_cast<float>(acc[i][j][r]);
          out[e] = (d * wsv[i][r]) * asv[j];
          bad |= nb + e < N && !isfinite(wsv[i][r]);
        }
        float* dst = y + m * N + nb;
        if (nb + 3 < N && (N & 3) == 0) {
          *reinterpret_cast<f32x4_a4*>(dst) = f32x4_a4{out[0], out[1], out[2], out[3]};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (nb + e < N) dst[e] = out[e];
        }
      }
    }
  }
  if (status != nullptr && __any(bad) && lane == 0) *status = 3;
}

// The W8A8 GEMM over the full-line ring (qc_int8_ring.h): A = W (n), B = X
// (m), and the reference's epilogue on the wave's accumulators.
template <int TN, int TM, int S, int WGN, int WGM, int KL>
__global__ __launch_bounds__(64 * WGN * WGM) void int8_gemm_ring(
    const int8_t* __restrict__ W, const int8_t* __restrict__ X, const float* __restrict__ ws,
    const float* __restrict__ as, const int32_t* __restrict__ row_sum, const int* __restrict__ zp,
    float* __restrict__ y, int32_t* __restrict__ acc_out, int M, int N, int K, int tiles_n,
    int tiles_m, int asym, int* status) {
  using R = Int8Ring<TN, TM, S, WGN, WGM, KL>;
  __shared__ __attribute__((aligned(1024))) int8_t ring[R::kBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tn, tm;
  tile_of(blockIdx.x, tiles_n * tiles_m, tiles_n, tiles_m, tn, tm);
  const long long n0 = static_cast<long long>(tn) * TN;
  const long long m0 = static_cast<long long>(tm) * TM;
  v16i acc[R::FN][R::FM];
  R::run(W, X, M, N, K, n0, m0, ring, acc);
  write_tile32<R::FN, R::FM>(acc, m0 + R::wave_m(wave), n0 + R::wave_n(wave), lane, M, N, ws,
                             as, row_sum, zp, y, acc_out, asym, status);
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

  write_tile<FN, FM>(acc, m0 + wm, n0 + wn, lane, M, N, ws, as, row_sum, zp, y, acc_out, asym,
                     status);
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

template <int TN, int TM, int S, int WGN, int WGM, int KL = 128>
hipError_t launch_ring(const int8_t* W, const int8_t* X, const float* ws, const float* as,
                       const int32_t* row_sum, const int* zp, float* y, int32_t* acc_out,
                       long long m, long long n, long long k, bool asymmetric, int* status,
                       hipStream_t s) {
  const long long tiles_n = (n + TN - 1) / TN;
  const long long tiles_m = (m + TM - 1) / TM;
  int8_gemm_ring<TN, TM, S, WGN, WGM, KL>
      <<<static_cast<unsigned>(tiles_n * tiles_m), 64 * WGN * WGM, 0, s>>>(
      W, X, ws, as, row_sum, zp, y, acc_out, (int)m, (int)n, (int)k, (int)tiles_n, (int)tiles_m,
      asymmetric ? 1 : 0, status);
  return hipGetLastError();
}

template <int TN, int TM, int S>
hipError_t launch_dma(const int8_t* W, const int8_t* X, const float* ws, const float* as,
                      const int32_t* row_sum, const int* zp, float* y, int32_t* acc_out,
                      long long m, long long n, long long k, bool asymmetric, int* status,
                      hipStream_t s) {
  const long long tiles_n = (n + TN - 1) / TN;
  const long long tiles_m = (m + TM - 1) / TM;
  int8_gemm_dma<TN, TM, S><<<static_cast<unsigned>(tiles_n * tiles_m), kThreads, 0, s>>>(
      W, X, ws, as, row_sum, zp, y, acc_out, (int)m, (int)n, (int)k, (int)tiles_n, (int)tiles_m,
      asymmetric ? 1 : 0, status);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_int8_gemm(const int8_t* W, const int8_t* X, const float* ws, const float* as,
                            const int32_t* row_sum, const int* zp, float* y, int32_t* acc_out,
                            long long m, long long n, long long k, bool asymmetric, int* status,
                            hipStream_t s, int route) {
  const bool aligned = reinterpret_cast<uintptr_t>(W) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(X) % 16 == 0 && k % 16 == 0;
  const bool fits = m <= 0x7FFFFFFFLL && n <= 0x7FFFFFFFLL && k <= kMaxK32;
  const bool can_ring = aligned && fits && k % 32 == 0;
  const bool can_dma = aligned && fits && k % kStepK == 0;
  const bool can_staged = aligned && fits;
  if (route == kInt8Ring && !can_ring) route = kInt8Auto;
  if (route == kInt8Dma && !can_dma) route = kInt8Auto;
  if (route == kInt8Staged && !can_staged) route = kInt8Auto;
  if (route == kInt8Auto)
    route = can_ring ? kInt8Ring : can_staged ? kInt8Staged : kInt8Simple;
  const bool wide = m >= 256;
  switch (route) {
    case kInt8Ring: {
      // Largest tile that still gives (about) every CU a workgroup: the
      // bytes moved per MFMA through a CU's global->LDS path bound this
      // kernel, and a 256 x 256 tile moves 2/3 of what 128 x 256 does.
      auto tiles = [&](long long tn, long long tm) { return ((n + tn - 1) / tn) * ((m + tm - 1) / tm); };
      const long long cus = device_cu_count();
      // up to 32 activation rows (e.g. the canonical projections' digit
      // planes): one 32-row m-tile and an 8-deep ring keep more weight bytes
      // in flight (N=14336 K=4096, 6..24 rows: 11.6-12.0 against 13.5-13.8 us)
      if (m <= 32 && tiles(64, 32) >= cus * 3 / 4)
        return launch_ring<64, 32, 8, 2, 1>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k,
                                            asymmetric, status, s);
      if (wide && tiles(256, 256) >= cus * 3 / 4)
        return launch_ring<256, 256, 2, 4, 2>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k,
                                              asymmetric, status, s);
      if (wide && tiles(128, 256) >= cus * 3 / 4)
        return launch_ring<128, 256, 3, 2, 4>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k,
                                              asymmetric, status, s);
      if (tiles(128, 128) >= cus * 3 / 4)
        return launch_ring<128, 128, 4, 2, 4>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k,
                                              asymmetric, status, s);
      return launch_ring<64, 128, 4, 2, 2>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k,
                                           asymmetric, status, s);
    }
    case kInt8Dma:
      if (wide)
        return launch_dma<128, 256, 4>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k,
                                       asymmetric, status, s);
      return launch_dma<128, 128, 4>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k, asymmetric,
                                     status, s);
    case kInt8Staged:
      if (wide)
        return launch_tile<128, 256>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k, asymmetric,
                                     status, s);
      return launch_tile<128, 128>(W, X, ws, as, row_sum, zp, y, acc_out, m, n, k, asymmetric,
                                   status, s);
    default:
      break;
  }
  const long long items = m * n;
  int8_gemm_simple<<<static_cast<unsigned>((items + kThreads - 1) / kThreads), kThreads, 0, s>>>(
      W, X, ws, as, row_sum, zp, y, acc_out, m, n, k, asymmetric ? 1 : 0, status);
  return hipGetLastError();
}

}  // namespace qc
