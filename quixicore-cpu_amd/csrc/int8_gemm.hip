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

// Output tile of workgroup `b` in an XCD-aware order.  Workgroups are handed
// to the 8 XCDs round-robin (b % 8), each with its own L2, so the tiles one
// XCD runs are made a contiguous range of a banded order (bands of kBandM
// m-tiles, n-tiles within a band): an XCD then reads few W and X panels.
constexpr int kXcds = 8;
constexpr int kBandM = 4;
__device__ __forceinline__ void tile_of(int b, int total, int tiles_n, int tiles_m, int& tn,
                                        int& tm) {
  const int q = total / kXcds, r = total % kXcds;
  const int xcd = b % kXcds, idx = b / kXcds;
  const int t = xcd * q + (xcd < r ? xcd : r) + idx;
  const int band = t / (tiles_n * kBandM);
  const int rem = t - band * tiles_n * kBandM;
  const int left = tiles_m - band * kBandM;
  const int gm = left < kBandM ? left : kBandM;
  tn = rem / gm;
  tm = band * kBandM + rem % gm;
}

// s_waitcnt vmcnt(N), leaving expcnt and lgkmcnt unconstrained (gfx9
// encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
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
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

// global_load_lds_dwordx4: every lane sends 16 bytes from its own global
// address to LDS byte lds + 16 * lane (`lds` is wave-uniform, passed in M0).
// The address-space cast only exists in the device pass.
__device__ __forceinline__ void load_lds16(const int8_t* g, int8_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
#endif
}

// Workgroup barrier for the direct-to-LDS pipeline.  __syncthreads() would
// make the compiler drain every outstanding global->LDS load (vmcnt(0)) and
// defeat the multi-stage prefetch; here the waits are explicit and the empty
// asm statements only stop the compiler moving memory accesses across.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
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

typedef int v16i __attribute__((ext_vector_type(16)));

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

// Full-line ring kernel (K % 32 == 0).  Each K step covers 128 bytes of every
// W and X row of the tile, i.e. whole 128-byte cache lines: the global->LDS
// path delivers markedly more per CU for whole lines than for half lines.
//
// LDS: an S-deep ring of stages; a stage holds W[TN][128] then X[TM][128],
// row-major, with the 16-byte chunk c of row r stored at position
// c ^ ((r >> 1) & 7).  A global_load_lds_dwordx4 moves 8 rows (1 KB): lane l
// writes position l&7 of row l>>3 and so fetches logical chunk
// (l&7) ^ ((r >> 1) & 7).
//
// MFMA: v_mfma_i32_32x32x32_i8 (one wavefront sustains close to the CU's
// int8 rate with it, unlike the 16x16x64 form).  A step is four K quarters
// of 32; the operand of quarter q for a 32-row fragment is, in lane l,
// row l&31, chunk 2q + (l>>5), the same lane->k map for W and X.  Those 64
// reads fall on all 16 four-bank slots 4 times each under the swizzle above.
//
// Schedule (wavefront-uniform, branch-free in the steady state):
//   prologue: issue the loads of steps 0..S-1 into stages 0..S-1;
//   step k, quarter q = 0..2: read the fragments of quarter q+1 while the
//     MFMAs of quarter q run;
//   quarter 3: wait for this wave's loads of step k+1, barrier (all waves'
//     loads are in and every wave has finished reading stage k), issue the
//     loads of step k+S into stage k (with S >= 3 only the first quarter of
//     them; the rest go out before the MFMAs of quarters 1..3 of step k+1),
//     read quarter 0 of step k+1, then the MFMAs of quarter 3.
// Past the last step the loads repeat the last step into stages that are
// never read again, which keeps every wait count a constant.  The last step
// runs separately and, when K is not a multiple of 128, skips the quarters
// past K (their loads read a clamped in-row address and are never used).
template <int TN, int TM, int S, int WGN, int WGM, int KL>
__global__ __launch_bounds__(64 * WGN * WGM) void int8_gemm_ring(
    const int8_t* __restrict__ W, const int8_t* __restrict__ X, const float* __restrict__ ws,
    const float* __restrict__ as, const int32_t* __restrict__ row_sum, const int* __restrict__ zp,
    float* __restrict__ y, int32_t* __restrict__ acc_out, int M, int N, int K, int tiles_n,
    int tiles_m, int asym, int* status) {
  static_assert(KL == 128 || KL == 64, "K step is a whole or a half cache line");
  constexpr int kLine = KL;
  constexpr int QPS = KL / 32;                       // K quarters per step
  constexpr int RPL = 1024 / KL;                     // rows per 1 KB load
  constexpr int CPR = KL / 16;                       // 16-byte chunks per row
  constexpr int NW = WGN * WGM;                      // WGN x WGM grid of wavefronts
  constexpr int WN = TN / WGN, WM = TM / WGM;        // wave tile
  constexpr int FN = WN / 32, FM = WM / 32;          // 32 x 32 tiles per wave
  constexpr int GW = TN / RPL / NW, GX = TM / RPL / NW;  // 1 KB loads per wave per step
  constexpr int G = GW + GX;
  constexpr int kStage = (TN + TM) * kLine;
  static_assert(FN >= 1 && FM >= 1 && GW >= 1 && GX >= 1 && S >= 2, "tile shape");
  static_assert(KL == 64 || (GW % 2 == 0 && GX % 2 == 0), "8-row groups alternate swizzle parity");
  static_assert(G * (S - 1) < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) int8_t ring[S * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tn, tm;
  tile_of(blockIdx.x, tiles_n * tiles_m, tiles_n, tiles_m, tn, tm);
  const long long n0 = static_cast<long long>(tn) * TN;
  const long long m0 = static_cast<long long>(tm) * TM;

  // Load j of a wave covers operand rows r = RPL * (wave * GW + j) + lane / CPR
  // (W; likewise X with GX), lane writing slot lane % CPR of its row.  Swizzle
  // key of row r: (r >> 1) & (CPR - 1).  128-byte lines: 4 * (j & 1) +
  // (lane >> 4), as GW and GX are even; 64-byte halves: (lane >> 3) & 3.
  const int8_t* src[G];
  int coff[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    coff[par] = KL == 128 ? ((lane & 7) ^ (4 * par + (lane >> 4))) * 16
                          : ((lane & 3) ^ ((lane >> 3) & 3)) * 16;
#pragma unroll
  for (int j = 0; j < GW; ++j) {
    long long r = n0 + RPL * (wave * GW + j) + lane / CPR;
    r = r < N ? r : N - 1;
    src[j] = W + r * K;
  }
#pragma unroll
  for (int j = 0; j < GX; ++j) {
    long long r = m0 + RPL * (wave * GX + j) + lane / CPR;
    r = r < M ? r : M - 1;
    src[GW + j] = X + r * K;
  }
  auto issue = [&](int step, int stage) {
    int8_t* base = ring + stage * kStage;
    const int k0 = step * kLine;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      int off = k0 + coff[j & 1];
      off = off < K - 16 ? off : K - 16;
      int8_t* dst = j < GW ? base + (wave * GW + j) * 1024
                           : base + TN * kLine + (wave * GX + (j - GW)) * 1024;
      load_lds16(src[j] + off, dst);
    }
  };

  // Fragment offsets of quarter q within a 32-row block: row lane&31,
  // logical chunk 2q + (lane>>5), stored at that chunk ^ key(row).
  const int t = KL == 128 ? (lane >> 5) ^ ((lane >> 1) & 7) : (lane >> 5) ^ ((lane >> 1) & 3);
  int foff[QPS];
#pragma unroll
  for (int q = 0; q < QPS; ++q) foff[q] = (lane & 31) * kLine + ((2 * q) ^ t) * 16;

  v16i acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  const int wn = (wave / WGM) * WN;
  const int wm = (wave % WGM) * WM;
  const int nq = K / 32;                    // K quarters in total
  const int nk = (nq + QPS - 1) / QPS;      // steps

  v4i fa[2][FN], fb[2][FM];
  auto read_frags = [&](int stage, int q, int slot) {
    const int8_t* sw = ring + stage * kStage + wn * kLine + foff[q];
    const int8_t* sx = ring + stage * kStage + (TN + wm) * kLine + foff[q];
#pragma unroll
    for (int i = 0; i < FN; ++i) fa[slot][i] = *reinterpret_cast<const v4i*>(sw + 32 * i * kLine);
#pragma unroll
    for (int j = 0; j < FM; ++j) fb[slot][j] = *reinterpret_cast<const v4i*>(sx + 32 * j * kLine);
  };
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[slot][i], fb[slot][j], acc[i][j],
                                                          0, 0, 0);
  };

#pragma unroll
  for (int st = 0; st < S; ++st) issue(st < nk ? st : nk - 1, st);
  wait_vmcnt<G * (S - 1)>();
  ring_barrier();
  read_frags(0, 0, 0);
  // With three or more stages the loads of a step are spread over the
  // quarters of the next one (part 0 after the barrier, part q before
  // quarter q's MFMAs) instead of being queued by all waves at once: they
  // are needed only S - 2 steps later.  With two stages they are needed at
  // the end of the next step and go out together.
  constexpr int SPREAD = S >= 3 ? QPS : 1;
  int stage = 0;
  int pstep = 0, pstage = 0;                // the step being loaded and its stage
  auto issue_part = [&](int part) {
    int8_t* base = ring + pstage * kStage;
    const int k0 = pstep * kLine;
#pragma unroll
    for (int j = part * G / SPREAD; j < (part + 1) * G / SPREAD; ++j) {
      int off = k0 + coff[j & 1];
      off = off < K - 16 ? off : K - 16;
      int8_t* dst = j < GW ? base + (wave * GW + j) * 1024
                           : base + TN * kLine + (wave * GX + (j - GW)) * 1024;
      load_lds16(src[j] + off, dst);
    }
  };
  for (int k = 0; k + 1 < nk; ++k) {
#pragma unroll
    for (int q = 1; q < QPS; ++q) {
      if (q < SPREAD && k > 0) issue_part(q);
      read_frags(stage, q, q & 1);
      mfmas((q - 1) & 1);
    }
    // Loads issued: steps up to k+S-1, all parts; step k+1 must be in.
    wait_vmcnt<G * (S - 2)>();
    wait_lgkmcnt0();
    ring_barrier();
    pstep = k + S < nk ? k + S : nk - 1;
    pstage = stage;
    issue_part(0);
    stage = stage + 1 < S ? stage + 1 : 0;
    read_frags(stage, 0, 0);
    mfmas((QPS - 1) & 1);
  }
  {
    const int qn = nq - QPS * (nk - 1);    // 1..QPS quarters in the last step
#pragma unroll
    for (int q = 1; q < QPS; ++q) {
      if (q < qn) read_frags(stage, q, q & 1);
      if (q - 1 < qn) mfmas((q - 1) & 1);
    }
    if (QPS - 1 < qn) mfmas((QPS - 1) & 1);
  }
  // No global->LDS load may still be in flight when the workgroup's LDS is
  // released.
  wait_vmcnt<0>();
  write_tile32<FN, FM>(acc, m0 + wm, n0 + wn, lane, M, N, ws, as, row_sum, zp, y, acc_out, asym,
                       status);
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
