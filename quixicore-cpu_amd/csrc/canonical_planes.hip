// The row-plane route of the canonical int8 projections (two or more
// activation rows; qc_cint8.h has the limits and the entry): each activation
// row encoded once as three int8 digit planes, the weight codes streamed once
// through the int8 MFMA main loop (qc_int8_ring.h), the combination, scales and
// epilogue in the GEMM.  Compiled with the MFMA accumulators in VGPRs
// (-mllvm -amdgpu-mfma-vgpr-form): the grouped fold reads them after every K
// step, and AGPRs would cost a v_accvgpr_read per value (N = 14336, K = 4096,
// groups of 128: M = 16 / 64 / 512 took 35.1 / 57.9 / 262.8 us with AGPRs,
// 32.9 / 51.8 / 254.5 us without).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "qc_cint8.h"
#include "qc_device.h"
#include "qc_digits.h"
#include "qc_int8_ring.h"
#include "qc_internal.h"

namespace qc {

// ---- Row-plane route: two or more activation rows, one scale per weight row
// (or three or more with scale groups of 64 or a multiple of 128 columns,
// five or more with groups of 32)
//
// Every activation row m is encoded once as 22-bit fixed point under one
// exponent for the whole row: e(m) = frexp(max_k |x[m][k]|) - 21 and
// q = rint(x * 2^-e), clamped to [-2^21, 2^21 - 1], split into three int8
// planes q = 2^14 d0 + 2^7 d1 + d2 (d0 in [-128, 127], d1, d2 in [0, 127]).
// The int8 MFMA main loop gives the exact int32 sums
// D_t[m][n] = sum_k code[n][k] d_t[m][k] of all planes.
// The planes of row m are rows 4m + t (t < 3; row 4m + 3 is zero) of an
// int8 matrix [4M][K], the main loop's operand A against the weight codes as
// operand B (qc_int8_ring.h), so each lane's accumulators hold D_0..D_2 of
// one (m, n) and the GEMM's epilogue finishes the output: after the prep, one
// launch per matrix, or one for SwiGLU over gate and up together (per chunk
// of kPlanesChunkM rows).  Writing every D_t to scratch for a separate
// finish kernel instead took 1.5x as long at M = 512 (208 against 137 us,
// N = 14336, K = 4096): 88 MB of int32 sums written and read back.
// The combination forms 2^14 D0 + 2^7 D1 + D2 exactly (an integer below
// 2^53, in double), minus z (2^14 S0 + 2^7 S1 + S2), S_t = sum_k d_t[m][k],
// for an integral zero point z, rounds it once to f32 and scales it by 2^e
// and the row's scale, then runs the shared epilogue.  Each x is held to within
// 2^-21 max_k |x_m|, so |y - y_exact| <= sqrt(K) 2^-21 ||x_m|| ||w_hat_n||:
// 3.1e-5 at K = 4096 and 6.1e-5 at K = 16384 after the contract's
// normalisation.  A row holding NaN or +-inf is computed in f32 from the
// codes and x instead (the reference's result class).
// With scale groups the prep also writes S_t per group and the GEMM folds
// each group's sums into an f32 accumulator at the group's last K step
// (cint8_planes_gemm, GROUPED); the group's scales, zero points and digit
// sums reach the GEMM through the ring's LDS with that step's operands.
namespace {

constexpr int kPlanesChunkM = 1024;     // activation rows per pass: bounds the scratch
constexpr int kPlanesNonfinite = 0x40000000;

// The prep kernel: 1024 threads per activation row, each holding up to 16 of
// its values (four groups of four, K <= 16384) in registers, so the row is
// read once with every load in flight.
constexpr int kPrepThreads = 1024;
constexpr int kPrepWaves = kPrepThreads / 64;
constexpr int kPrepGroups = kPlanesMaxK / (4 * kPrepThreads);

// Maximum over the workgroup of non-negative values (DPP within each wave,
// then the 16 wave maxima read back as four 16-byte words), to every lane.
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max_nonneg(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float4* r4 = reinterpret_cast<const float4*>(red);
  float r = 0.0f;
#pragma unroll
  for (int w = 0; w < kPrepWaves / 4; ++w) {
    const float4 q = r4[w];
    r = fmaxf(r, fmaxf(fmaxf(q.x, q.y), fmaxf(q.z, q.w)));
  }
  return r;
}

// Sum over the 64 lanes of a wavefront, in lane 63 (row sums by row_shr, then
// row broadcasts; lanes a DPP mask leaves out add 0).
template <int CTRL, int ROW_MASK, int BANK_MASK, bool BOUND_ZERO>
__device__ __forceinline__ int dpp_i32_masked(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, BANK_MASK, BOUND_ZERO);
}
__device__ __forceinline__ int wave_sum_lane63_i32(int v) {
  int t = v + dpp_i32_masked<0x111, 0xF, 0xF, true>(v);
  t += dpp_i32_masked<0x112, 0xF, 0xF, true>(v);
  t += dpp_i32_masked<0x113, 0xF, 0xF, true>(v);
  t += dpp_i32_masked<0x114, 0xF, 0xE, false>(t);
  t += dpp_i32_masked<0x118, 0xF, 0xC, false>(t);
  t += dpp_i32_masked<0x142, 0xA, 0xF, false>(t);
  t += dpp_i32_masked<0x143, 0xC, 0xF, false>(t);
  return t;
}

// The three digit sums over the workgroup (exact in int32), to every lane.
__device__ __forceinline__ void block_sum3(int (&v)[3], int (*red)[kPrepWaves]) {
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    v[t] = wave_sum_lane63_i32(v[t]);
    if ((threadIdx.x & 63) == 63) red[t][threadIdx.x >> 6] = v[t];
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const int4* r4 = reinterpret_cast<const int4*>(red[t]);
    int r = 0;
#pragma unroll
    for (int w = 0; w < kPrepWaves / 4; ++w) {
      const int4 q = r4[w];
      r += (q.x + q.y) + (q.z + q.w);
    }
    v[t] = r;
  }
}

// Four consecutive activations of row xr at column c (16-byte loads for
// aligned f32 rows).
__device__ __forceinline__ void load4(const void* x, long long xr, int c, int xtype, bool vec,
                                      float (&v)[4]) {
  if (vec) {
    const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + xr + c);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = load_x(x, xr + c + i, xtype);
  }
}

// One workgroup per activation row (x rows blockIdx.x, ldx apart); the
// planes of row m are rows 4m + t (row 4m + 3 is zeroed).  A row holding NaN
// or +-inf gets the maximum +inf, zero digits and the flag exponent
// kPlanesNonfinite.  The digit sums S_t go to dsum[(m * ngroups + g) * 3 + t]
// over each group g of gsize columns (GROUPED: gsize 32, 64 or a multiple of
// 128, with k % 128 == 0, so the gsize / 4 lanes of a group, at most a half
// wave, lie in one half wave), else over the row (ngroups = 1); only the
// zero-point terms read them, so without zero points (sums false) they are
// neither formed nor written.
constexpr int kPlanesMaxGroups = kPlanesMaxK / 32;
static_assert(kPlanesMaxGroups * 32 >= kPlanesMaxK, "group sums of the smallest groups");
static_assert(kPrepWaves % 4 == 0, "wave partials read as 16-byte words");
template <bool GROUPED>
__global__ __launch_bounds__(kPrepThreads) void cint8_planes_prep(
    const void* __restrict__ x, int xtype, long long ldx, int k, bool vec, int gsize,
    int ngroups, bool sums, int8_t* __restrict__ planes, int* __restrict__ rexp,
    int* __restrict__ dsum) {
  __shared__ __attribute__((aligned(16))) float fred[kPrepWaves];
  __shared__ __attribute__((aligned(16))) int ired[3][kPrepWaves];
  __shared__ int gsum[GROUPED ? 3 * kPlanesMaxGroups : 1];
  if constexpr (GROUPED) {
    if (sums)
      for (int i = threadIdx.x; i < 3 * ngroups; i += kPrepThreads) gsum[i] = 0;
  }
  const int m = blockIdx.x;
  const long long xr = static_cast<long long>(m) * ldx;
  float v[kPrepGroups][4];
  float mx = 0.0f;
#pragma unroll
  for (int g = 0; g < kPrepGroups; ++g) {
    const int c = 4 * (static_cast<int>(threadIdx.x) + g * kPrepThreads);
    if (c < k) {
      load4(x, xr, c, xtype, vec, v[g]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[g][i] = 0.0f;
    }
  }
#pragma unroll
  for (int g = 0; g < kPrepGroups; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, isfinite(v[g][i]) ? fabsf(v[g][i]) : INFINITY);
  mx = block_max(mx, fred);
  const bool bad = !isfinite(mx);
  int ex = 0;
  (void)frexpf(mx, &ex);                       // mx < 2^ex
  const int e = ex - 21;
  int sum[3] = {0, 0, 0};
  int8_t* p0 = planes + (4LL * m) * k;
#pragma unroll
  for (int g = 0; g < kPrepGroups; ++g) {
    const int c = 4 * (static_cast<int>(threadIdx.x) + g * kPrepThreads);
    if (c >= k) continue;                       // whole half waves (k % 128 == 0 when grouped)
    if constexpr (GROUPED) sum[0] = sum[1] = sum[2] = 0;
    uint32_t w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int q = bad ? 0 : __float2int_rn(ldexpf(v[g][i], -e));
      q = q > 2097151 ? 2097151 : q;
      const int d0 = q >> 14, d1 = (q >> 7) & 127, d2 = q & 127;
      sum[0] += d0;
      sum[1] += d1;
      sum[2] += d2;
      w0 |= static_cast<uint32_t>(d0 & 0xFF) << (8 * i);
      w1 |= static_cast<uint32_t>(d1) << (8 * i);
      w2 |= static_cast<uint32_t>(d2) << (8 * i);
    }
    *reinterpret_cast<uint32_t*>(p0 + c) = w0;
    *reinterpret_cast<uint32_t*>(p0 + k + c) = w1;
    *reinterpret_cast<uint32_t*>(p0 + 2LL * k + c) = w2;
    *reinterpret_cast<uint32_t*>(p0 + 3LL * k + c) = 0u;
    if (GROUPED && sums) {
      // the gl consecutive lanes of one group (4 columns each)
      const int gl = gsize < 128 ? gsize / 4 : 32;
#pragma unroll
      for (int t = 0; t < 3; ++t)
        for (int off = 16; off > 0; off >>= 1)
          if (off < gl) sum[t] += __shfl_xor(sum[t], off);
      if ((threadIdx.x & (gl - 1)) == 0) {
        const int grp = c / gsize;
#pragma unroll
        for (int t = 0; t < 3; ++t) atomicAdd(&gsum[3 * grp + t], sum[t]);
      }
    }
  }
  if (threadIdx.x == 0) rexp[m] = bad ? kPlanesNonfinite : e;
  if (!sums) return;
  if constexpr (GROUPED) {
    __syncthreads();
    for (int i = threadIdx.x; i < 3 * ngroups; i += kPrepThreads)
      dsum[3LL * m * ngroups + i] = gsum[i];
  } else {
    block_sum3(sum, ired);
    if (threadIdx.x == 0) {
      dsum[3 * m] = sum[0];
      dsum[3 * m + 1] = sum[1];
      dsum[3 * m + 2] = sum[2];
    }
  }
}

// Projection of activation row (m0 + mm) on row n of one matrix from its
// plane sums a0..a2 (D_0..D_2).
__device__ __forceinline__ float plane_value(int32_t a0, int32_t a1, int32_t a2, const int8_t* w,
                                             const float* scale, const float* zp, long long n,
                                             int mm, int m0, const int* rexp, const int* dsum,
                                             const void* x, int xtype, long long ldx, int k) {
  const int e = rexp[mm];
  const float sc = scale[n];
  if (e == kPlanesNonfinite) {        // the reference's f32 form, block by block
    const int8_t* codes = w + static_cast<long long>(n) * k;
    const long long xr = static_cast<long long>(m0 + mm) * ldx;
    const float z = zp != nullptr ? zp[n] : 0.0f;
    float acc = 0.0f;
    for (int b = 0; b < k; b += 32) acc += cint8_block_f32(codes + b, x, xr + b, xtype, z);
    return sc * acc;
  }
  // 2^14 D0 + 2^7 D1 + D2 (|D_t| < 2^26 for K <= 16384) and the zero-point
  // term are integers below 2^53: exact in double, then rounded once to f32
  const double d = fma(static_cast<double>(a0), 16384.0,
                       fma(static_cast<double>(a1), 128.0, static_cast<double>(a2)));
  float f;
  if (zp != nullptr) {
    const double sx = fma(static_cast<double>(dsum[3 * mm]), 16384.0,
                          fma(static_cast<double>(dsum[3 * mm + 1]), 128.0,
                              static_cast<double>(dsum[3 * mm + 2])));
    int zi;
    if (integral_zero(zp[n], zi)) {
      f = static_cast<float>(fma(-static_cast<double>(zi), sx, d));   // exact: |z sx| < 2^52
    } else {
      f = fmaf(-zp[n], static_cast<float>(sx), static_cast<float>(d));
    }
  } else {
    f = static_cast<float>(d);
  }
  return sc * ldexpf(f, e);
}

// The fused form's matrices and output.  Mode 0: one matrix (w, scale,
// zero) with, on matrix 0 of the call, bias and activation (epi != 0).
// SwiGLU: gate (w, scale, zero) and up (w2, scale2, zero2) of `rows` rows
// each, y = SiLU(gate) * up.  Scales and zero points are [rows][groups], a
// group being gsize columns (groups 1: one per row).
struct PlaneOut {
  const int8_t* w;
  const float* scale;
  const float* zero;
  const int8_t* w2;
  const float* scale2;
  const float* zero2;
  void* y;
  long long ld;
  int ytype;
  int rows;
  const float* bias;
  int act;           // with epi != 0: bias (when given), then linear_activation
  int epi;
  int groups;
  int gsize;
};

// 2^14 a + 2^7 b + c in f32 (each term exact, the sum rounded).
__device__ __forceinline__ float combine_f(long long a, long long b, long long c) {
  return fmaf(static_cast<float>(a), 16384.0f, fmaf(static_cast<float>(b), 128.0f,
                                                    static_cast<float>(c)));
}

// A row holding NaN or +-inf against group-scaled weights: sum over blocks
// of s_g * sum_j (code_j - z_g) x_j in f32, as the digit-dot kernels form it
// for such blocks (the reference's result class).
__device__ __forceinline__ float planes_row_f32_grouped(const int8_t* w, const float* scale,
                                                     const float* zp, long long n, int groups,
                                                     int gsize, const void* x, int xtype,
                                                     long long xr, int k) {
  float acc = 0.0f;
  for (int b = 0; b < k; b += 32) {
    const long long si = n * groups + b / gsize;
    const float z = zp != nullptr ? zp[si] : 0.0f;
    acc += scale[si] * cint8_block_f32(w + n * k + b, x, xr + b, xtype, z);
  }
  return acc;
}

// Operand B of the SwiGLU form: 32-row blocks alternate between gate (even
// blocks) and up (odd blocks), blocks 2c and 2c + 1 covering rows 32c..32c+31
// of both matrices (rows past the last clamped to it).
struct PairedRows {
  const int8_t* gate;
  const int8_t* up;
  long long rows, k;
  __device__ const int8_t* operator()(long long r) const {
    const long long blk = r >> 5;
    long long n = (blk >> 1) * 32 + (r & 31);
    n = n < rows ? n : rows - 1;
    // a bitwise select: a conditional between the two pointers is compiled
    // as an indexed load from a two-entry array in private memory
    const uint64_t g = reinterpret_cast<uintptr_t>(gate), u = reinterpret_cast<uintptr_t>(up);
    const uint64_t base = g ^ ((g ^ u) & (0 - static_cast<uint64_t>(blk & 1)));
    return reinterpret_cast<const int8_t*>(base) + n * k;
  }
};

// a if !second, else b, as a bitwise select (a lane-varying conditional
// between two pointers becomes an indexed load from private memory)
template <class T>
__device__ __forceinline__ const T* pick(const T* a, const T* b, bool second) {
  const uint64_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return reinterpret_cast<const T*>(x ^ ((x ^ y) & (0 - static_cast<uint64_t>(second))));
}

// The grouped fold's side data (an Int8Ring side policy): per K step, for
// each of its GPS groups u (one, or two for groups of 32 columns in 64-column
// steps), the scale and zero point (lanes 2r, 2r + 1; the scale again when
// there are no zero points) of row r of each 32-row block of the tile's B
// rows (slots u T + 0..TS-1), then the digit sums S_0..S_2 of 16 activation
// rows per slot (lanes 4r + t, t < 3; lane 4r + 3 repeats S_2), so that a
// row's values are one 8- or 16-byte LDS read.  Slots past those repeat the
// first scale.  Each wave issues kLoads slots; read() keeps, at a group's
// last step (ready), what the wave's fragments need.
template <int TN, int TM, int WGN, int WGM, bool SWIGLU, int KL, int GPS>
struct GroupSide {
  static constexpr int NW = WGN * WGM;
  static constexpr int FN = TN / WGN / 32, FM = TM / WGM / 32;
  static constexpr int TS = TM / 32, TD = (TN / 4 + 15) / 16, T = TS + TD;
  static constexpr int kLoads = (GPS * T + NW - 1) / NW;
  const int8_t* src[kLoads];   // this lane's address for group 0
  int stride[kLoads];          // bytes per group (wave-uniform)
  int gofs[kLoads];            // the slot's group within its step (GPS > 1)
  int spg, rleft, wn, wm;
  bool ready;
  float sc[GPS][FM], zr[GPS][FM];
  int sx[GPS][FN][4][3];

  __device__ void init(const PlaneOut& o, const int* dsum, int mc, int tn, int tm, int wave,
                       int wn_, int wm_) {
    const int lane = threadIdx.x & 63;
    spg = GPS == 1 ? o.gsize / KL : 1;
    rleft = spg;
    ready = false;
    wn = wn_;
    wm = wm_;
#pragma unroll
    for (int q = 0; q < kLoads; ++q) {
      const int slot = wave * kLoads + q;       // wave-uniform
      const int t = slot % T;
      gofs[q] = slot / T;
      if (slot >= GPS * T) {
        src[q] = reinterpret_cast<const int8_t*>(o.scale);
        stride[q] = 0;
        gofs[q] = 0;
      } else if (t < TS) {
        const long long c = static_cast<long long>(tm) * (TM / 32) + t;   // B block
        const bool second = SWIGLU && (c & 1);
        long long n = (SWIGLU ? (c >> 1) * 32 : c * 32) + (lane >> 1);
        n = n < o.rows ? n : o.rows - 1;
        const float* scale = second ? o.scale2 : o.scale;
        const float* zero = second ? o.zero2 : o.zero;
        zero = zero != nullptr ? zero : scale;
        src[q] = reinterpret_cast<const int8_t*>(pick(scale, zero, lane & 1) + n * o.groups);
        stride[q] = 4;
      } else {
        int r = tn * (TN / 4) + 16 * (t - TS) + (lane >> 2);
        r = r < mc ? r : mc - 1;
        const int comp = (lane & 3) < 3 ? (lane & 3) : 2;
        src[q] = reinterpret_cast<const int8_t*>(dsum + static_cast<long long>(r) * o.groups * 3 +
                                                 comp);
        stride[q] = 12;
      }
    }
  }
  __device__ void issue(int step, int wave, int8_t* base) const {
#pragma unroll
    for (int q = 0; q < kLoads; ++q) {
      const int grp = GPS == 1 ? step / spg : step * GPS + gofs[q];
      load_lds4(src[q] + grp * stride[q], base + (wave * kLoads + q) * 256);
    }
  }
  __device__ void read(int, const int8_t* base) {
    if constexpr (GPS == 1) {
      ready = --rleft == 0;
      if (!ready) return;
      rleft = spg;
    } else {
      ready = true;
    }
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < GPS; ++u) {
      const int8_t* b = base + u * T * 256;
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int bj = wm / 32 + j;
        const float2 sz = reinterpret_cast<const float2*>(b)[bj * 32 + (lane & 31)];
        sc[u][j] = sz.x;
        zr[u][j] = sz.y;
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int row = wn / 4 + 8 * i + 2 * g + (lane >> 5);
          const int4 v = reinterpret_cast<const int4*>(b)[(TS + row / 16) * 16 + row % 16];
          sx[u][i][g][0] = v.x;
          sx[u][i][g][1] = v.y;
          sx[u][i][g][2] = v.z;
        }
    }
  }
};

// The fused form: planes [4 mc][k] (operand A, TN rows per tile) against the
// weight codes (operand B, TM rows per tile), then for each (activation row,
// weight row n) the combination and the shared epilogue, stored as
// y[(m0 + r) * ld + n].  Lanes 0-31 of a store hold 32 consecutive n.  With
// SWIGLU the B tiles pair gate and up blocks (PairedRows): in a wave tile of
// 64 B rows (FM even), fragments j and j + 1 hold gate and up of the same n.
// GROUPED (gsize a multiple of the KL-column K step -- 64-column half-line
// steps for groups of 64, else 128-column steps -- or, GPS = 2, groups of 32
// in 64-column steps, folded after each 32-column quarter): at the end of each
// group's last step the int32 plane sums of the group are folded into f32,
// s_g * (2^14 A0 + 2^7 A1 + A2) with A_t = D_t - z_g S_t exact for an
// integral zero point (else 2^14 D0 + ... - z_g (2^14 S0 + ...) in f32),
// and cleared; the output is the sum over groups times 2^e.  With digits of
// at most 128 in magnitude and int8 codes, |D_t| <= 2^14 gsize and
// |z S_t| <= 2^7 gsize |z|: A_t is formed in int32 (a 24-bit multiply) when
// |z| <= zlim keeps both within int32 (every integral zero point for groups
// of 128), else in int64 on a branch the wave takes only when one of its
// lanes needs it; each A_t is then rounded to f32 once, so the two forms give
// the same bits.
// The GEMM's per-quarter hook for the ring, with the ring's fresh-sum period.
template <int FRESH, class F>
struct FoldStep {
  static constexpr int kFresh = FRESH;
  F f;
  template <class Acc>
  __device__ void operator()(int k, int q, Acc& a) const {
    f(k, q, a);
  }
};

template <int TN, int TM, int S, int WGN, int WGM, bool SWIGLU, bool GROUPED, int KL, int GPS,
          bool SPAN>
__global__ __launch_bounds__(64 * WGN * WGM) void cint8_planes_gemm(
    const int8_t* __restrict__ planes, int mc, const PlaneOut o, const int* __restrict__ rexp,
    const int* __restrict__ dsum, const void* __restrict__ x, int xtype, long long ldx, int m0,
    int k, int tiles_n, int tiles_m) {
  // Tiles of up to 128 plane rows serve up to 32 activation rows, all in one A
  // tile: each weight row is then read by one workgroup (non-temporal loads;
  // K=4096, N=14336: M=2 17.3 -> 15.7 us, M=8 18.3 -> 17.2, SwiGLU M=16 32.6 ->
  // 29.6; with two or more A tiles, M=512, the hint cost 1.5%).
  using R = Int8Ring<TN, TM, S, WGN, WGM, KL, (TN <= 128)>;
  using Side =
      std::conditional_t<GROUPED, GroupSide<TN, TM, WGN, WGM, SWIGLU, KL, GPS>, Int8NoSide>;
  static_assert(!SWIGLU || R::FM % 2 == 0, "gate / up fragment pairs");
  __shared__ __attribute__((aligned(1024))) int8_t ring[R::template kBytesWith<Side>];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tn, tm;
  tile_of(blockIdx.x, tiles_n * tiles_m, tiles_n, tiles_m, tn, tm);
  const long long p0 = static_cast<long long>(tn) * TN + R::wave_n(wave);   // plane rows
  const long long b0 = static_cast<long long>(tm) * TM + R::wave_m(wave);   // B rows
  v16i acc[R::FN][R::FM];
  // output row n of fragment j (SwiGLU: the pair's n, for gate j even and up j odd)
  auto out_row = [&](int j) -> long long {
    return (SWIGLU ? b0 / 2 + 16 * (j & ~1) : b0 + 32 * j) + (lane & 31);
  };
  // activation row (chunk-relative) of fragment row group (i, g)
  auto act_row = [&](int i, int g) -> int {
    return static_cast<int>((p0 + 32 * i + 8 * g + 4 * (lane >> 5)) >> 2);
  };
  float facc[GROUPED ? R::FN : 1][GROUPED ? R::FM : 1][4];
#pragma unroll
  for (int i = 0; i < (GROUPED ? R::FN : 1); ++i)
#pragma unroll
    for (int j = 0; j < (GROUPED ? R::FM : 1); ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) facc[i][j][g] = 0.0f;
  // GROUPED: the scales, zero points and digit sums of each group arrive with
  // the operand tiles of the group's last step (GroupSide)
  Side side;
  if constexpr (GROUPED)
    side.init(o, dsum, mc, tn, tm, wave, R::wave_n(wave), R::wave_m(wave));
  const long long gs = o.gsize;
  const int zlim = GROUPED ? static_cast<int>(((1LL << 31) - 1 - (gs << 14)) / (gs << 7)) : 0;
  // (SwiGLU: gate and up both have zero points or neither)
  const bool has_zero = o.zero != nullptr;
  // Groups that lie within one K step (GPS per step) end at fixed quarters:
  // the ring starts each group's sums from zero.  A group spanning several
  // steps (SPAN: 256 columns and more) carries its sums over steps, and the
  // fold clears them.
  static_assert(!SPAN || (GROUPED && KL == 128 && GPS == 1), "multi-step groups");
  constexpr int FRESH = GROUPED && !SPAN ? R::QPS / GPS : 0;
  auto fold = [&](int, int q, v16i (&a)[R::FN][R::FM]) {
    if constexpr (GROUPED) {
      // a group's last quarter (q is a constant in the unrolled quarter loops)
      constexpr int QPG = R::QPS / GPS;
      if ((q + 1) % QPG != 0) return;
      const int u = (q + 1) / QPG - 1;
      if (!side.ready) return;                  // uniform: not the group's last step
      if (!has_zero) {                          // uniform: s_g (2^14 D0 + 2^7 D1 + D2)
#pragma unroll
        for (int j = 0; j < R::FM; ++j) {
          const float sg = side.sc[u][j];
#pragma unroll
          for (int i = 0; i < R::FN; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g)
              facc[i][j][g] = fmaf(sg, combine(a[i][j][4 * g], a[i][j][4 * g + 1],
                                               a[i][j][4 * g + 2]),
                                   facc[i][j][g]);
          if constexpr (FRESH == 0) {
#pragma unroll
            for (int i = 0; i < R::FN; ++i)
#pragma unroll
              for (int e = 0; e < 16; ++e)
                if ((e & 3) != 3) a[i][j][e] = 0;
          }
        }
        return;
      }
#pragma unroll
      for (int j = 0; j < R::FM; ++j) {
        // zi: the integral zero point the int32 form subtracts (0 for none,
        // a fractional one or one beyond zlim); zf: the zero point the f32
        // form subtracts (0 for none or an integral one within zlim)
        const float sg = side.sc[u][j];
        const float z = has_zero ? side.zr[u][j] : 0.0f;
        int zr = 0;
        const bool integral = integral_zero(z, zr);
        const bool narrow = integral && zr >= -zlim && zr <= zlim;
        const bool wide = integral && !narrow;
        const int zi = narrow ? zr : 0;
        const float zf = narrow ? 0.0f : z;
        float fv[R::FN][4];
#pragma unroll
        for (int i = 0; i < R::FN; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int* sx = side.sx[u][i][g];  // (zi = 0 without zero points)
            fv[i][g] = combine(a[i][j][4 * g] + __mul24(-zi, sx[0]),
                               a[i][j][4 * g + 1] + __mul24(-zi, sx[1]),
                               a[i][j][4 * g + 2] + __mul24(-zi, sx[2]));
          }
        if (has_zero) {
          if (__any(zf != 0.0f)) {              // fractional (or wide) zero points: f32 form
#pragma unroll
            for (int i = 0; i < R::FN; ++i)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const int* sx = side.sx[u][i][g];
                fv[i][g] = fmaf(-zf, combine(sx[0], sx[1], sx[2]), fv[i][g]);
              }
          }
          if (__any(wide)) {                    // integral beyond zlim: exact in int64
#pragma unroll
            for (int i = 0; i < R::FN; ++i)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const int* sx = side.sx[u][i][g];
                const long long d0 = a[i][j][4 * g], d1 = a[i][j][4 * g + 1];
                const long long d2 = a[i][j][4 * g + 2];
                if (wide)
                  fv[i][g] = combine_f(d0 - zr * static_cast<long long>(sx[0]),
                                       d1 - zr * static_cast<long long>(sx[1]),
                                       d2 - zr * static_cast<long long>(sx[2]));
              }
          }
        }
#pragma unroll
        for (int i = 0; i < R::FN; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g) facc[i][j][g] = fmaf(sg, fv[i][g], facc[i][j][g]);
        // the next group's sums start from zero: its first MFMAs take a zero
        // accumulator (FRESH), or the sums are cleared here (plane row 3 of
        // every activation row is zero: its sums stay 0)
        if constexpr (FRESH == 0) {
#pragma unroll
          for (int i = 0; i < R::FN; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e)
              if ((e & 3) != 3) a[i][j][e] = 0;
        }
      }
    }
  };
  const FoldStep<FRESH, decltype(fold)> step{fold};
  if constexpr (SWIGLU)
    R::run_rows(planes, PairedRows{o.w, o.w2, o.rows, k}, 4 * mc, k,
                static_cast<long long>(tn) * TN, static_cast<long long>(tm) * TM, ring, acc, step,
                &side);
  else
    R::run_rows(planes, Int8Rows{o.w, o.rows, k}, 4 * mc, k, static_cast<long long>(tn) * TN,
                static_cast<long long>(tm) * TM, ring, acc, step, &side);
  // projection of activation row r on the row of fragment j
  auto value = [&](int i, int j, int g, int r, long long n) -> float {
    const bool second = SWIGLU && (j & 1);
    const int8_t* const w = second ? o.w2 : o.w;
    const float* const scale = second ? o.scale2 : o.scale;
    const float* const zp = second ? o.zero2 : o.zero;
    if constexpr (GROUPED) {
      const int e = rexp[r];
      if (e == kPlanesNonfinite)
        return planes_row_f32_grouped(w, scale, zp, n, o.groups, o.gsize, x, xtype,
                                      static_cast<long long>(m0 + r) * ldx, k);
      return ldexpf(facc[i][j][g], e);
    } else {
      return plane_value(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], w, scale,
                         zp, n, r, m0, rexp, dsum, x, xtype, ldx, k);
    }
  };
  constexpr int JS = SWIGLU ? 2 : 1;
#pragma unroll
  for (int j = 0; j < R::FM; j += JS) {
    const long long n = out_row(j);
    if (n >= o.rows) continue;
#pragma unroll
    for (int i = 0; i < R::FN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r = act_row(i, g);
        if (r >= mc) continue;
        float v = value(i, j, g, r, n);
        if constexpr (SWIGLU) {
          const float up = value(i, j + 1, g, r, n);
          v = (v / (1.0f + expf(-v))) * up;
        } else if (o.epi) {
          if (o.bias != nullptr) v += o.bias[n];
          v = linear_activation(v, o.act);
        }
        store_y(o.y, static_cast<long long>(m0 + r) * o.ld + n, o.ytype, v);
      }
  }
}

template <int TN, int TM, int S, int WGN, int WGM, bool SWIGLU, bool GROUPED, int KL, int GPS,
          bool SPAN>
hipError_t launch_planes_gemm(const int8_t* planes, int mc, const PlaneOut& o, const int* rexp,
                              const int* dsum, const void* x, int xtype, long long ldx, int m0,
                              int k, hipStream_t s) {
  const int tiles_n = (4 * mc + TN - 1) / TN;
  // SwiGLU: 64 B rows per 32 output rows
  const long long brows = SWIGLU ? 64LL * ((o.rows + 31) / 32) : o.rows;
  const int tiles_m = static_cast<int>((brows + TM - 1) / TM);
  cint8_planes_gemm<TN, TM, S, WGN, WGM, SWIGLU, GROUPED, KL, GPS, SPAN>
      <<<tiles_n * tiles_m, 64 * WGN * WGM, 0, s>>>(planes, mc, o, rexp, dsum, x, xtype, ldx, m0,
                                                    k, tiles_n, tiles_m);
  return hipGetLastError();
}

// Tile by plane rows: up to 64 activation rows the whole plane matrix in one
// A tile and 64 output rows per workgroup (224 workgroups at N = 14336): 64
// weight rows, or 64 gate and 64 up rows in wave tiles of 64 B rows; up to
// 128 rows two A tiles of 256 by 128 B rows (224 workgroups at N = 14336, where
// 448 of 256 x 64 took 1.4x as long); above, the W8A8 kernel's 256 x 256 tile.
// KL = 64 (groups of 64 or 32 columns: one or two groups per half-line K
// step): the same tiles with about twice the stages (half the bytes each),
// within the 6-bit vmcnt and the 160 KB of LDS; GPS = 2 carries twice the
// side loads.
template <bool SWIGLU, bool GROUPED, int KL, int GPS = 1, bool SPAN = false>
hipError_t launch_fused(const int8_t* planes, int mc, const PlaneOut& o, const int* rexp,
                        const int* dsum, const void* x, int xtype, long long ldx, int m0, int k,
                        hipStream_t s) {
  static_assert(KL == 128 || GROUPED, "half-line steps only for small groups");
  static_assert(GPS == 1 || KL == 64, "two groups per step: groups of 32");
  constexpr int TM = SWIGLU ? 128 : 64;
  constexpr bool H = KL == 64, T2 = GPS == 2;
#define QC_PLANES(TN_, TM_, S_, WGN_, WGM_, SW_)                                     \
  launch_planes_gemm<TN_, TM_, S_, WGN_, WGM_, SW_, GROUPED, KL, GPS, SPAN>(              \
      planes, mc, o, rexp, dsum, x, xtype, ldx, m0, k, s)
  // (grouped SwiGLU: 5 stages, as its side loads would take 6 past the vmcnt range)
  if (mc <= 8)
    return QC_PLANES(32, TM,
                     H ? (SWIGLU ? (T2 ? 7 : 8) : (T2 ? 10 : 12))
                       : SWIGLU ? (GROUPED ? 5 : 6) : 8,
                     1, 2, SWIGLU);
  // From 9 rows, wave tiles of 32 plane rows (more waves per tile, so each
  // holds a quarter or half of the fragments and of the grouped fold's work):
  // K=4096, N=14336, M=16: row scales 23.8 -> 22.6 us, groups of 128 32.3 ->
  // 27.8, of 64 46.7 -> 37.3; M=32: 27.5 -> 26.8 / 33.0 -> 31.7; M=64: 35.5 ->
  // 33.4 / 49.9 -> 45.1.  64-column steps: 8 waves over a B tile of 64 rows
  // (four 1 KB blocks, loaded by waves 0..3) from 33 rows, and for groups of
  // 32 or SwiGLU from 17: groups of 64 at M=48 / 64 75.2 / 75.0 -> 67.8 / 66.8
  // us, groups of 32 at M=24 / 32 / 48 / 64 68.2 / 68.8 / 116 / 117 -> 54.0 /
  // 54.7 / 90.1 / 91.2, SwiGLU M=32 73.6 -> 64.5 (groups of 64) and 117 ->
  // 92.6 (32); groups of 64 at 17-32 rows were 2.6 us slower that way.  (SwiGLU
  // at 33-64 rows gained nothing from 8 waves.)
  if (mc <= 16)
    return QC_PLANES(64, TM, H ? (SWIGLU ? (T2 ? 6 : 8) : 10) : SWIGLU ? 4 : 6, 2, 2, SWIGLU);
  if (mc <= 32) {
    if constexpr (H) return QC_PLANES(128, TM, 8, (T2 || SWIGLU) ? 4 : 2, 2, SWIGLU);
    else return QC_PLANES(128, TM, 4, 4, 2, SWIGLU);
  }
  if (mc <= 64) {
    if constexpr (SWIGLU) return QC_PLANES(256, TM, H ? (T2 ? 5 : 6) : 3, 4, 2, true);
    else if constexpr (H) return QC_PLANES(256, TM, 6, 8, 1, false);
    else return QC_PLANES(256, TM, 3, 8, 1, false);
  }
  // group sums in registers beside 256 x 256 tiles would spill: 256 x 128 above 64 rows
  if constexpr (GROUPED) {
    return QC_PLANES(256, 128, H ? (T2 ? 5 : 6) : 3, 4, 2, SWIGLU);
  } else {
    if (mc <= 128) return QC_PLANES(256, 128, 3, 4, 2, SWIGLU);
    return QC_PLANES(256, 256, 2, 4, 2, SWIGLU);
  }
#undef QC_PLANES
}

// Groups of 64 columns take half-line K steps (one group per step), groups of
// 32 the same steps with a fold after each quarter (two groups per step).
template <bool SWIGLU, bool GROUPED>
hipError_t launch_fused_kl(const int8_t* planes, int mc, const PlaneOut& o, const int* rexp,
                           const int* dsum, const void* x, int xtype, long long ldx, int m0,
                           int k, hipStream_t s) {
  if constexpr (GROUPED) {
    if (o.gsize == 64)
      return launch_fused<SWIGLU, true, 64>(planes, mc, o, rexp, dsum, x, xtype, ldx, m0, k, s);
    if (o.gsize == 32)
      return launch_fused<SWIGLU, true, 64, 2>(planes, mc, o, rexp, dsum, x, xtype, ldx, m0, k,
                                               s);
  }
  if (GROUPED && o.gsize > 128)   // groups of several 128-column steps
    return launch_fused<SWIGLU, GROUPED, 128, 1, GROUPED>(planes, mc, o, rexp, dsum, x, xtype, ldx,
                                                          m0, k, s);
  return launch_fused<SWIGLU, GROUPED, 128>(planes, mc, o, rexp, dsum, x, xtype, ldx, m0, k, s);
}

size_t up256(size_t b) { return (b + 255) / 256 * 256; }

// All checks done by the caller, which routes only 16-byte aligned codes here
// and, with groups, k % 128 == 0 and group sizes of 32, 64 or a multiple of
// 128 columns.
template <bool GROUPED>
hipError_t launch_planes(const CSegs& sg, const CInt8Launch& L, int m, int k, hipStream_t s) {
  const int nmat = L.mode == 1 ? 2 : L.nw;
  const size_t es = L.xtype == QC_STORAGE_F32 ? 4 : 2;
  const bool vec = L.xtype == QC_STORAGE_F32 && reinterpret_cast<uintptr_t>(L.x) % 16 == 0 &&
                   L.ldx % 4 == 0;
  const int ngroups = GROUPED ? sg.groups : 1;
  const int gsize = GROUPED ? sg.gsize : k;
  // the digit sums only enter the zero-point terms
  bool sums = false;
  for (int i = 0; i < nmat; ++i) sums = sums || sg.zero[i] != nullptr;
  // chunks of kPlanesChunkM rows, one after the other in one buffer
  const int mc0 = std::min(kPlanesChunkM, m);
  const size_t bytes = up256(4ull * mc0 * k) + up256(4ull * mc0) + up256(12ull * mc0 * ngroups);
  std::unique_lock<std::mutex> hold;
  uint8_t* base = nullptr;
  hipError_t e = call_scratch(s, bytes, hold, reinterpret_cast<void**>(&base));
  if (e != hipSuccess) return e;
  for (int m0 = 0; m0 < m && e == hipSuccess; m0 += kPlanesChunkM) {
    const int mc = std::min(kPlanesChunkM, m - m0);
    int8_t* planes = reinterpret_cast<int8_t*>(base);
    int* rexp = reinterpret_cast<int*>(base + up256(4ull * mc * k));
    int* dsum = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(rexp) + up256(4ull * mc));
    const void* xc = static_cast<const uint8_t*>(L.x) + es * static_cast<size_t>(m0) * L.ldx;
    cint8_planes_prep<GROUPED><<<mc, kPrepThreads, 0, s>>>(xc, L.xtype, L.ldx, k, vec, gsize,
                                                           ngroups, sums, planes, rexp, dsum);
    e = hipGetLastError();
    if (e == hipSuccess && L.mode == 1) {
      const PlaneOut o{sg.w[0], sg.scale[0], sg.zero[0], sg.w[1], sg.scale[1], sg.zero[1],
                       sg.y[0], sg.ld[0], sg.ytype[0], static_cast<int>(L.w[0].rows),
                       nullptr, 0, 0, ngroups, gsize};
      e = launch_fused_kl<true, GROUPED>(planes, mc, o, rexp, dsum, L.x, L.xtype, L.ldx, m0, k,
                                         s);
      continue;
    }
    for (int i = 0; i < nmat && e == hipSuccess; ++i) {
      const PlaneOut o{sg.w[i], sg.scale[i], sg.zero[i], nullptr, nullptr, nullptr, sg.y[i],
                       sg.ld[i], sg.ytype[i], static_cast<int>(L.w[i].rows), sg.bias, sg.act,
                       i == 0 && (sg.bias != nullptr || sg.act != 0) ? 1 : 0, ngroups, gsize};
      e = launch_fused_kl<false, GROUPED>(planes, mc, o, rexp, dsum, L.x, L.xtype, L.ldx, m0, k,
                                          s);
    }
  }
  return e;
}

}  // namespace

hipError_t launch_cint8_planes(const CSegs& sg, const CInt8Launch& L, int m, int k, bool grouped,
                               hipStream_t s) {
  return grouped ? launch_planes<true>(sg, L, m, k, s) : launch_planes<false>(sg, L, m, k, s);
}

}  // namespace qc
