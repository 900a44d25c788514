// Small-batch q8_0 / q4_0 GEMM (2 <= M, in tiles of 16 activation rows) on
// gfx950 MFMA: int8 digit planes for up to 8 rows per pass, f16 (q8_0) or
// bf16 (q4_0) operands above, and a 2-D tiled kernel for M >= 64.
//
// Semantics as the reference's qgemm (kernels/quantization/qgemm_ref.cpp:
// 156-162, one qgemv per activation row: y[m][n] = sum_b d[n][b] *
// sum_{k in b} q[n][k] * x[m][k]); the f32 outputs are held to the contract
// bound |y - y_exact| <= 1e-4 * ||x_m|| * ||w_n|| like the M = 1 path.
//
// Numerics of the f16 / bf16 layouts.  Each activation (scaled per row by a
// power of two) is split into two values, hi and lo = the rounding of
// x - hi, so x - hi - lo is within 2^-17 |x| (bf16) or 2^-22 |x| (f16); the
// q8_0 codes (|q| <= 128, in f16) and the q4_0 nibbles (0..15, in bf16) are
// exact.  One v_mfma_f32_16x16x32_{f16,bf16} covers exactly one 32-element
// block, so the block dot sum_k q*hi + sum_k q*lo comes out of two MFMAs with
// f32 accumulation and is then scaled by the block's fp16 d with one FMA per
// output.  For q4_0 the -8 offset enters through the MFMA's C input: the
// block starts from bias = -8 * sum_k (hi + lo), precomputed per activation
// row and block.  Worst-case error, normalised by ||x_m|| * ||w_n||: the
// split, about 32 * 2^-24 * 15/8 * sqrt(32) ~ 2e-5 from the f32 accumulation
// of the q4 block sums, plus 2^-24 per block for the scaled accumulation --
// well inside 1e-4.
//
// Data flow.  A prep kernel (qgemm_prep for the digit layouts, prep_rows
// for f16 / bf16) writes the activation fragments in the MFMA operand layout
// ([block][m-tile][hi | lo][64 lanes][16 B]) plus the q4 bias, and zeroes y
// when two K halves will add into it; for the digit layouts the GEMM usually
// builds them itself instead (FOLD, below).  The GEMM workgroup (4 or
// 8 wavefronts, 16 weight rows each) runs a ring of LDS stages, each
// holding 4 block pairs (256 K) of its weight rows -- whole row segments,
// copied with global_load_lds_dwordx4, so every weight byte crosses the
// memory system once in full cache lines -- and the activation fragments of
// those blocks, which all its wavefronts share.  Each lane then picks its
// codes and scales out of LDS.  The ring is 3 stages deep where LDS allows
// (2 for q8_0 with 32 activation rows).
//
// K is split over `ks` workgroups per row slab when N alone gives too
// few workgroups.  With ks = 2 both halves add atomically into a y that the
// prep kernel zeroed (two addends onto zero: order-independent); with
// ks > 2 the partial sums go to a workspace and a small kernel adds them in
// index order.  Results are deterministic either way.  Having the slab's
// last workgroup add the partial sums instead (a per-slab counter behind a
// device-scope fence) measured slower than the extra launch: +2.4 to +17 us
// at N=4096, M=8..32; with agent-scope write-through stores and loads and no
// L2 writeback, equal at M=8 and +2 to +10 us at M=16 / 32.
#include <algorithm>
#include <memory>
#include <mutex>
#include <type_traits>
#include <vector>

#include "qc_device.h"
#include "qc_internal.h"
#include "qc_lds_dma.h"

namespace qc {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kStagePairs = 4;           // block pairs per ring stage
constexpr int kStageBlocks = 2 * kStagePairs;

// Bytes of activation fragments per block and dense m-tile: hi and lo, 64
// lanes x 16 B.
constexpr int kFragBytes = 2048;

// Activation layout per 32-element block, by XL (rows per pass, M <= XL):
//  * XL = 16 / 32, bf16 mode (T = XL / 16 m-tiles): [m-tile][hi | lo][64
//    lanes][16 B], exactly the MFMA operand registers, plus (q4_0) a separate
//    bias array [block][m-tile][16 rows] of f32;
//  * XL = 4 / 8, digit mode (T = XL / 4 tiles of 4 rows): the int8 digit
//    planes of each row as v_mfma_i32_16x16x32_i8 A operands, [tile][64
//    lanes][8 B] with operand row 4 (m & 3) + d holding digit d of row m (d = 3
//    is zero); then per row {int32 e, f32 gate}; then (q4_0) per row the
//    int32 C input {-8 sum_k digit_d, d = 0..3}.  The digits of a row share
//    one exponent per stage of 8 blocks; every block record of the stage
//    holds it.
template <int XL, bool BIAS>
struct XBlock {
  static constexpr bool digits = XL <= 8;
  static constexpr int T = digits ? XL / 4 : XL / 16;   // operand tiles
  static constexpr int meta_off = digits ? T * 512 : 0;
  static constexpr int bias_off = meta_off + 8 * XL;
  static constexpr int bytes = digits ? bias_off + (BIAS ? 16 * XL : 0) : T * kFragBytes;
  static constexpr int bias_bytes = digits || !BIAS ? 0 : T * 64;    // separate array
  static constexpr int prep_groups = digits ? 1 : T;                 // prep workgroups per block
  static constexpr int stage_bytes = kStageBlocks * bytes;           // x bytes of a ring stage
  static_assert(bytes % 16 == 0, "whole 16-byte chunks");
};

template <int FMT>
struct PairLayout;
// q8_0 pair (68 B): d0 @0, q0 @2..33, d1 @34, q1 @36..67.  Lane group j
// (lane >> 4) needs codes 8j..8j+7 of each block.
template <>
struct PairLayout<kQ8_0> {
  static constexpr int bytes = 68;
  __device__ static int blk0_dword(int j) { return 2 * j; }   // 3 dwords, bytes 2.. of them
  __device__ static int blk1_dword(int j) { return 9 + 2 * j; }
  static constexpr int scale1_dword = 8;                       // d1 in the high half
};
// q4_0 pair (36 B): d0 @0, nibbles @2..17, d1 @18, nibbles @20..35.  Byte i of
// a block holds code i (low nibble) and code i+16 (high nibble), so lane
// groups j and j+2 read the same 8 bytes.
template <>
struct PairLayout<kQ4_0> {
  static constexpr int bytes = 36;
  __device__ static int blk0_dword(int j) { return 2 * (j & 1); }
  __device__ static int blk1_dword(int j) { return 5 + 2 * (j & 1); }
  static constexpr int scale1_dword = 4;
};

typedef uint32_t u32x3_a4 __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

// MFMA operand type of the bf16-layout routes: q8_0 runs in f16 (codes and
// hi/lo activations), q4_0 in bf16.
template <int FMT>
struct OpType {
  using T = bf16x8;
};
template <>
struct OpType<kQ8_0> {
  using T = f16x8;
};

__device__ __forceinline__ f32x4 mfma_op(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_op(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Eight codes of this lane for one block as an MFMA operand (lo: codes 0..3,
// hi: codes 4..7 of the lane's eight bytes).
template <int FMT>
__device__ __forceinline__ typename OpType<FMT>::T codes_op(uint32_t lo, uint32_t hi, int j) {
  if constexpr (FMT == kQ8_0) {
    // Code byte q flipped to q + 128 (0..255) under the high byte 0x64 of
    // f16(1024) is f16(1024 + q + 128), exactly; one packed f16 subtraction
    // of 1152 leaves q.  v_perm_b32 interleaves two code bytes with 0x64.
    const uint32_t a = lo ^ 0x80808080u, b = hi ^ 0x80808080u;
    const f16x2 k = f16x2{static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    const f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u)) - k;
    const f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u)) - k;
    const f16x2 p2 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u)) - k;
    const f16x2 p3 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u)) - k;
    return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  } else {
    const int sh = (j >> 1) * 4;          // lane groups 2, 3 take the high nibbles
    const uint32_t a = (lo >> sh) & 0x0F0F0F0Fu, b = (hi >> sh) & 0x0F0F0F0Fu;
    // A nibble byte u (0..15) is the OCP e4m3 encoding of u * 2^-9
    // (subnormal below 8, exponent field 1 from 8), so the scaled fp8
    // conversion gives bf16(u) exactly, two bytes per instruction (low word:
    // bytes 0, 1; high word: bytes 2, 3).
    const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(a, 512.0f, false);
    const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(a, 512.0f, true);
    const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(b, 512.0f, false);
    const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(b, 512.0f, true);
    return bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  }
}

// Waits until at most G * min(D, ahead) loads are outstanding (`ahead` is a
// constant once the stage loop is unrolled).
template <int G, int D>
__device__ __forceinline__ void wait_stages(int ahead) {
  if constexpr (D <= 0) {
    wait_vmcnt<0>();
  } else {
    if (ahead >= D) wait_vmcnt<G * D>();
    else wait_stages<G, D - 1>(ahead);
  }
}
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}
// Barrier that neither drains outstanding global->LDS loads (the waits are
// explicit) nor lets the compiler move memory accesses across it.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}


// Activation fragments of the bf16 / f16 layouts (q4_0 / q8_0), 2 KB per
// (16-row m-tile, block): lane l holds row 16t + (l & 15), elements
// 8(l >> 4) .. +7 of the block as hi (bytes 0..1023) and lo = the rounding
// of v - hi (bytes 1024..2047), and (q4_0) the bias -8 * sum(hi + lo) per
// row and block, the MFMA's C input for the nibble offset.  Small-batch
// passes store fragment (b, t) at b * T + t over nbp blocks (those past K
// zero), the panel route at t * nb + b.
//
// Per-row power-of-two scale: the fragments hold v = x * 2^-e(m), with e(m)
// from the frexp exponent of max |x[m][:]| (0 for a zero or non-finite row)
// so that the row's largest element is in [0.5, 1) (bf16) or [2^14, 2^15)
// (f16): no element that matters is subnormal in the operand type (which
// would leave it a few bits) and no product overflows; rexp[m] = e(m), and
// outputs are scaled back by 2^e(m), exactly.  A row holding NaN or +-inf
// gets rexp[m] = kRowNonfinite instead, and the GEMMs recompute its outputs
// in the reference's f32 form (nonfinite_blocks_f32).
//
// One 256-thread workgroup per row of the layout (rows past M are zero): the
// row's maximum, then its fragments, in one launch; workgroups `rows` and up
// only clear y (zero_count floats), beside the row work rather than after it.  Thread t converts the
// half blocks h = t + 256 i; the two halves of a block sit in lanes t, t ^ 1,
// and the bias sum keeps the order ((s0 + s1) + (s2 + s3)) of the four
// 8-element chunk sums.  Workgroup 0 also copies the weights' short final
// stage into `tail_pad` (small-batch passes), and all of them clear y when
// two K ranges add into it.
constexpr int kRowNonfinite = 0x40000000;   // no exponent takes this value

// p[0..count) = 0 by `stride` threads, this one being thread `first`: 16-byte
// stores when p is 16-byte aligned.
__device__ __forceinline__ void clear_floats(float* p, long long count, long long first,
                                             long long stride) {
  long long done = 0;
  if (reinterpret_cast<uintptr_t>(p) % 16 == 0) {
    const long long n4 = count / 4;
    for (long long i = first; i < n4; i += stride)
      reinterpret_cast<float4*>(p)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    done = 4 * n4;
  }
  for (long long i = done + first; i < count; i += stride) p[i] = 0.0f;
}

// Workgroups of prep_rows that only clear y (about 16 floats per thread).
inline int clear_workgroups(long long count) {
  const long long w = (count + 256 * 16 - 1) / (256 * 16);
  return static_cast<int>(w < 512 ? w : 512);
}

template <bool PANEL, bool BIAS>
__global__ __launch_bounds__(256) void prep_rows(const float* __restrict__ x, int M, int K,
                                                 int nbo, int T, uint8_t* __restrict__ xf,
                                                 float* __restrict__ bias,
                                                 int* __restrict__ rexp, float* zero_y,
                                                 long long zero_count,
                                                 const uint8_t* __restrict__ tail_src, int tail,
                                                 uint8_t* __restrict__ tail_pad, int pad_bytes,
                                                 int rows) {
  if (static_cast<int>(blockIdx.x) >= rows) {
    clear_floats(zero_y, zero_count, static_cast<long long>(blockIdx.x - rows) * 256 + threadIdx.x,
                 static_cast<long long>(gridDim.x - rows) * 256);
    return;
  }
  __shared__ float smax[4];
  __shared__ int sbad[4];
  // Workgroups are dealt to the 8 XCDs in turn (id mod 8), and each 128-byte
  // line of a fragment holds 8 consecutive rows: give those rows to one XCD
  // (ids 8q + c of each group of 64 take rows 8c + q), so each line is
  // assembled in one L2 instead of being written back in pieces from eight.
  const int m = rows % 64 == 0
                    ? (blockIdx.x & ~63) | ((blockIdx.x & 7) << 3) | ((blockIdx.x >> 3) & 7)
                    : static_cast<int>(blockIdx.x);
  const int tid = threadIdx.x;
  const bool live = m < M;
  const int nb = K / 32;
  const float* xr = x + static_cast<long long>(live ? m : 0) * K;
  if (blockIdx.x == 0 && tail > 0)
    for (int i = tid; i < pad_bytes; i += 256) tail_pad[i] = i < tail ? tail_src[i] : 0;

  // max |x[m][:]|, four independent loads in flight per step; z stays 0
  // unless an element is NaN or +-inf (0 * x is then NaN)
  float mx = 0.f, z = 0.f;
  auto see = [&](float v) {
    mx = fmaxf(mx, fabsf(v));
    z = fmaf(0.0f, v, z);
  };
  auto see4 = [&](const float4& a) {
    see(a.x);
    see(a.y);
    see(a.z);
    see(a.w);
  };
  if (live) {
    int i = tid;
    if (reinterpret_cast<uintptr_t>(xr) % 16 == 0) {
      const float4* x4 = reinterpret_cast<const float4*>(xr);
      const int n4 = K / 4;
      for (; i + 768 < n4; i += 1024) {
        const float4 a = x4[i], b = x4[i + 256], c = x4[i + 512], d = x4[i + 768];
        see4(a);
        see4(b);
        see4(c);
        see4(d);
      }
      for (; i < n4; i += 256) see4(x4[i]);
    } else {
      for (; i + 768 < K; i += 1024) {
        const float a = xr[i], b = xr[i + 256], c = xr[i + 512], d = xr[i + 768];
        see(a);
        see(b);
        see(c);
        see(d);
      }
      for (; i < K; i += 256) see(xr[i]);
    }
  }
  mx = wave_max_nonneg(mx);
  const int wbad = __any(z != 0.0f) ? 1 : 0;
  if ((tid & 63) == 0) {
    smax[tid >> 6] = mx;
    sbad[tid >> 6] = wbad;
  }
  __syncthreads();
  mx = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
  const bool bad = (sbad[0] | sbad[1] | sbad[2] | sbad[3]) != 0;
  int e = 0;
  if (mx > 0.f && mx <= 3.402823466e38f) (void)frexpf(mx, &e);
  // q4_0 (bf16): largest element in [0.5, 1); q8_0 (f16): in [2^14, 2^15), so
  // that only elements below 2^-28 of the row's maximum reach f16 subnormals
  if constexpr (!BIAS) e -= 15;
  if (live && tid == 0) rexp[m] = bad ? kRowNonfinite : e;
  if (bad) e = 0;

  const int t = m >> 4, r = m & 15;
  const int nh = 2 * nbo;                          // half blocks of the layout's row
  for (int h0 = 0; h0 < nh; h0 += 256) {           // uniform trip count: the shuffle below
    const int h = h0 + tid;
    const int blk = h >> 1, half = h & 1;
    const bool in = live && blk < nb;
    float v[16];
    if (in) {
      const float* src = xr + 32 * blk + 16 * half;
      if (reinterpret_cast<uintptr_t>(xr) % 16 == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<float4*>(&v[4 * i]) = reinterpret_cast<const float4*>(src)[i];
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = src[i];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = ldexpf(v[i], -e);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = 0.0f;
    }
    float sc[2];
    const long long f = PANEL ? static_cast<long long>(t) * nbo + blk
                              : static_cast<long long>(blk) * T + t;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      using Op = std::conditional_t<BIAS, bf16x8, f16x8>;
      using El = std::conditional_t<BIAS, __bf16, _Float16>;
      Op hi, lo;
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        hi[i] = static_cast<El>(v[8 * c + i]);
        const float hv = static_cast<float>(hi[i]);
        lo[i] = static_cast<El>(v[8 * c + i] - hv);
        sum += hv + static_cast<float>(lo[i]);
      }
      sc[c] = sum;
      if (h < nh) {
        uint8_t* dst = xf + f * kFragBytes + 16 * (r + 16 * (2 * half + c));
        *reinterpret_cast<Op*>(dst) = hi;
        *reinterpret_cast<Op*>(dst + 1024) = lo;
      }
    }
    if constexpr (BIAS) {
      float sp = sc[0] + sc[1];
      sp += __shfl_xor(sp, 1);
      if (h < nh && half == 0) bias[f * 16 + r] = -8.0f * sp;
    }
  }
}

// The digits of activation row m over one stage of 8 blocks, built by one
// whole wavefront: lane l holds elements 4 (l & 7) .. +3 of block l >> 3
// (v, zero past K or M), and the records go to the stage's x area
// `stage_rec` (XBlock layout) when `write`.  The row shares one exponent
// over the stage: e = frexp exponent of max |x| over its 256 elements - 21,
// q = rint(x * 2^-e) clamped to [-2^21, 2^21), q = 2^14 d0 + 2^7 d1 + d2, so
// each element is held to within 2^-22 of the stage maximum.  A stage row
// with a non-finite value gets gate NaN and zero digits.
template <int XL, bool BIAS>
__device__ __forceinline__ void digit_stage_row(const float (&v)[4], int m, bool write,
                                                uint8_t* stage_rec) {
  using XB = XBlock<XL, BIAS>;
  const int lane = threadIdx.x & 63;
  const int part = lane & 7, b = lane >> 3;
  float mx = 0.f;
  int fin = 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mx = fmaxf(mx, fabsf(v[i]));
    fin &= isfinite(v[i]) ? 1 : 0;
  }
  mx = wave_max_nonneg(mx);                        // NaN lanes are caught by fin
  fin = __all(fin) ? 1 : 0;
  int ex = 0;
  (void)frexpf(mx, &ex);                           // mx < 2^ex
  const int e = fin ? ex - 21 : 0;
  uint32_t pk[3] = {0u, 0u, 0u};
  int sum[3] = {0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int q = fin ? __float2int_rn(ldexpf(v[i], -e)) : 0;   // |x * 2^-e| <= 2^21
    q = q > 2097151 ? 2097151 : q;
    const int dg[3] = {q >> 14, (q >> 7) & 127, q & 127};
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      pk[d] |= static_cast<uint32_t>(dg[d] & 0xFF) << (8 * i);
      sum[d] += dg[d];
    }
  }
  uint8_t* rec = stage_rec + b * XB::bytes;
  if (write) {
    // operand row r = 4 (m & 3) + d, k = 4 part + i: lane r + 16 (part >> 1),
    // bytes 4 (part & 1) .. +3 of its 8
    uint8_t* a = rec + (m >> 2) * 512 + 4 * (part & 1);
#pragma unroll
    for (int d = 0; d < 4; ++d)
      *reinterpret_cast<uint32_t*>(a + 8 * (4 * (m & 3) + d + 16 * (part >> 1))) = d < 3 ? pk[d] : 0u;
  }
  if constexpr (BIAS) {
#pragma unroll
    for (int d = 0; d < 3; ++d) sum[d] = group8_sum(sum[d]);
  }
  if (write && part == 0) {
    int* meta = reinterpret_cast<int*>(rec + XB::meta_off) + 2 * m;
    meta[0] = e;
    meta[1] = __float_as_int(fin ? 1.0f : __builtin_nanf(""));
    if constexpr (BIAS) {
      int* c = reinterpret_cast<int*>(rec + XB::bias_off) + 4 * m;
      c[0] = -8 * sum[0];
      c[1] = -8 * sum[1];
      c[2] = -8 * sum[2];
      c[3] = 0;
    }
  }
}

// Digit fragments of the compact layouts (M <= 8): one 64-thread workgroup
// per (stage, row), stage records of XBlock::stage_bytes.  Workgroup 0 also
// copies the weights' last row's short final stage (`tail` bytes from
// `tail_src`) into the zero-padded `tail_pad` (pad_bytes), which the GEMM
// reads instead of running past the end of W.
template <int XL, bool BIAS>
__global__ __launch_bounds__(64) void qgemm_prep(const float* __restrict__ x, int M, int K,
                                                 uint8_t* __restrict__ xf, float* zero_y,
                                                 long long zero_count,
                                                 const uint8_t* __restrict__ tail_src, int tail,
                                                 uint8_t* __restrict__ tail_pad, int pad_bytes) {
  if (blockIdx.x == 0 && tail > 0)
    for (int i = threadIdx.x; i < pad_bytes; i += 64) tail_pad[i] = i < tail ? tail_src[i] : 0;
  using XB = XBlock<XL, BIAS>;
  static_assert(XB::digits, "the bf16 layouts are built by prep_rows");
  const int l = threadIdx.x;
  const int nb = K / 32;
  {
    // lane l: elements 4 (l & 7) .. +3 of block 8 st + (l >> 3) of row m
    const int st = blockIdx.x / XL, m = blockIdx.x % XL;
    const int blk = kStageBlocks * st + (l >> 3);
    const bool live = m < M && blk < nb;
    const float* src = x + static_cast<long long>(live ? m : 0) * K + (live ? 32 * blk : 0) +
                       4 * (l & 7);
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = live ? src[i] : 0.0f;
    digit_stage_row<XL, BIAS>(v, m, true, xf + static_cast<long long>(st) * XB::stage_bytes);
  }
  // y is accumulated with two atomic adds when K is split in two: clear it.
  clear_floats(zero_y, zero_count, static_cast<long long>(blockIdx.x) * 64 + l,
               static_cast<long long>(gridDim.x) * 64);
}

// Sum of the ks partial results in index order (K split more than twice).
__global__ __launch_bounds__(256) void qgemm_reduce(const float* __restrict__ partial,
                                                    float* __restrict__ y, long long count,
                                                    int ks) {
  for (long long o = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; o < count;
       o += static_cast<long long>(gridDim.x) * 256) {
    // Four partial sums in flight at once (indices clamped to the last set,
    // so every load is in bounds), added in index order as before: with one
    // load per loop trip each was waited for before the next was issued.
    float sum = 0.0f;
    for (int q0 = 0; q0 < ks; q0 += 4) {
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[j] = partial[static_cast<long long>(min(q0 + j, ks - 1)) * count + o];
      sum = q0 == 0 ? v[0] : sum + v[0];
#pragma unroll
      for (int j = 1; j < 4; ++j)
        if (q0 + j < ks) sum += v[j];
    }
    y[o] = sum;
  }
}

// Weight rows of one ring stage (4 block pairs): whole 16-byte chunks, so a
// wavefront's 16 rows are copied to LDS with global_load_lds_dwordx4 as
// contiguous row segments (every byte read once, full cache lines).
template <int FMT>
struct WStage {
  static constexpr int row_bytes = kStagePairs * PairLayout<FMT>::bytes;  // 272 / 144
  static constexpr int chunks = row_bytes / 16;                          // 17 / 9
  static_assert(row_bytes % 16 == 0, "stage rows must be whole chunks");
  static constexpr int wave_chunks = 16 * chunks;
  static constexpr int loads = (wave_chunks + 63) / 64;                   // per wave per stage
  static constexpr int last_lanes = wave_chunks - 64 * (loads - 1);      // active in the last
  static constexpr int wave_bytes = 16 * row_bytes;
};

// KG: K ranges sharing one workgroup (one ring per range); FOLD: x staging
// area of the digit build.
template <int FMT, int XL, int NW, int KG = 1, bool FOLD = false>
struct StageLayout {
  using XB = XBlock<XL, FMT == kQ4_0>;
  static constexpr bool bias = FMT == kQ4_0;
  static constexpr int w_bytes = NW * WStage<FMT>::wave_bytes;
  static constexpr int x_bytes = XB::stage_bytes;
  static constexpr int bias_bytes = kStageBlocks * XB::bias_bytes;   // dense q4_0 only
  static constexpr int bytes = w_bytes + x_bytes + bias_bytes;
  // Ring depth: three stages when they fit the 160 KB LDS, else two (deeper
  // rings measured slower on MI355X).
  static constexpr int xstage_bytes = FOLD ? 16 * 64 * XL : 0;
  static constexpr int ring = KG * (3 * bytes + xstage_bytes) <= 160 * 1024 ? 3 : 2;
  // The x bytes of a stage are xc 16-byte chunks; wave w copies chunks
  // [w * cpw, (w + 1) * cpw) with gx loads (the last ones partial).
  static constexpr int xc = x_bytes / 16;
  static constexpr int cpw = (xc + NW - 1) / NW;
  static constexpr int gx = (cpw + 63) / 64;
  static_assert((NW - 1) * cpw + 64 * (gx - 1) < xc, "every x load keeps an active lane");
  static constexpr int g = WStage<FMT>::loads + gx + (bias_bytes ? 1 : 0);  // loads per wave per stage
};

// NW wavefronts per workgroup, 16 weight rows each.
//
// FOLD (digit layouts, K % 256 == 0, x 16-byte aligned): no prep launch.  The
// workgroup builds each stage's digit records itself, from x: the x values
// of stage s + S - 1 are loaded into registers (before that stage's weight
// loads, so waiting for them leaves the weights in flight) while stage s is
// computed, then turned into digits (digit_stage_row, the prep kernel's own
// arithmetic, so the records are the same bytes) and written into the free
// ring slot, which the next barriers publish.
//
// KG = 2 (digit layouts): the two K ranges of a row slab run in one
// workgroup, NW waves each with a ring of their own, and meet in LDS at the
// end (range 0 + range 1, always in that order): no atomics, so y needs no
// clearing and, with FOLD, the call no prep launch (the q8_0 4-row layout:
// see run()).
template <int FMT, int XL, int NW, int NST, bool FOLD, int KG = 1>
__global__ __launch_bounds__(64 * NW * KG) void qgemm_mfma(
    const uint8_t* __restrict__ W, const uint8_t* __restrict__ xf, const float* __restrict__ x,
    const float* __restrict__ bias, float* __restrict__ y, float* __restrict__ partial,
    const uint8_t* __restrict__ tail_pad, const int* __restrict__ rexp, int M, int N, int K,
    int nslabs, int ks_count, int nstages) {
  using L = StageLayout<FMT, XL, NW, KG, FOLD>;
  using XB = typename L::XB;
  using WS = WStage<FMT>;
  static_assert(!FOLD || XB::digits, "only the digit layouts are built in the GEMM");
  static_assert(KG == 1 || (KG == 2 && XB::digits), "K ranges meet in LDS in digit mode");
  constexpr int T = XB::T;
  constexpr int kSlab = 16 * NW;
  constexpr int S = L::ring;
  constexpr int G = FOLD ? WS::loads : L::g;   // ring loads per wave per stage
  constexpr int kBiasPerWave = L::bias_bytes / NW;
  static_assert(L::bias_bytes % (16 * NW) == 0, "bias split");
  static_assert(G * (S - 1) < 64, "vmcnt range");
  // One LDS array per ring slot: slot indices are compile-time after
  // unrolling, so the compiler can tell the reads of one slot from the
  // global->LDS writes into another and adds no waits of its own.
  __shared__ __attribute__((aligned(1024))) uint8_t ring0[KG * L::bytes];
  __shared__ __attribute__((aligned(1024))) uint8_t ring1[KG * L::bytes];
  __shared__ __attribute__((aligned(1024))) uint8_t ring2[S > 2 ? KG * L::bytes : 16];

  const int lane = threadIdx.x & 63;
  // kgrp: this wave's K range within the workgroup; wave: its index there
  const int wall = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kgrp = KG == 1 ? 0 : wall / NW;
  const int wave = KG == 1 ? wall : wall % NW;
  const int tid = static_cast<int>(threadIdx.x) - kgrp * 64 * NW;
  auto slot_base = [&](int slot) -> uint8_t* {
    return (slot == 0 ? ring0 : slot == 1 ? ring1 : ring2) + kgrp * L::bytes;
  };
  const int j = lane >> 4;
  const int slab = blockIdx.x % nslabs;
  const int ks = (blockIdx.x / nslabs) * KG + kgrp;
  // NST stages per workgroup (the last K range may hold fewer).
  const int st0 = ks * NST;
  const int st1 = st0 + NST < nstages ? st0 + NST : nstages;
  const int npairs = K / 64;
  const long long row_bytes = static_cast<long long>(K / 32) * (PairLayout<FMT>::bytes / 2);
  const int n = slab * kSlab + wave * 16 + (lane & 15);

  // Every global->LDS load addresses a wave-uniform base (scalar registers)
  // plus a per-lane 32-bit offset that never changes, so no register holding
  // an in-flight load's address is ever reused (which would make the
  // compiler wait for that load).  W must therefore span < 4 GiB.
  // Weight chunk c = 64 q + lane of the wave's 16 stage rows is row
  // c / chunks, bytes 16 (c % chunks) of the row's stage segment.
  uint32_t wrow_off[WS::loads], wchunk[WS::loads];
  bool wlast[WS::loads];   // chunk of W's last row
#pragma unroll
  for (int q = 0; q < WS::loads; ++q) {
    int c = 64 * q + lane;
    c = c < WS::wave_chunks ? c : WS::wave_chunks - 1;
    int r = slab * kSlab + wave * 16 + c / WS::chunks;
    r = r < N ? r : N - 1;
    wrow_off[q] = static_cast<uint32_t>(static_cast<long long>(r) * row_bytes);
    wchunk[q] = static_cast<uint32_t>(16 * (c % WS::chunks));
    wlast[q] = r == N - 1;
  }
  // A last stage with fewer than 4 pairs runs past each row's end into the
  // following rows; those bytes belong to skipped pairs.  W's last row takes
  // its final stage from the zero-padded copy, and any chunk that would run
  // past the end of W (holding skipped bytes only) reads the copy as well.
  const bool short_tail = npairs % kStagePairs != 0;
  const unsigned long long w_end = static_cast<unsigned long long>(N) * row_bytes;
  const uint32_t xoff = static_cast<uint32_t>(16 * (wave * L::cpw + lane));
  const uint32_t boff = static_cast<uint32_t>(wave * kBiasPerWave + lane * 16);
  auto issue = [&](int stage, int slot) {
    const int st = stage < st1 ? stage : st1 - 1;
    const uint8_t* base = slot_base(slot);
    const uint32_t seg = static_cast<uint32_t>(st) * WS::row_bytes;
    if (short_tail && st == nstages - 1) {
#pragma unroll
      for (int q = 0; q < WS::loads; ++q) {
        const unsigned long long a = static_cast<unsigned long long>(wrow_off[q]) + seg + wchunk[q];
        const uint8_t* src = wlast[q] || a + 16 > w_end ? tail_pad + wchunk[q] : W + a;
        const uint8_t* dst = base + wave * WS::wave_bytes + q * 1024;
        if (q + 1 < WS::loads || lane < WS::last_lanes) dma16_addr(src, dst);
      }
    } else {
#pragma unroll
      for (int q = 0; q < WS::loads; ++q) {
        const uint8_t* dst = base + wave * WS::wave_bytes + q * 1024;
        if (q + 1 < WS::loads || lane < WS::last_lanes) dma16(W, wrow_off[q] + seg + wchunk[q], dst);
      }
    }
    if constexpr (!FOLD) {
      const uint8_t* xs = xf + static_cast<long long>(st) * L::x_bytes;
#pragma unroll
      for (int i = 0; i < L::gx; ++i) {
        const int c = 64 * i + lane;   // chunk wave * cpw + c of the stage
        if (c < L::cpw && wave * L::cpw + c < L::xc)
          dma16(xs, xoff + i * 1024, base + L::w_bytes + 16 * (wave * L::cpw + 64 * i));
      }
    }
    if constexpr (L::bias_bytes > 0) {
      // Wave w moves bias bytes [w, w+1) * kBiasPerWave of the stage with
      // its first kBiasPerWave / 16 lanes.
      const uint8_t* bs = reinterpret_cast<const uint8_t*>(bias) +
                          static_cast<long long>(st) * L::bias_bytes;
      if (lane < kBiasPerWave / 16)
        dma16(bs, boff, base + L::w_bytes + L::x_bytes + wave * kBiasPerWave);
    }
  };

  // FOLD: task tau = tid + NT * t of a stage is (row m, block b, part p) with
  // m = tau >> 6, b = (tau >> 3) & 7, p = tau & 7 -- one wavefront per row --
  // each 16 bytes of x; a workgroup with more threads leaves its last waves
  // idle.
  // The x bytes of a stage are copied into `xstage` (task tau at byte 16 tau)
  // by global->LDS loads like the weights', so every load in flight stays
  // invisible to the compiler and every wait explicit; rows past M read row
  // 0 and are zeroed when the digits are built.
  constexpr int kTasks = 64 * XL, kThreadsWg = 64 * NW;
  constexpr int TPT = kTasks >= kThreadsWg ? kTasks / kThreadsWg : 1;
  __shared__ __attribute__((aligned(16))) uint8_t xstage_all[FOLD ? KG * 16 * kTasks : 16];
  uint8_t* const xstage = xstage_all + (FOLD ? kgrp * 16 * kTasks : 0);
  const bool xtask = kTasks >= kThreadsWg || wave * 64 < kTasks;   // wave-uniform
  uint32_t xsrc[TPT];
#pragma unroll
  for (int t = 0; t < TPT; ++t) {
    const int tau = tid + kThreadsWg * t;
    const int m = tau >> 6;
    xsrc[t] = static_cast<uint32_t>(4 * (static_cast<long long>(m < M ? m : 0) * K + 4 * lane));
  }
  auto load_x = [&](int stage) {
    if constexpr (FOLD) {
      const int st = stage < st1 ? stage : st1 - 1;
      const uint8_t* base = reinterpret_cast<const uint8_t*>(x) +
                            static_cast<long long>(st) * (4 * 32 * kStageBlocks);
      if (xtask) {
#pragma unroll
        for (int t = 0; t < TPT; ++t)
          dma16(base, xsrc[t], xstage + 16 * (kThreadsWg * t + 64 * wave));
      }
    }
  };
  auto build_x = [&](int slot) {
    if constexpr (FOLD) {
      uint8_t* rec0 = slot_base(slot) + L::w_bytes;
      if (xtask) {
#pragma unroll
        for (int t = 0; t < TPT; ++t) {
          const int tau = tid + kThreadsWg * t;
          const int m = tau >> 6;
          const bool live = m < M;
          const f32x4 xv = *reinterpret_cast<const f32x4*>(xstage + 16 * tau);
          const float v[4] = {live ? xv[0] : 0.f, live ? xv[1] : 0.f, live ? xv[2] : 0.f,
                              live ? xv[3] : 0.f};
          digit_stage_row<XL, FMT == kQ4_0>(v, m, true, rec0);
        }
      }
    }
  };

  f32x4 acc[T];     // bf16 mode: output (m = 16t + 4j + e, n)
  float accd[T];    // digit mode: output (m = 4t + j, n)
  uint32_t badrows = 0u;   // digit mode: bit t when row 4t + j met a non-finite stage
#pragma unroll
  for (int t = 0; t < T; ++t) {
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    accd[t] = 0.f;
  }

  // The LDS operands of one block pair: the lane's code bytes and scales and,
  // per block and tile, the activation operand (digit planes, or hi / lo)
  // and the q4_0 C input.  compute() loads pair pp + 1 before it computes
  // pair pp, so the LDS latency is covered by a pair's MFMAs and VALU work.
  using Op = typename OpType<FMT>::T;
  struct PairOps {
    u32x3_a4 b0;
    u32x2_a4 b1;
    uint32_t s0, s1;
    long a[2][T];       // digit mode
    i32x4 cb[2][T];     // digit mode, q4_0
    Op xh[2][T], xl[2][T];
    f32x4 bb[2][T];     // dense mode, q4_0
  };
  auto load_ops = [&](const uint8_t* row, const uint8_t* xs, int pp) {
    PairOps o;
    const uint32_t* pr = reinterpret_cast<const uint32_t*>(row + pp * PairLayout<FMT>::bytes);
    o.b0 = *reinterpret_cast<const u32x3_a4*>(pr + PairLayout<FMT>::blk0_dword(j));
    o.b1 = *reinterpret_cast<const u32x2_a4*>(pr + PairLayout<FMT>::blk1_dword(j));
    o.s0 = pr[0];
    o.s1 = pr[PairLayout<FMT>::scale1_dword];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int blk = 2 * pp + h;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        if constexpr (XB::digits) {
          const uint8_t* rec = xs + blk * XB::bytes;
          o.a[h][t] = *reinterpret_cast<const long*>(rec + t * 512 + 8 * lane);
          if constexpr (L::bias)
            o.cb[h][t] = *reinterpret_cast<const i32x4*>(rec + XB::bias_off + 16 * (4 * t + j));
        } else {
          const uint8_t* f = xs + (blk * T + t) * kFragBytes + lane * 16;
          o.xh[h][t] = *reinterpret_cast<const Op*>(f);
          o.xl[h][t] = *reinterpret_cast<const Op*>(f + 1024);
          if constexpr (L::bias)
            o.bb[h][t] = *reinterpret_cast<const f32x4*>(xs + L::x_bytes + (blk * T + t) * 64 + 16 * j);
        }
      }
    }
    return o;
  };

  // Branch-free, so the compiler can overlap the pairs' LDS reads, code
  // conversions and MFMAs.  A pair past K or a stage past st1 (clamped
  // reloads) adds c * 0: its codes are finite integers and its activation
  // fragments zero or finite, so c is finite, and its scale is replaced by 0.
  auto compute = [&](int stage, int slot, bool live) {
    const uint8_t* base = slot_base(slot);
    const uint8_t* row = base + wave * WS::wave_bytes + (lane & 15) * WS::row_bytes;
    const uint8_t* xs = base + L::w_bytes;
    float sacc[T];    // digit mode: this stage's sum, before its exponent
#pragma unroll
    for (int t = 0; t < T; ++t) sacc[t] = 0.f;
    PairOps cur = load_ops(row, xs, 0);
#pragma unroll
    for (int pp = 0; pp < kStagePairs; ++pp) {
      PairOps nxt;
      if (pp + 1 < kStagePairs) nxt = load_ops(row, xs, pp + 1);
      __builtin_amdgcn_sched_barrier(0);
      const bool valid = live && stage * kStagePairs + pp < npairs;   // wave-uniform
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t c0 = h == 0 ? __builtin_amdgcn_alignbyte(cur.b0.y, cur.b0.x, 2) : cur.b1.x;
        const uint32_t c1 = h == 0 ? __builtin_amdgcn_alignbyte(cur.b0.z, cur.b0.y, 2) : cur.b1.y;
        const uint32_t dbits = h == 0 ? (cur.s0 & 0xFFFFu) : (cur.s1 >> 16);
        if constexpr (XB::digits) {
          // B operand: the lane's 8 codes as int8 (q8_0 as stored; q4_0
          // nibbles 0..15, the -8 entering through the C input).
          uint32_t w0 = c0, w1 = c1;
          if constexpr (FMT == kQ4_0) {
            const int sh = (j >> 1) * 4;
            w0 = (c0 >> sh) & 0x0F0F0F0Fu;
            w1 = (c1 >> sh) & 0x0F0F0F0Fu;
          }
          const long wq = static_cast<long>(w0) | (static_cast<long>(w1) << 32);
          const float dw = valid ? half_bits_to_float(dbits) : 0.0f;
#pragma unroll
          for (int t = 0; t < T; ++t) {
            i32x4 c = {0, 0, 0, 0};
            if constexpr (L::bias) c = cur.cb[h][t];
            // D lane (n, j): digit sums S_0..S_3 of row m = 4t + j (S_3 = 0)
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8(cur.a[h][t], wq, c, 0, 0, 0);
            // 2^7 S1 + S2 is exact in int32 (|S| < 2^20), and its float
            // conversion is the same single rounding as fmaf(S1, 128, S2)
            const float f = fmaf(static_cast<float>(c[0]), 16384.f,
                                 static_cast<float>((c[1] << 7) + c[2]));
            sacc[t] = fmaf(dw, f, sacc[t]);
          }
        } else {
          const Op wv = codes_op<FMT>(c0, c1, j);
          const float d = valid ? half_bits_to_float(dbits) : 0.0f;
#pragma unroll
          for (int t = 0; t < T; ++t) {
            f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
            if constexpr (L::bias) c = cur.bb[h][t];
            c = mfma_op(cur.xh[h][t], wv, c);
            c = mfma_op(cur.xl[h][t], wv, c);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[t][e] = fmaf(c[e], d, acc[t][e]);
          }
        }
      }
      if (pp + 1 < kStagePairs) cur = nxt;
    }
    if constexpr (XB::digits) {
      // the stage's exponent and gate of row m = 4t + j, from block 0's
      // record (a clamped reload of a stage past the workgroup's range adds
      // nothing, whatever its gate)
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int2 me = *reinterpret_cast<const int2*>(xs + XB::meta_off + 8 * (4 * t + j));
        const float v = ldexpf(sacc[t] * __int_as_float(me.y), me.x);
        accd[t] += live ? v : 0.0f;
        badrows |= live && me.y != __float_as_int(1.0f) ? 1u << t : 0u;
      }
    }
  };

  // Fully unrolled over the workgroup's NST stages (straight-line code).
  // Each step waits for its stage, meets the workgroup (so the slot the
  // next issue overwrites is no longer read), issues the loads S-1 stages
  // ahead and then computes, so S-1 stages are in flight during the
  // compute.  Stages past st1 only issue (clamped) loads.
  //
  // FOLD: each stage's x loads go out just before its ring loads, and are
  // waited for (vmcnt <= G: the ring loads issued after them may stay in
  // flight) once the current stage is computed; the digits then go into the
  // stage's slot.  In-order retirement makes that wait also cover every
  // earlier stage's ring loads, so at a step's start only the most recent
  // stage's ring loads can be outstanding and the stage wait below stays
  // exact.
#pragma unroll
  for (int i = 0; i < S - 1; ++i)
    if (i < NST) {
      if constexpr (FOLD) {
        if (i > 0) {   // every wave is done reading xstage
          wait_lgkmcnt0();
          ring_barrier();
        }
      }
      load_x(st0 + i);
      issue(st0 + i, i);
      if constexpr (FOLD) {
        wait_vmcnt<G>();
        build_x(i);
      }
    }
#pragma unroll
  for (int i = 0; i < NST; ++i) {
    const int cur = st0 + i;
    // Stage `cur` has landed; the issues of min(S-2, NST-1-i) later stages
    // may still be in flight.
    wait_stages<G, S - 2>(NST - 1 - i);
    wait_lgkmcnt0();
    ring_barrier();
    if (i + S - 1 < NST) {
      load_x(cur + S - 1);
      issue(cur + S - 1, (i + S - 1) % S);
    }
    compute(cur, i % S, cur < st1);
    if constexpr (FOLD) {
      if (i + S - 1 < NST) {
        wait_vmcnt<G>();
        build_x((i + S - 1) % S);
      }
    }
    // Materialise the accumulators here: otherwise the compiler sinks the
    // scale FMAs of every stage into the (conditional) store block and keeps
    // all MFMA results of the workgroup live until then.
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if constexpr (XB::digits) asm volatile("" : "+v"(accd[t]));
      else asm volatile("" : "+v"(acc[t]));
    }
  }
  wait_vmcnt<0>();   // no global->LDS load may outlive the workgroup's LDS
  // Blocks [b0, b1) of this K range.  An activation row holding NaN or +-inf
  // (digit mode: a stage gate NaN; the f16 / bf16 layouts: rexp marked) has
  // its outputs recomputed in the reference's f32 form.
  const int b0 = st0 * kStageBlocks;
  const int b1 = st1 * kStageBlocks < K / 32 ? st1 * kStageBlocks : K / 32;
  const uint8_t* const wrow_n = W + static_cast<long long>(n < N ? n : N - 1) * row_bytes;
  if constexpr (XB::digits) {
    if (__any(badrows != 0u)) {
#pragma unroll 1
      for (int t = 0; t < T; ++t) {
        const int m = 4 * t + j;
        if (((badrows >> t) & 1u) != 0u && n < N && m < M) {
          const float v = nonfinite_blocks_f32<FMT>(wrow_n, x + static_cast<long long>(m) * K, b0, b1);
#pragma unroll
          for (int u = 0; u < T; ++u)
            if (u == t) accd[u] = v;
        }
      }
    }
  }
  if constexpr (KG == 2) {
    // range 1's sums to LDS (the rings are no longer read), then range 0
    // adds them and stores
    float* ex = reinterpret_cast<float*>(ring0);
    wait_lgkmcnt0();
    ring_barrier();
    if (kgrp == 1) {
#pragma unroll
      for (int t = 0; t < T; ++t) ex[t * 64 * NW + tid] = accd[t];
    }
    wait_lgkmcnt0();
    ring_barrier();
    if (kgrp == 1) return;
#pragma unroll
    for (int t = 0; t < T; ++t) accd[t] = accd[t] + ex[t * 64 * NW + tid];
  }

  // acc[t][e] is output (m = 16t + 4j + e, n).  One K range: store.  Two:
  // both add into the zeroed y (0 + a + b == 0 + b + a, so the result does
  // not depend on which finishes first).  More: partial sums for the
  // reduction kernel.
  if (n >= N) return;
  auto store = [&](int m, float v) {
    const long long o = static_cast<long long>(m) * N + n;
    if (ks_count == 1) y[o] = v;
    else if (ks_count == 2) atomicAdd(y + o, v);
    else partial[static_cast<long long>(ks) * M * N + o] = v;
  };
  bool special = false;   // f16 / bf16 layouts: a row of this lane holds NaN or +-inf
  auto put = [&](int m, float v) {
    if (m >= M) return;
    if constexpr (!XB::digits) {
      const int r = rexp[m];
      if (r == kRowNonfinite) {   // stored by the loop below
        special = true;
        return;
      }
      v = ldexpf(v, r);   // undo the row scale
    }
    store(m, v);
  };
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if constexpr (XB::digits) {
      put(4 * t + j, accd[t]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) put(16 * t + 4 * j + e, acc[t][e]);
    }
  }
  if constexpr (!XB::digits) {
    if (__any(special)) {
#pragma unroll 1
      for (int q = 0; q < 4 * T; ++q) {
        const int m = 16 * (q >> 2) + 4 * j + (q & 3);
        if (m < M && rexp[m] == kRowNonfinite)
          store(m, nonfinite_blocks_f32<FMT>(wrow_n, x + static_cast<long long>(m) * K, b0, b1));
      }
    }
  }
}


// Scratch (activation fragments, q4 bias, partial sums, row exponents) of
// one qgemm call.  Region 0 holds one pass's fragments and partial sums,
// region 1 the call's row exponents (live across all passes).  Allocating
// entry points take buffers 0 and 1 of the stream's cache entry
// (stream_workspace, qc_internal.h).
//
// Where a call's scratch comes from: a per-stream cache entry (whose `call`
// lock the caller holds), or a fixed region given by the caller -- region 1
// at [0, fixed_split), region 0 at [fixed_split, fixed_bytes).  A fixed
// region never grows: a request beyond it fails with hipErrorOutOfMemory
// before anything is launched (the first pass of a call needs the most).
struct Scratch {
  StreamWorkspace* w = nullptr;
  uint8_t* fixed = nullptr;
  size_t fixed_split = 0, fixed_bytes = 0;
  int max_ks = 0;   // > 0: K split limit for the small-batch plan (see plan_for)
  int fold = 0;     // digit layouts: 0 = build the digits in the GEMM where it can, -1 = never

  hipError_t get(hipStream_t s, size_t bytes, void** out, int tag = 0) {
    if (w == nullptr) {
      const size_t lo = tag == 1 ? 0 : fixed_split;
      const size_t hi = tag == 1 ? fixed_split : fixed_bytes;
      if (bytes > hi - lo) return hipErrorOutOfMemory;
      *out = fixed + lo;
      return hipSuccess;
    }
    return stream_buffer(w, s, bytes, tag, out);
  }
};

struct MfmaArgs {
  const uint8_t* W;
  const uint8_t* xf;
  const float* x;
  const float* bias;
  float* y;
  float* partial;
  const uint8_t* tail_pad;
  const int* rexp;
  int m, n, k, nslabs, ks, nstages;
};

// KG = 2: a.ks must be 2; one workgroup of 2 NW waves per row slab, which
// stores y itself (ks_count 1).
template <int FMT, int XL, int NW, int NST, bool FOLD, int KG = 1>
hipError_t launch_nst(const MfmaArgs& a, hipStream_t s) {
  qgemm_mfma<FMT, XL, NW, NST, FOLD, KG><<<a.nslabs * (a.ks / KG), 64 * NW * KG, 0, s>>>(
      a.W, a.xf, a.x, a.bias, a.y, a.partial, a.tail_pad, a.rexp, a.m, a.n, a.k, a.nslabs,
      KG == 2 ? 1 : a.ks, a.nstages);
  return hipGetLastError();
}

template <int FMT, int XL, int NW, bool FOLD, int KG = 1>
hipError_t launch_nw(int nst, const MfmaArgs& a, hipStream_t s) {
  switch (nst) {
    case 16: return launch_nst<FMT, XL, NW, 16, FOLD, KG>(a, s);
    case 8: return launch_nst<FMT, XL, NW, 8, FOLD, KG>(a, s);
    case 4: return launch_nst<FMT, XL, NW, 4, FOLD, KG>(a, s);
    case 2: return launch_nst<FMT, XL, NW, 2, FOLD, KG>(a, s);
    default: return launch_nst<FMT, XL, NW, 1, FOLD, KG>(a, s);
  }
}

// Workgroup width (NW wavefronts = 16 NW rows) and stages per workgroup
// (NST; K is split ceil(nstages / NST) ways) from a simple cost model of
// this kernel on gfx950: one workgroup per CU at a time (LDS), a CU streams
// at most ~37 GB/s on its own and the chip ~5.2 TB/s, a stage costs a wave
// c(XL) of compute (0.67 / 1.25 / 1.4 / 2.15 us for 4 / 8 / 16 / 32
// activation rows, fitted on MI355X; 1.4x that for an 8-wave workgroup,
// whose two waves per SIMD share it), a workgroup costs ~1.5 us of latency,
// and a K split beyond two ways costs a reduction kernel (~3.5 us).  The
// compute term is what makes N = 4096 with 8-32 rows split K four ways
// (6-20% faster than two).
struct Plan {
  int nw, nst, ks;
};
// max_ks > 0 limits the K split to max(max_ks, the fewest ranges possible),
// which bounds the partial-sum scratch.
template <int FMT>
Plan plan_for(int n, int nstages, int cus, int max_ks = 0, int xl = 4) {
  const double c_stage = xl <= 4 ? 0.67e-6 : xl <= 8 ? 1.25e-6 : xl <= 16 ? 1.4e-6 : 2.15e-6;
  Plan best{8, 16, (nstages + 15) / 16};
  double best_t = 1e30;
  const int ks_cap = max_ks > 0 ? std::max(max_ks, (nstages + 15) / 16) : nstages;
  for (int nw : {8, 4}) {
    const int nslabs = (n + 16 * nw - 1) / (16 * nw);
    for (int nst : {16, 8, 4, 2, 1}) {
      const int ks = (nstages + nst - 1) / nst;
      // for K <= 4096, more than four K ranges measured slower (the
      // reduction reads ks partial sets)
      if (ks > ks_cap || (nstages <= 16 && ks > 4)) continue;
      const long long wgs = static_cast<long long>(nslabs) * ks;
      const long long active = wgs < cus ? wgs : cus;
      const long long rounds = (wgs + cus - 1) / cus;
      const double rate = std::min(37e9, 5.2e12 / static_cast<double>(active));
      const double wg_bytes = 16.0 * nw * nst * kStagePairs * PairLayout<FMT>::bytes;
      const double wg_compute = nst * c_stage * (nw == 8 ? 1.4 : 1.0);
      const double t = rounds * (std::max(wg_bytes / rate, wg_compute) + 1.5e-6) +
                       (ks > 2 ? 3.5e-6 : 0.0);
      if (t < best_t * 0.999) {
        best_t = t;
        best = Plan{nw, nst, ks};
      }
    }
  }
  return best;
}

template <int FMT, int XL>
hipError_t run(const uint8_t* W, const float* x, float* y, int m, int n, int k, hipStream_t s,
               int waves, int stages, int* rexp, Scratch& scratch) {
  const int nb = k / 32;
  const int nstages = (nb + kStageBlocks - 1) / kStageBlocks;
  const int nbp = nstages * kStageBlocks;
  Plan plan = plan_for<FMT>(n, nstages, device_cu_count(), scratch.max_ks, XL);
  if (waves) plan.nw = waves;                      // test / tuning overrides
  if (stages) {
    plan.nst = stages;
    plan.ks = (nstages + stages - 1) / stages;
  }
  const int nslabs = (n + 16 * plan.nw - 1) / (16 * plan.nw);
  const int ks = plan.ks;
  using XB = XBlock<XL, FMT == kQ4_0>;
  // the bf16 / f16 layouts store and apply per-row exponents
  if (!XB::digits && rexp == nullptr) return hipErrorInvalidValue;
  // Digit layouts without the prep launch: the GEMM builds the digits (no
  // short last stage to pad, x loadable in 16-byte pieces, and no y to clear
  // for a two-way K split).
  // A two-way K split either keeps the prep launch (which clears y for the
  // two atomic halves) or, for q8_0 with up to 4 rows, runs both ranges in
  // one workgroup, meeting in LDS (K=4096 N=14336 M=4: 18.4 -> 17.0 us).
  // With 8 rows, or q4_0's half-size weights, the digit builds the paired
  // workgroup repeats cost more than the launch (q4_0 M=8 17.8 -> 22.5 us).
  const bool can_fold = XB::digits && scratch.fold >= 0 && k % (32 * kStageBlocks) == 0 &&
                        reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                        static_cast<long long>(m) * k * 4 < (1LL << 32);
  const bool paired = can_fold && ks == 2 && XL == 4 && FMT == kQ8_0;
  const bool fold = can_fold && (ks != 2 || paired);
  const size_t xf_bytes = fold ? 0 : static_cast<size_t>(nstages) * XB::stage_bytes;
  const size_t bias_bytes = static_cast<size_t>(nbp) * XB::bias_bytes;
  const size_t part_bytes = ks > 2 ? static_cast<size_t>(ks) * m * n * sizeof(float) : 0;
  const size_t pad_bytes = WStage<FMT>::row_bytes;
  const size_t total = xf_bytes + bias_bytes + part_bytes + pad_bytes + 256;
  void* ws = nullptr;
  hipError_t e = scratch.get(s, total, &ws);
  if (e != hipSuccess) return e;
  uint8_t* xf = static_cast<uint8_t*>(ws);
  float* bias = reinterpret_cast<float*>(xf + xf_bytes);
  float* partial = reinterpret_cast<float*>(xf + xf_bytes + bias_bytes);
  uint8_t* tail_pad = xf + xf_bytes + bias_bytes + part_bytes;

  const long long outs = static_cast<long long>(m) * n;
  const long long row_bytes = static_cast<long long>(nb) * PairLayout<FMT>::bytes / 2;
  const int tail = (k / 64) % kStagePairs * PairLayout<FMT>::bytes;
  const uint8_t* tail_src = W + (n - 1) * row_bytes + static_cast<long long>(nstages - 1) * WStage<FMT>::row_bytes;
  if (!fold) {
    if constexpr (XB::digits)
      qgemm_prep<XL, FMT == kQ4_0><<<nstages * XL, 64, 0, s>>>(x, m, k, xf, y, ks == 2 ? outs : 0,
                                                               tail_src, tail, tail_pad,
                                                               static_cast<int>(pad_bytes));
    else
      prep_rows<false, FMT == kQ4_0>
          <<<XL + (ks == 2 ? clear_workgroups(outs) : 0), 256, 0, s>>>(
              x, m, k, nbp, XB::T, xf, bias, rexp, y, ks == 2 ? outs : 0, tail_src, tail,
              tail_pad, static_cast<int>(pad_bytes), XL);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const MfmaArgs a{W, xf, x, bias, y, partial, tail_pad, rexp, m, n, k, nslabs, ks, nstages};
  if constexpr (XB::digits) {
    if (paired) {
      // the same waves per row slab as the plan: 4 per K range
      if constexpr (XL == 4 && FMT == kQ8_0) {
        MfmaArgs p = a;
        p.nslabs = (n + 63) / 64;
        e = launch_nw<FMT, XL, 4, true, 2>(plan.nst, p, s);
      }
    } else if (fold)
      e = plan.nw == 8 ? launch_nw<FMT, XL, 8, true>(plan.nst, a, s)
                       : launch_nw<FMT, XL, 4, true>(plan.nst, a, s);
    else
      e = plan.nw == 8 ? launch_nw<FMT, XL, 8, false>(plan.nst, a, s)
                       : launch_nw<FMT, XL, 4, false>(plan.nst, a, s);
  } else {
    e = plan.nw == 8 ? launch_nw<FMT, XL, 8, false>(plan.nst, a, s)
                     : launch_nw<FMT, XL, 4, false>(plan.nst, a, s);
  }
  if (e != hipSuccess || ks <= 2) return e;
  const long long blocks = (outs + 255) / 256;
  qgemm_reduce<<<static_cast<unsigned>(blocks < 4096 ? blocks : 4096), 256, 0, s>>>(partial, y, outs, ks);
  return hipGetLastError();
}

// ------------------------------------------------ panel route, M >= 64 ---
//
// The reference switches qgemm_prepacked to a row-panel GEMM at M >= 64
// (kernels/quantization/qgemm_panel.cpp:234-286).  Here every M >= 64 call
// (qgemm and qgemm_prepacked) runs one 2-D tiled GEMM instead of passes of 32
// rows, each of which re-streams the whole weight matrix.  Numerics are those
// of the f16 / bf16 passes above (hi/lo activations, exact codes, per-block
// f32 scaling), so the contract bound is unchanged.
//
// Workgroup: 8 wavefronts as 2 (m) x 4 (n), each computing 64 x 64 outputs
// as 4 x 4 tiles of v_mfma_f32_16x16x32_{f16,bf16}; workgroup tile 128 x 256.  K
// runs in stages of one block pair (64 elements) through a 3-deep LDS ring
// filled by global_load_lds: the activation fragments of the workgroup's 8
// m-tiles (hi, lo, and the q4_0 bias) as 16-byte chunks, and the pair's bytes
// of its 256 weight rows as dwords.  Every wavefront issues the same loads
// per stage (spare weight lanes re-read a valid dword into padding), so the
// waits are exact counts, as in the small-batch kernel.
constexpr int kPTN = 4;                           // 16x16 tiles per wave (n)
constexpr int kPWM = 2, kPWN = 4;                 // waves per workgroup (m, n)
constexpr int kPWaves = kPWM * kPWN;
constexpr int kPBN = 16 * kPTN * kPWN;            // 256 rows of W per workgroup

// TM: 16x16 tiles per wave along m (4: 128 x 256 workgroup tiles with a
// 3-deep ring; 8: 256 x 256 with a 2-deep ring).
template <int FMT, int TM>
struct PanelStage {
  static constexpr bool bias = FMT == kQ4_0;
  static constexpr int bm = 16 * TM * kPWM;                         // rows of x per workgroup
  static constexpr int mt = bm / 16;                                // m-tiles per workgroup
  static constexpr int pd = PairLayout<FMT>::bytes / 4;             // 17 / 9 dwords per row
  static constexpr int x_bytes = mt * 2 * kFragBytes;               // 32 / 64 KB
  static constexpr int x_loads = x_bytes / 16 / (64 * kPWaves);     // 4 / 8 chunks per lane
  static constexpr int b_bytes = bias ? mt * 2 * 64 : 0;            // 1 / 2 KB
  static constexpr int w_dwords = kPBN * pd;
  static constexpr int w_loads = (w_dwords + 64 * kPWaves - 1) / (64 * kPWaves);  // 9 / 5
  static constexpr int w_bytes = kPWaves * w_loads * 256;           // with padding
  static constexpr int bytes = x_bytes + b_bytes + w_bytes;
  static constexpr int ring = 3 * bytes <= 160 * 1024 ? 3 : 2;
  static constexpr int g = x_loads + (bias ? 1 : 0) + w_loads;      // loads per wave per stage
  static_assert(x_bytes % (16 * 64 * kPWaves) == 0, "whole x loads");
  static_assert(ring * bytes <= 160 * 1024, "LDS");
  static_assert(g * (ring - 1) < 64, "vmcnt range");
  static_assert(mt % kPWaves == 0 && mt / kPWaves <= 8 && ((mt / kPWaves) & (mt / kPWaves - 1)) == 0,
                "bias loads: 8 lanes per m-tile, a power-of-two count of whole m-tiles per wave");
};

template <int FMT, int TM>
__global__ __launch_bounds__(64 * kPWaves, 1) void qgemm_panel(
    const uint8_t* __restrict__ W, const uint8_t* __restrict__ xf, const float* __restrict__ bias,
    float* __restrict__ y, const int* __restrict__ rexp, const float* __restrict__ x, int M,
    int N, int K, int pairs_per_split, int ks_count) {
  using PS = PanelStage<FMT, TM>;
  constexpr int PB = PairLayout<FMT>::bytes;
  constexpr int G = PS::g;
  constexpr int R = PS::ring;
  constexpr int BR = PS::mt / kPWaves;           // bias m-tiles per wave (1 / 2)
  __shared__ __attribute__((aligned(1024))) uint8_t ring0[PS::bytes];
  __shared__ __attribute__((aligned(1024))) uint8_t ring1[PS::bytes];
  __shared__ __attribute__((aligned(1024))) uint8_t ring2[R > 2 ? PS::bytes : 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % kPWM, wn = wave / kPWM;
  const int j = lane >> 4;
  const int n0 = blockIdx.x * kPBN;
  const int mt0 = blockIdx.y * PS::mt;
  const int nb = K / 32, npairs = K / 64;
  const int p0 = blockIdx.z * pairs_per_split;
  const int p1 = min(p0 + pairs_per_split, npairs);
  const long long row_bytes = static_cast<long long>(nb) * (PB / 2);

  // Sources: a wave-uniform base per workgroup and stage (scalar registers)
  // plus a per-lane 32-bit offset that never changes, so issuing a stage
  // costs no vector arithmetic.  x chunk c = (wave * x_loads + i) * 64 + lane:
  // m-tile c >> 8, byte 16 (c & 255) of its pair (blocks 2p, 2p + 1 adjacent).
  const uint8_t* xbase = xf + static_cast<long long>(mt0) * nb * kFragBytes;
  uint32_t xoff[PS::x_loads];
#pragma unroll
  for (int i = 0; i < PS::x_loads; ++i) {
    const int c = (wave * PS::x_loads + i) * 64 + lane;
    xoff[i] = static_cast<uint32_t>((c >> 8) * nb * kFragBytes + 16 * (c & 255));
  }
  // bias: wave w, lanes 0 .. 8 BR - 1, 128 B of each of m-tiles
  // BR w .. BR w + BR - 1 (the pair's two blocks)
  const uint8_t* bbase = reinterpret_cast<const uint8_t*>(bias) +
                         static_cast<long long>(mt0) * nb * 64;
  const uint32_t boff = static_cast<uint32_t>((wave * BR + ((lane >> 3) & (BR - 1))) * nb * 64 +
                                              16 * (lane & 7));
  // weight dword d = (wave * w_loads + i) * 64 + lane: row d / pd, dword
  // d % pd; d past the stage re-reads the stage's last dword
  const uint8_t* wbase = W + static_cast<long long>(n0) * row_bytes;
  uint32_t woff[PS::w_loads];
#pragma unroll
  for (int i = 0; i < PS::w_loads; ++i) {
    int d = (wave * PS::w_loads + i) * 64 + lane;
    d = d < PS::w_dwords ? d : PS::w_dwords - 1;
    const int r = min(n0 + d / PS::pd, N - 1) - n0;
    woff[i] = static_cast<uint32_t>(r * row_bytes + 4 * (d % PS::pd));
  }
  auto slot_base = [&](int slot) -> uint8_t* { return slot == 0 ? ring0 : slot == 1 ? ring1 : ring2; };
  // Load l (0 .. G - 1; a constant after unrolling) of stage p into a slot:
  // the x chunks, then (q4_0) the bias, then the weight dwords.
  auto issue_one = [&](int p, int slot, int l) {
    uint8_t* base = slot_base(slot);
    if (l < PS::x_loads) {
      dma16(xbase + static_cast<long long>(2 * p) * kFragBytes, xoff[l < PS::x_loads ? l : 0],
            base + 16 * (wave * PS::x_loads + l) * 64);
    } else if (PS::bias && l == PS::x_loads) {
      if (lane < 8 * BR) dma16(bbase + 128 * p, boff, base + PS::x_bytes + 128 * BR * wave);
    } else {
      const int wl = l - PS::x_loads - (PS::bias ? 1 : 0);
      dma4(wbase + static_cast<long long>(p) * PB, woff[wl >= 0 ? wl : 0],
           base + PS::x_bytes + PS::b_bytes + 256 * (wave * PS::w_loads + wl));
    }
  };
  auto issue = [&](int p, int slot) {
#pragma unroll
    for (int l = 0; l < G; ++l) issue_one(p, slot, l);
  };

  f32x4 acc[TM][kPTN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < kPTN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Decoded weight fragments of one half stage (one block of the pair):
  // codes as bf16 and the block scales of the wave's 4 n-tiles.
  using Op = typename OpType<FMT>::T;
  struct HalfW {
    Op w[kPTN];
    float d[kPTN];
  };
  auto decode = [&](int slot, int h, HalfW& o) {
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(slot_base(slot) + PS::x_bytes + PS::b_bytes);
#pragma unroll
    for (int tn = 0; tn < kPTN; ++tn) {
      const uint32_t* pr = sw + (wn * 64 + tn * 16 + (lane & 15)) * PS::pd;
      uint32_t c0, c1, dbits;
      if (h == 0) {
        const uint32_t b0x = pr[PairLayout<FMT>::blk0_dword(j)];
        const uint32_t b0y = pr[PairLayout<FMT>::blk0_dword(j) + 1];
        const uint32_t b0z = pr[PairLayout<FMT>::blk0_dword(j) + 2];
        c0 = __builtin_amdgcn_alignbyte(b0y, b0x, 2);
        c1 = __builtin_amdgcn_alignbyte(b0z, b0y, 2);
        dbits = pr[0] & 0xFFFFu;
      } else {
        c0 = pr[PairLayout<FMT>::blk1_dword(j)];
        c1 = pr[PairLayout<FMT>::blk1_dword(j) + 1];
        dbits = pr[PairLayout<FMT>::scale1_dword] >> 16;
      }
      o.w[tn] = codes_op<FMT>(c0, c1, j);
      o.d[tn] = half_bits_to_float(dbits);
    }
  };
  // The 2 x kPTN MFMAs of m-tile tm against one decoded half, each tile's
  // block sum scaled into the accumulators.
  auto mma = [&](int slot, int h, int tm, const HalfW& hw) {
    const uint8_t* base = slot_base(slot);
    const int mt = wm * TM + tm;
    const uint8_t* f = base + (mt * 2 + h) * kFragBytes + 16 * lane;
    const Op xh = *reinterpret_cast<const Op*>(f);
    const Op xl = *reinterpret_cast<const Op*>(f + 1024);
    f32x4 c0 = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (PS::bias)
      c0 = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base + PS::x_bytes) +
                                           (mt * 2 + h) * 16 + 4 * j);
#pragma unroll
    for (int tn = 0; tn < kPTN; ++tn) {
      f32x4 c = mfma_op(xh, hw.w[tn], c0);
      c = mfma_op(xl, hw.w[tn], c);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[tm][tn][e] = fmaf(c[e], hw.d[tn], acc[tm][tn][e]);
    }
  };
  auto pin_acc = [&]() {
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < kPTN; ++b) asm volatile("" : "+v"(acc[a][b]));
  };

  // Ring of R stages.  Stages p0 .. p0 + R - 2 are in flight before the
  // loop.  Step i starts with the wave's wait for stage p0 + i + 1 and a
  // workgroup barrier, after which that stage is visible to every wave and
  // no wave reads stage p0 + i - 1, whose slot receives stage p0 + i + R - 1.
  // Those loads are spread over block 0's MFMAs so that the eight waves do
  // not queue them all at once.  Weights are decoded one half stage ahead:
  // block 1's decode overlaps block 0's MFMAs, and block 0 of stage
  // p0 + i + 1 is decoded during block 1's.  Past the last stage the loads
  // repeat stage p1 - 1 into the free slot and the decode reads a slot whose
  // result is unused, so every step is the same straight-line code.
  // Unrolled by the ring depth so every slot index is a constant.
  static_assert(R >= 3, "the next stage must land while the current one is read");
  const int count = p1 - p0;
  if (count > 0) {
#pragma unroll
    for (int i = 0; i < R - 1; ++i)
      if (i < count) issue(p0 + i, i);
    wait_stages<G, R - 2>(min(R - 2, count - 1));
    wait_lgkmcnt0();
    ring_barrier();
    HalfW h0, h1;
    decode(0, 0, h0);
    auto step = [&](int i, int slot) {
      // stages issued after stage i + 1 and possibly still in flight
      wait_stages<G, R - 3>(min(R - 3, count - 2 - i));
      wait_lgkmcnt0();
      ring_barrier();
      const int pi = min(p0 + i + R - 1, p1 - 1);
      const int si = (slot + R - 1) % R;
      decode(slot, 1, h1);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
        for (int l = tm * G / TM; l < (tm + 1) * G / TM; ++l) issue_one(pi, si, l);
        mma(slot, 0, tm, h0);
      }
      decode((slot + 1) % R, 0, h0);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) mma(slot, 1, tm, h1);
      pin_acc();
    };
    for (int i = 0; i < count; i += R) {
#pragma unroll
      for (int u = 0; u < R; ++u)
        if (i + u < count) step(i + u, u);
    }
  }
  wait_vmcnt<0>();   // no global->LDS load may outlive the workgroup's LDS

  // acc[tm][tn][e] is output (m = 16 (mt0 + 4 wm + tm) + 4 j + e,
  // n = n0 + 64 wn + 16 tn + (lane & 15)).
  bool special = false;
#pragma unroll
  for (int tn = 0; tn < kPTN; ++tn) {
    const int n = n0 + wn * 64 + tn * 16 + (lane & 15);
    if (n >= N) continue;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 16 * (mt0 + wm * TM + tm) + 4 * j + e;
        if (m >= M) continue;
        const long long o = static_cast<long long>(m) * N + n;
        const int r = rexp[m];
        if (r == kRowNonfinite) {   // stored by the loop below
          special = true;
          continue;
        }
        const float v = ldexpf(acc[tm][tn][e], r);   // undo the row scale
        if (ks_count == 1) y[o] = v;
        else atomicAdd(y + o, v);
      }
    }
  }
  // Rows holding NaN or +-inf: the reference's f32 form over this K range.
  if (__any(special)) {
#pragma unroll 1
    for (int q = 0; q < kPTN * TM * 4; ++q) {
      const int tn = q / (TM * 4), tm = (q / 4) % TM, e = q % 4;
      const int n = n0 + wn * 64 + tn * 16 + (lane & 15);
      const int m = 16 * (mt0 + wm * TM + tm) + 4 * j + e;
      if (n >= N || m >= M || rexp[m] != kRowNonfinite) continue;
      const float v = nonfinite_blocks_f32<FMT>(W + static_cast<long long>(n) * row_bytes,
                                                x + static_cast<long long>(m) * K, 2 * p0, 2 * p1);
      const long long o = static_cast<long long>(m) * N + n;
      if (ks_count == 1) y[o] = v;
      else atomicAdd(y + o, v);
    }
  }
}

// K ranges of the 2-D GEMM: two (atomic adds onto a cleared y, two addends
// onto zero: order-independent) when both halves' workgroups still run in one
// round at one workgroup per CU, else one.
int panel_split(int m, int n, int k, int cus, int bm) {
  const long long tiles = static_cast<long long>((m + bm - 1) / bm) * ((n + kPBN - 1) / kPBN);
  return 2 * tiles <= cus && k / 64 >= 2 ? 2 : 1;
}

// Route for m >= 64 from two time models fitted on MI355X (q8_0 and q4_0
// alike): a 2-D GEMM workgroup spends ~2.45 us per block pair of its K range
// (MFMA and VALU issue bound, independent of how full the chip is), in
// ceil(workgroups / CUs) rounds; a pass of 32 rows costs max(N K / 2.3e12 s,
// 17 us).  The passes win for small M at small N or long K.
bool panel_pays(int m, int n, int k, int cus) {
  constexpr int bm = PanelStage<kQ8_0, 4>::bm;
  const int ks = panel_split(m, n, k, cus, bm);
  const long long tiles = static_cast<long long>((m + bm - 1) / bm) * ((n + kPBN - 1) / kPBN);
  const long long rounds = (tiles * ks + cus - 1) / cus;
  const double panel = rounds * ((k / 64 + ks - 1) / ks) * 2.45e-6 + 4e-6;
  const double passes = ((m + 31) / 32) * std::max(static_cast<double>(n) * k / 2.3e12, 17e-6);
  return panel < passes;
}

template <int FMT, int TM>
hipError_t run_panel(const uint8_t* W, const float* x, float* y, int m, int n, int k,
                     hipStream_t s, int split, int* rexp, Scratch& scratch) {
  using PS = PanelStage<FMT, TM>;
  if (rexp == nullptr) return hipErrorInvalidValue;   // per-row exponents (see prep_rows)
  const int nb = k / 32, npairs = k / 64;
  const int mblocks = (m + PS::bm - 1) / PS::bm, nblocks = (n + kPBN - 1) / kPBN;
  const int mtiles = mblocks * PS::mt;
  // per-lane 32-bit source offsets within a workgroup's rows
  if (static_cast<long long>(kPBN) * nb * (PairLayout<FMT>::bytes / 2) >= (1LL << 32) ||
      static_cast<long long>(PS::mt) * nb * kFragBytes >= (1LL << 32))
    return hipErrorInvalidValue;
  int ks = panel_split(m, n, k, device_cu_count(), PS::bm);
  if (split == 1 || split == 2) ks = split;
  if (npairs < 2) ks = 1;
  const int per = (npairs + ks - 1) / ks;
  const size_t xf_bytes = static_cast<size_t>(mtiles) * nb * kFragBytes;
  const size_t bias_bytes = FMT == kQ4_0 ? static_cast<size_t>(mtiles) * nb * 64 : 0;
  void* ws = nullptr;
  hipError_t e = scratch.get(s, xf_bytes + bias_bytes + 256, &ws);
  if (e != hipSuccess) return e;
  uint8_t* xf = static_cast<uint8_t*>(ws);
  float* bias = reinterpret_cast<float*>(xf + xf_bytes);
  const long long outs = static_cast<long long>(m) * n;
  prep_rows<true, FMT == kQ4_0>
      <<<static_cast<unsigned>(16 * mtiles + (ks == 2 ? clear_workgroups(outs) : 0)), 256, 0, s>>>(
          x, m, k, nb, 0, xf, bias, rexp, y, ks == 2 ? outs : 0, nullptr, 0, nullptr, 0,
          16 * mtiles);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid(static_cast<unsigned>(nblocks), static_cast<unsigned>(mblocks),
                  static_cast<unsigned>(ks));
  qgemm_panel<FMT, TM><<<grid, 64 * kPWaves, 0, s>>>(W, xf, bias, y, rexp, x, m, n, k, per, ks);
  return hipGetLastError();
}

}  // namespace

namespace {

hipError_t qgemm_mfma_with(int fmt, const void* W, const float* x, float* y, int m, int n, int k,
                           hipStream_t s, int waves, int stages, int panel, Scratch& scratch) {
  const auto* w = static_cast<const uint8_t*>(W);
  // panel: 0 = from the shape (for m >= 64), -1 = never, 1 / 2 = always
  // (for m >= 2) with one / two K ranges
  const bool use_panel = panel > 0 || (panel == 0 && m >= 64 && panel_pays(m, n, k, device_cu_count()));
  // The bf16 layouts (the panel and passes of more than 8 rows) scale each
  // row by its power of two; their prep kernels store the exponents here.
  int* rexp = nullptr;
  if (use_panel || m > 8) {
    void* p = nullptr;
    hipError_t e = scratch.get(s, sizeof(int) * static_cast<size_t>(m) + 256, &p, 1);
    if (e != hipSuccess) return e;
    rexp = static_cast<int*>(p);
  }
  if (use_panel)
    return fmt == kQ8_0 ? run_panel<kQ8_0, 4>(w, x, y, m, n, k, s, panel, rexp, scratch)
                        : run_panel<kQ4_0, 4>(w, x, y, m, n, k, s, panel, rexp, scratch);
  for (int m0 = 0; m0 < m; m0 += 32) {
    const int mt = m - m0 < 32 ? m - m0 : 32;
    const float* xm = x + static_cast<long long>(m0) * k;
    float* ym = y + static_cast<long long>(m0) * n;
    int* rm = rexp != nullptr ? rexp + m0 : nullptr;
    // activation layout: compact rows for M <= 4 / 8, dense 16-row tiles above
    hipError_t e;
    if (fmt == kQ8_0)
      e = mt <= 4 ? run<kQ8_0, 4>(w, xm, ym, mt, n, k, s, waves, stages, rm, scratch)
        : mt <= 8 ? run<kQ8_0, 8>(w, xm, ym, mt, n, k, s, waves, stages, rm, scratch)
        : mt <= 16 ? run<kQ8_0, 16>(w, xm, ym, mt, n, k, s, waves, stages, rm, scratch)
                   : run<kQ8_0, 32>(w, xm, ym, mt, n, k, s, waves, stages, rm, scratch);
    else
      e = mt <= 4 ? run<kQ4_0, 4>(w, xm, ym, mt, n, k, s, waves, stages, rm, scratch)
        : mt <= 8 ? run<kQ4_0, 8>(w, xm, ym, mt, n, k, s, waves, stages, rm, scratch)
        : mt <= 16 ? run<kQ4_0, 16>(w, xm, ym, mt, n, k, s, waves, stages, rm, scratch)
                   : run<kQ4_0, 32>(w, xm, ym, mt, n, k, s, waves, stages, rm, scratch);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_qgemm_mfma(int fmt, const void* W, const float* x, float* y, int m, int n,
                             int k, hipStream_t s, int waves, int stages, int panel, int fold) {
  StreamWorkspace* ws = nullptr;
  const hipError_t e = stream_workspace(s, &ws);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> hold(ws->call);   // until the call's last launch
  Scratch scratch;
  scratch.w = ws;
  scratch.fold = fold;
  return qgemm_mfma_with(fmt, W, x, y, m, n, k, s, waves, stages, panel, scratch);
}


// ------------------------------------------- scratch that is never allocated ---
//
// For callers that cannot allocate (graph capture, serving loops): the
// qgemm scratch lives in this file-scope device array, one copy per GPU,
// held until the process ends.  Host code uses the address that
// hipGetSymbolAddress returns for the current device (the array's name is
// only a host-side handle).  Every no-allocation call on a GPU shares that
// GPU's array.  A per-device host mutex is held from a call's first launch to
// its last, so calls from several host threads on one stream queue their
// launch sequences one after the other; calls on different streams of one GPU
// can still overlap on the device and race.  Nothing in it has to start at
// zero: each call's prep kernels write every byte its GEMM kernels read.
static __device__ __align__(256) uint8_t noalloc_scratch[kQgemmNoAllocScratchBytes];

struct NoAllocDevice {
  void* base = nullptr;   // hipGetSymbolAddress of noalloc_scratch on this device
  std::mutex call;        // held by one call's launch sequence
};

static hipError_t noalloc_device(NoAllocDevice** out) {
  static std::mutex mu;
  static std::vector<std::unique_ptr<NoAllocDevice>> devices;   // [device], resolved once
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  if (static_cast<int>(devices.size()) <= dev) devices.resize(dev + 1);
  if (devices[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch));
    if (e != hipSuccess) return e;
    devices[dev].reset(new NoAllocDevice);
    devices[dev]->base = p;
  }
  *out = devices[dev].get();
  return hipSuccess;
}

hipError_t launch_qgemm_mfma_noalloc(int fmt, const void* W, const float* x, float* y, int m,
                                     int n, int k, hipStream_t s) {
  NoAllocDevice* d = nullptr;
  const hipError_t e = noalloc_device(&d);
  if (e != hipSuccess) return e;
  Scratch scratch;
  scratch.fixed = static_cast<uint8_t*>(d->base);
  // region 1: the row exponents; region 0: one pass's fragments and partials
  scratch.fixed_split = (sizeof(int) * static_cast<size_t>(m) + 256 + 255) / 256 * 256;
  scratch.fixed_bytes = kQgemmNoAllocScratchBytes;
  scratch.max_ks = 2;
  if (scratch.fixed_split >= scratch.fixed_bytes) return hipErrorOutOfMemory;
  std::lock_guard<std::mutex> hold(d->call);   // until the call's last launch
  // passes of at most 32 rows: the panel route's fragments grow with m
  return qgemm_mfma_with(fmt, W, x, y, m, n, k, s, 0, 0, -1, scratch);
}

}  // namespace qc
