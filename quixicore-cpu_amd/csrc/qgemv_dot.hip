// q8_0 / q4_0 decode GEMV (M = 1) on gfx950 with exact int8 dot products.
//
// Semantics: y[n] = sum_k dequant(W)[n][k] * x[k] with f32 activations
// (include/quixicore_cpu/qgemv.h:100-108, src/dispatch/qgemv.cpp:337-365 of
// the reference), within the contract tolerance |y - y64| <= 1e-4 *
// ||x||_2 * ||w_hat_row||_2 of the f64 oracle.
//
// Numerical method.  For every 32-element block b of x the workgroup picks the
// power of two 2^e_b with max|x_b| < 2^(e_b + 21) (e_b = frexp exponent - 21)
// and the integers q_j = rint(x_j * 2^-e_b), clamped to [-2^21, 2^21 - 1],
// split into three int8 digits (floor division):
//   q_j = 2^14 * d0_j + 2^7 * d1_j + d2_j,  d0 in [-128,127], d1, d2 in [0,127].
// So x_j = 2^e_b * q_j + err_j with |err_j| <= 2^(e_b-1) <= max|x_b| * 2^-21
// (2^-20 where the clamp applies): a 22-bit fixed-point copy of the block
// whose error, after the contract's normalisation by ||x||_2 ||w_hat_row||_2
// (Cauchy-Schwarz over blocks), is at most sqrt(32) * 2^-20 = 5.4e-6 and
// ~1e-8 typically.  Scaling by 2^-e_b is exact (v_ldexp), so subnormal and
// huge activations keep their precision.  Each block dot is then three exact
// int32 sums of int8 x int8 products (v_dot4_i32_i8, 4 MACs per instruction):
//   sum_j w_j x_j ~= 2^e_b * d_w * (2^14 S0 + 2^7 S1 + S2),  S_t = sum_j c_j d_t,j
// with c_j the q8_0 code, or the q4_0 nibble n_j with the -8 offset folded in
// exactly as S_t -= 8 * sum_j d_t,j.  When x holds NaN or +-inf, every row is
// recomputed after the main loop in the reference's f32 form (row_f32), which
// gives each output the reference's inf or NaN.  Blocks are accumulated in f32 in a fixed per-lane order
// and reduced across the wave in a fixed butterfly, so results are
// deterministic.
//
// Memory: W stays in the canonical GGUF layout.  Lane l owns the block pairs
// p = l, l+64, ... of its wave's rows (a pair is 68 B for q8_0, 36 B for q4_0,
// dword aligned when K/32 is even).  Each wave issues its first weight loads
// before anything else, so they are in flight while the workgroup builds the
// digits of x in LDS (the barrier after the digit build waits on LDS traffic
// only), and then keeps a small window of (pair, row) items in flight ahead
// of the one it computes.
#include <algorithm>

#include "qc_device.h"
#include "qc_digits.h"
#include "qc_internal.h"

namespace qc {
namespace {

// x values of this thread's half-blocks (16 elements each) of a chunk:
// h = threadIdx.x + NT j, j < HPT.  Issued before the weight loads so that
// waiting for them does not wait for the weights (vmcnt retires in order).
// Branch-free (an index past the chunk re-reads its last half-block, which
// build_digits then skips): a branch around the loads would make the compiler
// wait for them at the join, before the weight loads are issued.
template <int HPT, int NT, bool VEC>
__device__ __forceinline__ void load_x(float (&v)[HPT][16], const float* __restrict__ x, int clen) {
  const int nh = clen >> 4;
#pragma unroll
  for (int j = 0; j < HPT; ++j) {
    const int h = min(static_cast<int>(threadIdx.x) + NT * j, nh - 1);
    if constexpr (VEC) {
      const float4* src = reinterpret_cast<const float4*>(x + 16 * h);
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<float4*>(&v[j][4 * i]) = src[i];
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[j][i] = x[16 * h + i];
    }
  }
}

// Digits of the loaded half-blocks into LDS.
template <bool WITH_SUMS, int HPT, int NT>
__device__ __forceinline__ void build_digits(uint8_t* lds, const float (&xv)[HPT][16], int clen,
                                             int kc) {
  const int nh = clen >> 4;
#pragma unroll
  for (int j = 0; j < HPT; ++j) {
    const int h = threadIdx.x + NT * j;
    if (h >= nh) break;
    build_half<WITH_SUMS>(lds, xv[j], h, kc);
  }
}

// acc + 2^e * (d_w * gate) * (2^14 s0 + 2^7 s1 + s2)
__device__ __forceinline__ float block_acc(float acc, uint32_t dbits, float gate, int e, int s0,
                                           int s1, int s2) {
  const float t = (half_bits_to_float(dbits) * gate) * combine(s0, s1, s2);
  return acc + ldexpf(t, e);
}

// One row's sum over this lane's block pairs p = lane (mod 64) in f32, from
// memory: sum_b d_b * sum_j q_j x_j as the reference forms it
// (kernels/quantization/qgemv_ref.cpp:62-80).  Used for the rows whose x
// holds NaN or +-inf: every output of such an activation row is +-inf or
// NaN, set by its non-finite products alone, and this gives the reference's
// class (the digit path would give NaN throughout).  Rare, so a rolled loop
// after the main one, which keeps it out of the fast loop's code.
template <int FMT>
__device__ __forceinline__ float row_f32(const uint8_t* wrow, const float* x, int k, int lane) {
  constexpr int BB = Fmt<FMT>::block_bytes;
  float acc = 0.0f;
#pragma unroll 1
  for (int p = lane; p < (k >> 6); p += 64) {
    const uint8_t* wp = wrow + static_cast<long long>(p) * (2 * BB);
    const uint16_t d0 = *reinterpret_cast<const uint16_t*>(wp);
    const uint16_t d1 = *reinterpret_cast<const uint16_t*>(wp + BB);
    acc += half_bits_to_float(d0) * block_f32<FMT>(wp, 0, x + 64LL * p);
    acc += half_bits_to_float(d1) * block_f32<FMT>(wp, 1, x + 64LL * p + 32);
  }
  return acc;
}

// True when a block of the pair holds a non-finite value of x (gate NaN).
__device__ __forceinline__ bool pair_special(const PairDigits& g) {
  return !(g.gate[0] == 1.0f && g.gate[1] == 1.0f);
}

// acc += contribution of one pair (two blocks) of one row.
template <int FMT>
__device__ __forceinline__ float pair_dot(const uint32_t* w, const PairDigits& g, float acc) {
  if constexpr (FMT == kQ8_0) {
    int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = static_cast<int>(__builtin_amdgcn_alignbyte(w[i + 1], w[i], 2));
      a0 = __builtin_amdgcn_sdot4(c, static_cast<int>(g.d[0][i]), a0, false);
      a1 = __builtin_amdgcn_sdot4(c, static_cast<int>(g.d[1][i]), a1, false);
      a2 = __builtin_amdgcn_sdot4(c, static_cast<int>(g.d[2][i]), a2, false);
      const int e = static_cast<int>(w[9 + i]);
      b0 = __builtin_amdgcn_sdot4(e, static_cast<int>(g.d[0][8 + i]), b0, false);
      b1 = __builtin_amdgcn_sdot4(e, static_cast<int>(g.d[1][8 + i]), b1, false);
      b2 = __builtin_amdgcn_sdot4(e, static_cast<int>(g.d[2][8 + i]), b2, false);
    }
    acc = block_acc(acc, w[0] & 0xFFFFu, g.gate[0], g.e[0], a0, a1, a2);
    acc = block_acc(acc, w[8] >> 16, g.gate[1], g.e[1], b0, b1, b2);
  } else {
    int a0 = g.off[0][0], a1 = g.off[0][1], a2 = g.off[0][2];
    int b0 = g.off[1][0], b1 = g.off[1][1], b2 = g.off[1][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
      const int lo = static_cast<int>(q & 0x0F0F0F0Fu);
      const int hi = static_cast<int>((q >> 4) & 0x0F0F0F0Fu);
      a0 = __builtin_amdgcn_sdot4(lo, static_cast<int>(g.d[0][i]), a0, false);
      a1 = __builtin_amdgcn_sdot4(lo, static_cast<int>(g.d[1][i]), a1, false);
      a2 = __builtin_amdgcn_sdot4(lo, static_cast<int>(g.d[2][i]), a2, false);
      a0 = __builtin_amdgcn_sdot4(hi, static_cast<int>(g.d[0][4 + i]), a0, false);
      a1 = __builtin_amdgcn_sdot4(hi, static_cast<int>(g.d[1][4 + i]), a1, false);
      a2 = __builtin_amdgcn_sdot4(hi, static_cast<int>(g.d[2][4 + i]), a2, false);
      const uint32_t u = w[5 + i];
      const int lo1 = static_cast<int>(u & 0x0F0F0F0Fu);
      const int hi1 = static_cast<int>((u >> 4) & 0x0F0F0F0Fu);
      b0 = __builtin_amdgcn_sdot4(lo1, static_cast<int>(g.d[0][8 + i]), b0, false);
      b1 = __builtin_amdgcn_sdot4(lo1, static_cast<int>(g.d[1][8 + i]), b1, false);
      b2 = __builtin_amdgcn_sdot4(lo1, static_cast<int>(g.d[2][8 + i]), b2, false);
      b0 = __builtin_amdgcn_sdot4(hi1, static_cast<int>(g.d[0][12 + i]), b0, false);
      b1 = __builtin_amdgcn_sdot4(hi1, static_cast<int>(g.d[1][12 + i]), b1, false);
      b2 = __builtin_amdgcn_sdot4(hi1, static_cast<int>(g.d[2][12 + i]), b2, false);
    }
    acc = block_acc(acc, w[0] & 0xFFFFu, g.gate[0], g.e[0], a0, a1, a2);
    acc = block_acc(acc, w[4] >> 16, g.gate[1], g.e[1], b0, b1, b2);
  }
  return acc;
}

template <int FMT>
__device__ __forceinline__ void load_pair(uint32_t* d, const uint8_t* p) {
  const u32x4_a4* v = reinterpret_cast<const u32x4_a4*>(p);
  constexpr int NV = FMT == kQ8_0 ? 4 : 2;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const u32x4_a4 t = v[i];
    d[4 * i] = t.x; d[4 * i + 1] = t.y; d[4 * i + 2] = t.z; d[4 * i + 3] = t.w;
  }
  d[4 * NV] = reinterpret_cast<const uint32_t*>(p)[4 * NV];
}

// Row space of one launch: up to three weight matrices with their outputs,
// concatenated (logical row g of segment s is row g - start[s] of w[s]), or,
// with act >= 0, up (even logical rows) and gate (odd) of one row index
// interleaved, stored as out[i] = activation(gate[i]) * up[i] (act 0: SiLU,
// 1: GELU-tanh; kernels/quantization/qgemv_fused_ref.cpp:184-192).  The same
// x is shared by every row.
//
// RoPE (half > 0, kernels/quantization/qgemv_fused_ref.cpp:342-443): in the
// first nrope segments, logical rows 2j and 2j + 1 are rows d and d + half of
// head h (j = h * half + d) of that matrix, and the pair is stored rotated:
// out[d] = a * cos[d] - b * sin[d], out[d + half] = b * cos[d] + a * sin[d]
// for the head's rows a = row d, b = row d + half (rc / rs: the position's
// cos / sin rows, half values each).
struct GemvSegs {
  const uint8_t* w[3];
  float* y[3];
  int start[4];    // start[nseg] = total logical rows
  int nseg;
  int act;         // -1: plain segments
  int half;        // > 0: RoPE pairs in segments [0, nrope); head_dim = 2 * half
  int nrope;
  const float* rc;
  const float* rs;
};

// Weight row of logical row `local` of a RoPE segment.
__device__ __forceinline__ int rope_row(int local, int half) {
  const int j = local >> 1;
  const int head = j / half;
  return head * 2 * half + (j - head * half) + (local & 1) * half;
}

__device__ __forceinline__ float fused_activation(float v, int act) {
  constexpr float kSqrt2OverPi = 0.7978845608028654f;
  return act == 1 ? 0.5f * v * (1.0f + tanhf(kSqrt2OverPi * (v + 0.044715f * v * v * v)))
                  : v / (1.0f + expf(-v));
}

// Whole-line items: an item (64 consecutive block pairs of one row, one pair
// per lane: 2304 bytes for q4_0, 4352 for q8_0) is read as 2 or 4 16-byte
// chunks per lane, contiguous across the wave (lane l takes chunks l + 64 i),
// and a dword per lane for its last 256 bytes, with the non-temporal hint, and
// handed to the lanes through a per-wave LDS staging area, one item at a time.
// A lane's own 36- or 68-byte pair straddles cache lines: per-lane record
// loads keep re-requesting the same lines, and with the hint fetch them twice.
// As many dwords per lane as a record.  Measured on MI355X (same process):
// q4_0 4096 -> 14336 (7 rows per wave) 8.16 -> 7.80 us, q8_0 4096 -> 14336
// 13.0 -> 11.9, 4096 x 4096 5.41 -> 5.12, q8_0 up+gate 24.4 -> 23.4.  Kept on
// records: q4_0 with 1-2 rows per wave (4096 x 4096 4.30 -> 4.37 us, QKV 6.62
// -> 6.75 us that way) and K above 4096 (more than one pair per lane and
// chunk; the staging area then takes LDS that a second workgroup per CU would
// use: q8_0 14336 x 14336 42.5 -> 48.6 us, q4_0 14336 -> 4096 9.5 -> 9.9 us;
// only q8_0 14336 -> 4096, one workgroup per CU either way, gained, 13.8 ->
// 13.0 us).
template <int FMT>
constexpr int item_bytes() { return 128 * Fmt<FMT>::block_bytes; }   // 64 pairs
// 16-byte chunks per lane of an item (2 or 4), then a 256-byte tail of one
// dword per lane: the pair's dwords of a per-lane record
template <int FMT>
constexpr int item_x4() { return item_bytes<FMT>() / 1024; }
static_assert(item_bytes<kQ4_0>() % 1024 == 256 && item_bytes<kQ8_0>() % 1024 == 256,
              "whole chunks and a dword tail per lane");
template <int FMT, int NPM, int RB>
constexpr bool chunked() { return NPM == 1 && (FMT == kQ8_0 || RB >= 4); }
__host__ __device__ constexpr size_t stage_off(int kc) { return (lds_size(kc) + 15) / 16 * 16; }

// The first nbytes (<= item_bytes) of an item at `base` in whole lines:
// chunk i of lane l holds bytes 16 (l + 64 i), the tail dword bytes 1024 X4 +
// 4 l; a lane past nbytes re-reads the item's last bytes, so every lane loads
// and no register waits on a condition.  Lines read once: non-temporal.
template <int FMT>
__device__ __forceinline__ void load_item_lines(uint32_t* w, const uint8_t* base, int nbytes,
                                                int lane) {
  constexpr int IB = item_bytes<FMT>(), X4 = item_x4<FMT>();
  const bool whole = nbytes == IB;   // wave-uniform; a whole item needs no clamping
#pragma unroll
  for (int i = 0; i < X4; ++i) {
    const int off = whole ? 16 * lane + 1024 * i : min(16 * (lane + 64 * i), nbytes - 16);
    const u32x4_a4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(base + off));
    w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
  }
  w[4 * X4] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(
      base + (whole ? 1024 * X4 + 4 * lane : min(1024 * X4 + 4 * lane, nbytes - 4))));
}

// Those bytes into the wave's staging area (lanes then read what other lanes
// stored: wave_lds_sync orders the previous item's reads before these
// stores, and the stores before this item's reads).
template <int FMT>
__device__ __forceinline__ void stage_item(uint8_t* stage, const uint32_t* w, int nbytes,
                                           int lane) {
  constexpr int IB = item_bytes<FMT>(), X4 = item_x4<FMT>();
  wave_lds_sync();
  if (nbytes == IB) {   // a whole item (wave-uniform)
#pragma unroll
    for (int i = 0; i < X4; ++i)
      *reinterpret_cast<u32x4_a4*>(stage + 16 * lane + 1024 * i) =
          u32x4_a4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
    *reinterpret_cast<uint32_t*>(stage + 1024 * X4 + 4 * lane) = w[4 * X4];
  } else {
#pragma unroll
    for (int i = 0; i < X4; ++i) {
      const int off = 16 * (lane + 64 * i);
      if (off < nbytes)
        *reinterpret_cast<u32x4_a4*>(stage + min(off, nbytes - 16)) =
            u32x4_a4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
    }
    if (1024 * X4 + 4 * lane < nbytes)
      *reinterpret_cast<uint32_t*>(stage + 1024 * X4 + 4 * lane) = w[4 * X4];
  }
  wave_lds_sync();
}

// NW wavefronts of RB rows each, up to NPM pairs per lane per K chunk.  The (pair j,
// row r) items of a chunk are loaded in j-major order with at most WIN items
// in flight: item t + WIN is issued just before item t is computed, so the
// data arrive roughly in the order they are used (all at once, when WIN >=
// NPM * RB).  A bounded window keeps a wave from waiting on its first rows
// while the memory system still returns the others, which for several rows
// per wave leaves less compute after the last byte lands.
//
// MULTI false: one matrix (segs.w[0], segs.y[0], segs.start[1] rows).  MULTI
// true: the whole segment table, with the activation epilogue when act >= 0;
// the selection is kept out of the one-matrix kernel, whose prologue and
// epilogue it would lengthen.
template <int FMT, int NW, int RB, int NPM, int WIN, bool VEC, bool MULTI>
__global__ __launch_bounds__(64 * NW) void qgemv_dot_kernel(const GemvSegs segs,
                                                             const float* __restrict__ x, int k,
                                                             int kc) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int BB = Fmt<FMT>::block_bytes;
  constexpr int PD = Fmt<FMT>::pair_dwords;
  constexpr int T = NPM * RB;
  constexpr int NT = 64 * NW;
  constexpr int HPT = (NPM * 256 + NT - 1) / NT;   // half-blocks of x per thread
  constexpr bool CHUNKED = chunked<FMT, NPM, RB>();   // see item_bytes
  constexpr int IB = item_bytes<FMT>();
  const int lane = threadIdx.x & 63;
  const long long row_bytes = static_cast<long long>(k >> 5) * BB;
  const uint8_t* wrow[RB];
  int row0, total;
  if constexpr (!MULTI) {
    total = segs.start[1];
    row0 = (blockIdx.x * NW + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * RB;
#pragma unroll
    for (int r = 0; r < RB; ++r) wrow[r] = segs.w[0] + min(row0 + r, total - 1) * row_bytes;
  } else {
    // the wave index is uniform; saying so keeps the row and segment
    // selection in scalar registers (a per-lane selection indexes the kernel
    // arguments with vector loads, serialised before the first weight load).
    // The table is read into locals and selected by value: indexing the
    // argument array, or taking its address, moves it to scratch.
    row0 = (blockIdx.x * NW + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * RB;
    const uint8_t* const w0 = segs.w[0];
    const uint8_t* const w1 = segs.w[1];
    const uint8_t* const w2 = segs.w[2];
    const int s1 = segs.start[1], s2 = segs.start[2], nseg = segs.nseg, act = segs.act;
    const int half = segs.half, nrope = segs.nrope;
    total = nseg == 1 ? s1 : nseg == 2 ? s2 : segs.start[3];
    const bool three = nseg > 2;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int g = min(row0 + r, total - 1);
      const bool in2 = three && g >= s2, in1 = g >= s1;
      const uint8_t* const base = act >= 0 ? ((g & 1) ? w1 : w0) : in2 ? w2 : in1 ? w1 : w0;
      int local = act >= 0 ? g >> 1 : g - (in2 ? s2 : in1 ? s1 : 0);
      if (half > 0 && (in2 ? 2 : in1 ? 1 : 0) < nrope) local = rope_row(local, half);
      wrow[r] = base + static_cast<long long>(local) * row_bytes;
    }
  }
  float acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = 0.f;
  bool nonfinite = false;   // some block of x is NaN or +-inf (every row's output then is)

  for (int c0 = 0; c0 < k; c0 += kc) {
    const int clen = min(kc, k - c0);
    const int pbeg = c0 >> 6, pend = (c0 + clen) >> 6;
    const int p0 = first_pair(pbeg, lane);
    // 1. this thread's x values, then the first WIN weight items
    float xv[HPT][16];
    load_x<HPT, NT, VEC>(xv, x + c0, clen);
    uint32_t w[T][PD];
    // chunked items: pairs [q0c, q0c + nbytes / (2 BB)) of the row (one
    // clamped pair past the chunk); a chunk that would run past them is moved
    // back to end with them (its overlap rewrites the same bytes)
    auto span = [&](int j, int& q0c, int& nbytes) {
      const int q0 = pbeg + 64 * j;
      q0c = min(q0, pend - 1);
      nbytes = (q0 < pend ? min(64, pend - q0) : 1) * (2 * BB);
    };
    auto issue = [&](int t) {
      const int j = t / RB, r = t % RB;
      if constexpr (CHUNKED) {
        int q0c, nbytes;
        span(j, q0c, nbytes);
        load_item_lines<FMT>(w[t], wrow[r] + static_cast<long long>(q0c) * (2 * BB), nbytes, lane);
      } else {
        const int p = min(p0 + 64 * j, pend - 1);
        load_pair<FMT>(w[t], wrow[r] + static_cast<long long>(p) * (2 * BB));
      }
    };
#pragma unroll
    for (int t = 0; t < T && t < WIN; ++t) issue(t);
    // 2. digits of x for this chunk
    if (c0) lds_barrier();
    build_digits<FMT == kQ4_0, HPT, NT>(lds, xv, clen, kc);
    lds_barrier();
    // 3. exact block dots, issuing the window's next item before each
#pragma unroll
    for (int j = 0; j < NPM; ++j) {
      const int p = p0 + 64 * j;
      PairDigits g;
      read_digits<FMT>(g, lds, min(p, pend - 1) - pbeg, kc);
      nonfinite = nonfinite || __any(p < pend && pair_special(g));
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int t = j * RB + r;
        if (t + WIN < T) issue(t + WIN);
        if constexpr (CHUNKED) {
          // the item's bytes into the wave's staging area, then this lane's pair
          // (lanes read what other lanes stored: wave_lds_sync orders the
          // previous item's reads before these stores, and the stores before
          // this item's reads)
          uint8_t* const stage = lds + stage_off(kc) + (threadIdx.x >> 6) * IB;
          int q0c, nbytes;
          span(j, q0c, nbytes);
          stage_item<FMT>(stage, w[t], nbytes, lane);
          const uint32_t* rec =
              reinterpret_cast<const uint32_t*>(stage + (min(p, pend - 1) - q0c) * (2 * BB));
          if (p < pend) acc[r] = pair_dot<FMT>(rec, g, acc[r]);
        } else {
          if (p < pend) acc[r] = pair_dot<FMT>(w[t], g, acc[r]);
        }
      }
    }
  }
  // x held NaN or +-inf (wave-uniform, rare): the reference's f32 form
  if (nonfinite) {
#pragma unroll
    for (int r = 0; r < RB; ++r) acc[r] = row_f32<FMT>(wrow[r], x, k, lane);
  }
  if constexpr (!MULTI) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const float t = wave_sum_lane63(acc[r]);
      if (lane == 63 && row0 + r < total) segs.y[0][row0 + r] = t;
    }
  } else {
    float t[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) t[r] = wave_sum_lane63(acc[r]);
    if (lane != 63) return;
    const int s1 = segs.start[1], s2 = segs.start[2], act = segs.act;
    const bool three = segs.nseg > 2;
    float* const y0 = segs.y[0];
    float* const y1 = segs.y[1];
    float* const y2 = segs.y[2];
    if (act >= 0) {
      // RB is even and row0 even: rows (2i, 2i+1) = (up, gate) of row index i
#pragma unroll
      for (int r = 0; r + 1 < RB; r += 2)
        if (row0 + r < total) y0[(row0 + r) >> 1] = fused_activation(t[r + 1], act) * t[r];
      return;
    }
    const int half = segs.half;
    if (half > 0) {
      // RB, row0 and every segment start are even: rows (2j, 2j+1) are one
      // (d, d + half) pair of a RoPE segment, or two rows of a plain one
      const int nrope = segs.nrope;
#pragma unroll
      for (int r = 0; r + 1 < RB; r += 2) {
        const int g = row0 + r;
        if (g >= total) continue;
        const bool in2 = three && g >= s2, in1 = g >= s1;
        float* const out = in2 ? y2 : in1 ? y1 : y0;
        const int local = g - (in2 ? s2 : in1 ? s1 : 0);
        if ((in2 ? 2 : in1 ? 1 : 0) < nrope) {
          const int j = local >> 1;
          const int head = j / half;
          const int d = j - head * half;
          const float c = segs.rc[d], sn = segs.rs[d];
          const float a = t[r], b = t[r + 1];
          out[head * 2 * half + d] = a * c - b * sn;
          out[head * 2 * half + d + half] = b * c + a * sn;
        } else {
          out[local] = t[r];
          out[local + 1] = t[r + 1];
        }
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int g = row0 + r;
      if (g >= total) continue;
      const bool in2 = three && g >= s2, in1 = g >= s1;
      float* const out = in2 ? y2 : in1 ? y1 : y0;
      out[g - (in2 ? s2 : in1 ? s1 : 0)] = t[r];
    }
  }
}

// For the rows kernel, after its main loop, when some activation row in
// `mask` held a non-finite x value: the outputs of those activation rows for
// weight rows [row0, row0 + rb) are stored again in the reference's f32 form
// (qgemv's own row_f32 and reduction, so each stays bit-identical to qgemv of
// its row).  Out of line and called after the main loop, so the loop keeps
// its code and registers.
template <int FMT>
__device__ __noinline__ void rows_fix_group(const uint8_t* W, const float* x, float* y, int n,
                                            int k, int mb, int row0, int rb, uint32_t mask) {
  const int lane = threadIdx.x & 63;
  const long long row_bytes = static_cast<long long>(k >> 5) * Fmt<FMT>::block_bytes;
  for (int mm = 0; mm < mb; ++mm) {
    if (!((mask >> mm) & 1u)) continue;
    for (int r = 0; r < rb; ++r) {
      const uint8_t* wr = W + static_cast<long long>(min(row0 + r, n - 1)) * row_bytes;
      const float t = wave_sum_lane63(row_f32<FMT>(wr, x + static_cast<long long>(mm) * k, k, lane));
      if (lane == 63 && row0 + r < n) y[static_cast<long long>(mm) * n + row0 + r] = t;
    }
  }
}

// ------------------------------------------------------- small-batch rows
// qgemm for a few activation rows (kernels/quantization/qgemm_ref.cpp:
// 141-164: each row of y is the qgemv of that row of x).  The GEMV's method
// and lane mapping per row -- lane l owns pairs p = l (mod 64) in increasing
// order, the same digits, pair dots and wave reduction -- so every output is
// bit-identical to qc_hip_qgemv of its activation row.  MB activation rows
// share one pass over W: a workgroup builds the digits of all MB rows of a
// chunk of kc = 4096 columns in LDS (MB records of lds_size(kc)), and each of
// its waves runs every pair of its RB weight rows against the MB digit sets.
//
// When the whole K fits one chunk the grid is persistent: workgroup b builds
// the digits once and then takes row groups b, b + gridDim.x, ... (NW * RB
// rows each), with the next group's weights in flight while the current one
// is computed.  Otherwise each workgroup takes one row group and rebuilds the
// digits per chunk.  Rows of x past m are masked (their outputs not stored).
template <int FMT, int NW, int RB, int MB, bool VEC>
__global__ __launch_bounds__(64 * NW) void qgemm_rows_kernel(const uint8_t* __restrict__ W,
                                                             const float* __restrict__ x,
                                                             float* __restrict__ y, int n, int k,
                                                             int m, int kc) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int BB = Fmt<FMT>::block_bytes;
  constexpr int PD = Fmt<FMT>::pair_dwords;
  constexpr int NT = 64 * NW;
  constexpr int HB = 256;                          // half-blocks per row and chunk (kc <= 4096)
  constexpr int IPT = (MB * HB + NT - 1) / NT;     // (row, half-block) items per thread
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const long long row_bytes = static_cast<long long>(k >> 5) * BB;
  const size_t lsz = lds_size(kc);
  const int groups = (n + NW * RB - 1) / (NW * RB);
  const bool single = k <= kc;

  // digits of chunk [c0, c0 + clen) of every activation row into LDS
  auto build = [&](int c0, int clen) {
    const int nh = clen >> 4;
    float xv[IPT][16];
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int item = threadIdx.x + NT * j;
      const int r = min(item / HB, m - 1);
      const int h = min(item % HB, nh - 1);
      const float* src = x + static_cast<long long>(r) * k + c0 + 16 * h;
      if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<float4*>(&xv[j][4 * i]) = reinterpret_cast<const float4*>(src)[i];
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) xv[j][i] = src[i];
      }
    }
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int item = threadIdx.x + NT * j;
      const int r = item / HB, h = item % HB;
      if (r < MB && r < m && h < nh) build_half<FMT == kQ4_0>(lds + r * lsz, xv[j], h, kc);
    }
  };

  auto rows_of = [&](int g, const uint8_t** wrow) {
    const int row0 = (g * NW + wave) * RB;
#pragma unroll
    for (int r = 0; r < RB; ++r)
      wrow[r] = W + static_cast<long long>(min(row0 + r, n - 1)) * row_bytes;
    return row0;
  };

  auto store = [&](int row0, float (&acc)[RB][MB]) {
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int mm = 0; mm < MB; ++mm) {
        const float t = wave_sum_lane63(acc[r][mm]);
        if (lane == 63 && row0 + r < n && mm < m) y[static_cast<long long>(mm) * n + row0 + r] = t;
      }
  };

  // Bit mm: some lane's pair of activation row mm holds a non-finite x value
  // in the chunk just built (wave-uniform; rows past m have no digits).
  auto slow_rows = [&](int pend, int pbeg) {
    const int p = first_pair(pbeg, lane);
    const int pl = min(p, pend - 1) - pbeg;
    uint32_t mask = 0;
#pragma unroll
    for (int mm = 0; mm < MB; ++mm) {
      const float2 gv = *reinterpret_cast<const float2*>(lds + mm * lsz + gate_off(kc) + 8 * pl);
      const bool sp = p < pend && mm < m && !(gv.x == 1.0f && gv.y == 1.0f);
      if (__any(sp)) mask |= 1u << mm;
    }
    return mask;
  };
  auto fix_group = [&](uint32_t mask, int g) {
    rows_fix_group<FMT>(W, x, y, n, k, MB, (g * NW + wave) * RB, RB, mask);
  };

  if (single) {
    // one chunk: digits once, then a stream of row groups; two register sets
    // of weights alternate (statically, so neither leaves registers): one is
    // computed while the next group's loads fill the other
    uint32_t badbits = 0;   // bit mm: this lane's pair of row mm holds a non-finite x
    const int pend = k >> 6;
    const int p = lane;                            // this lane's only pair
    const int G = gridDim.x;
    uint32_t wa[RB][PD], wb[RB][PD];
    auto issue = [&](uint32_t (&w)[RB][PD], int g) {
      const uint8_t* wr[RB];
      rows_of(min(g, groups - 1), wr);
#pragma unroll
      for (int r = 0; r < RB; ++r)
        load_pair<FMT>(w[r], wr[r] + static_cast<long long>(min(p, pend - 1)) * (2 * BB));
    };
    auto compute = [&](const uint32_t (&w)[RB][PD], int g) {
      const uint8_t* wr[RB];
      const int row0 = rows_of(g, wr);
      float acc[RB][MB];
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int mm = 0; mm < MB; ++mm) acc[r][mm] = 0.f;
      if (p < pend) {
#pragma unroll
        for (int mm = 0; mm < MB; ++mm) {
          PairDigits dg;
          read_digits<FMT>(dg, lds + mm * lsz, p, kc);
          badbits |= pair_special(dg) ? 1u << mm : 0u;
#pragma unroll
          for (int r = 0; r < RB; ++r) acc[r][mm] = pair_dot<FMT>(w[r], dg, acc[r][mm]);
        }
      }
      store(row0, acc);
    };
    int g = blockIdx.x;
    issue(wa, g);
    build(0, k);
    lds_barrier();
    for (; g < groups; g += 2 * G) {
      if (g + G < groups) issue(wb, g + G);
      compute(wa, g);
      if (g + G >= groups) break;
      if (g + 2 * G < groups) issue(wa, g + 2 * G);
      compute(wb, g + G);
    }
    // did any lane meet a non-finite x value (rows past m have no digits)?
    uint32_t slowmask = 0;
#pragma unroll
    for (int mm = 0; mm < MB; ++mm)
      if (mm < m && __any((badbits >> mm) & 1u)) slowmask |= 1u << mm;
    if (slowmask != 0) {
#pragma unroll 1
      for (int gg = blockIdx.x; gg < groups; gg += G) fix_group(slowmask, gg);
    }
    return;
  }

  // several chunks: one row group per workgroup, digits rebuilt per chunk
  uint32_t slowmask = 0;
  const uint8_t* wrow[RB];
  const int row0 = rows_of(blockIdx.x, wrow);
  float acc[RB][MB];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int mm = 0; mm < MB; ++mm) acc[r][mm] = 0.f;
  for (int c0 = 0; c0 < k; c0 += kc) {
    const int clen = min(kc, k - c0);
    const int pbeg = c0 >> 6, pend = (c0 + clen) >> 6;
    const int p = first_pair(pbeg, lane);
    uint32_t w[RB][PD];
#pragma unroll
    for (int r = 0; r < RB; ++r) load_pair<FMT>(w[r], wrow[r] + static_cast<long long>(min(p, pend - 1)) * (2 * BB));
    if (c0) lds_barrier();
    build(c0, clen);
    lds_barrier();
    if (p < pend) {
#pragma unroll
      for (int mm = 0; mm < MB; ++mm) {
        PairDigits dg;
        read_digits<FMT>(dg, lds + mm * lsz, p - pbeg, kc);
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[r][mm] = pair_dot<FMT>(w[r], dg, acc[r][mm]);
      }
    }
    slowmask |= slow_rows(pend, pbeg);
  }
  store(row0, acc);
  if (slowmask != 0) fix_group(slowmask, blockIdx.x);
}

// ------------------------------------------------------------ qgemv_w8a8
// Activation-quantizing GEMV (src/dispatch/qgemv_w8a8.cpp:130-153;
// kernels/quantization/qgemv_w8a8_ref.cpp:18-41,120-177).  The workgroup
// quantizes each 32-element block of x exactly as the reference does
// (max = fmax(max, |x|), scale = max / 127, inverse = scale != 0 ? 1 / scale
// : 0, code = clamp(rint(x * inverse), -127, 127)) into LDS; each block dot
// is an exact int32 sum of v_dot4_i32_i8 (q4_0: nibbles, with the -8 folded
// in as -8 * the block's code sum); each block's term (float(dot) * d_w) *
// d_x goes to LDS, and one lane per row adds the terms in block order,
// sum = sum + term, as the reference's row loop does -- so y is bit-identical
// to the reference's.  Weights are read with the GEMV's pair-per-lane loads
// and load window.

constexpr int kW8Rec = 80;   // LDS bytes per pair: 64 codes, then {d_x0, d_x1, s_0, s_1}

// LDS layout of one chunk of kc elements: [kc/64 pair records]
// [NW waves][RB rows][kc/32 f32 block terms].
__host__ __device__ constexpr size_t w8_terms_off(int kc) {
  return static_cast<size_t>(kc / 64) * kW8Rec;
}
__host__ __device__ constexpr size_t w8_lds_size(int kc, int nw, int rb) {
  return w8_terms_off(kc) + static_cast<size_t>(nw) * rb * (kc / 32) * 4;
}
// the per-wave staging areas of whole-line items follow
__host__ __device__ constexpr size_t w8_stage_off(int kc, int nw, int rb) {
  return (w8_lds_size(kc, nw, rb) + 15) / 16 * 16;
}

// Codes, scales and (q4_0) code sums of the loaded half-blocks into LDS; the
// two halves of a block sit in lanes t and t^1.  A block holding NaN or
// +-inf gets d_x = NaN (its terms, hence its rows, become NaN) and sets
// *status = 3.
template <bool WITH_SUMS, int HPT, int NT>
__device__ __forceinline__ void build_codes(uint8_t* lds, const float (&xv)[HPT][16], int clen,
                                            int* status) {
  const int nh = clen >> 4;
#pragma unroll
  for (int j = 0; j < HPT; ++j) {
    const int h = threadIdx.x + NT * j;
    if (h >= nh) break;
    const float* v = xv[j];
    float m = 0.f;
    bool finite = true;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      m = fmaxf(m, fabsf(v[i]));
      finite = finite && isfinite(v[i]);
    }
    m = fmaxf(m, xor1_f32(m));
    finite = finite && (xor1_i32(finite ? 1 : 0) != 0);
    const float scale = m / 127.0f;
    const float inverse = scale != 0.0f ? 1.0f / scale : 0.0f;
    int c[16];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float r = rintf(v[i] * inverse);
      r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
      c[i] = finite ? static_cast<int>(r) : 0;
      sum += c[i];
    }
    uint8_t* rec = lds + (h >> 2) * kW8Rec;
    uint4 q;
    q.x = pack4(c[0], c[1], c[2], c[3]);    q.y = pack4(c[4], c[5], c[6], c[7]);
    q.z = pack4(c[8], c[9], c[10], c[11]);  q.w = pack4(c[12], c[13], c[14], c[15]);
    *reinterpret_cast<uint4*>(rec + (h & 3) * 16) = q;
    if constexpr (WITH_SUMS) sum += xor1_i32(sum);
    if ((h & 1) == 0) {
      const int blk = (h >> 1) & 1;
      reinterpret_cast<float*>(rec + 64)[blk] = finite ? scale : __builtin_nanf("");
      if constexpr (WITH_SUMS) reinterpret_cast<int*>(rec + 72)[blk] = sum;
    }
    if (!finite && status != nullptr) *status = 3;
  }
}

// The two block terms (float(dot) * d_w) * d_x of one pair of one row.
template <int FMT>
__device__ __forceinline__ void pair_terms(const uint32_t* w, const uint32_t (&cx)[16],
                                           const float4& meta, float& t0, float& t1) {
  int a, b;
  if constexpr (FMT == kQ8_0) {
    a = 0;
    b = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = static_cast<int>(__builtin_amdgcn_alignbyte(w[i + 1], w[i], 2));
      a = __builtin_amdgcn_sdot4(c, static_cast<int>(cx[i]), a, false);
      b = __builtin_amdgcn_sdot4(static_cast<int>(w[9 + i]), static_cast<int>(cx[8 + i]), b, false);
    }
  } else {
    a = -8 * __float_as_int(meta.z);
    b = -8 * __float_as_int(meta.w);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
      a = __builtin_amdgcn_sdot4(static_cast<int>(q & 0x0F0F0F0Fu), static_cast<int>(cx[i]), a, false);
      a = __builtin_amdgcn_sdot4(static_cast<int>((q >> 4) & 0x0F0F0F0Fu), static_cast<int>(cx[4 + i]), a, false);
      const uint32_t u = w[5 + i];
      b = __builtin_amdgcn_sdot4(static_cast<int>(u & 0x0F0F0F0Fu), static_cast<int>(cx[8 + i]), b, false);
      b = __builtin_amdgcn_sdot4(static_cast<int>((u >> 4) & 0x0F0F0F0Fu), static_cast<int>(cx[12 + i]), b, false);
    }
  }
  const uint32_t d1 = FMT == kQ8_0 ? (w[8] >> 16) : (w[4] >> 16);
  t0 = (static_cast<float>(a) * half_bits_to_float(w[0] & 0xFFFFu)) * meta.x;
  t1 = (static_cast<float>(b) * half_bits_to_float(d1)) * meta.y;
}

template <int FMT, int NW, int RB, int NPM, int WIN, bool VEC>
__global__ __launch_bounds__(64 * NW) void qgemv_w8a8_kernel(const uint8_t* __restrict__ W,
                                                             const float* __restrict__ x,
                                                             float* __restrict__ y, int n, int k,
                                                             int kc, int* status) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int BB = Fmt<FMT>::block_bytes;
  constexpr int PD = Fmt<FMT>::pair_dwords;
  constexpr int T = NPM * RB;
  constexpr int NT = 64 * NW;
  constexpr int HPT = (NPM * 256 + NT - 1) / NT;
  constexpr bool CHUNKED = chunked<FMT, NPM, RB>();   // whole-line items, as in qgemv_dot_kernel
  constexpr int IB = item_bytes<FMT>();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * NW + wave) * RB;
  const long long row_bytes = static_cast<long long>(k >> 5) * BB;
  const uint8_t* wrow[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) wrow[r] = W + min(row0 + r, n - 1) * row_bytes;
  float* terms = reinterpret_cast<float*>(lds + w8_terms_off(kc)) + wave * RB * (kc >> 5);
  float total = 0.f;   // lane r < RB: the block-order sum of row row0 + r

  for (int c0 = 0; c0 < k; c0 += kc) {
    const int clen = min(kc, k - c0);
    const int pbeg = c0 >> 6, pend = (c0 + clen) >> 6;
    const int p0 = first_pair(pbeg, lane);
    float xv[HPT][16];
    load_x<HPT, NT, VEC>(xv, x + c0, clen);
    uint32_t w[T][PD];
    // chunked items: pairs [q0c, q0c + nbytes / (2 BB)) of the row
    auto span = [&](int j, int& q0c, int& nbytes) {
      const int q0 = pbeg + 64 * j;
      q0c = min(q0, pend - 1);
      nbytes = (q0 < pend ? min(64, pend - q0) : 1) * (2 * BB);
    };
    auto issue = [&](int t) {
      const int j = t / RB, r = t % RB;
      if constexpr (CHUNKED) {
        int q0c, nbytes;
        span(j, q0c, nbytes);
        load_item_lines<FMT>(w[t], wrow[r] + static_cast<long long>(q0c) * (2 * BB), nbytes, lane);
      } else {
        const int p = min(p0 + 64 * j, pend - 1);
        load_pair<FMT>(w[t], wrow[r] + static_cast<long long>(p) * (2 * BB));
      }
    };
#pragma unroll
    for (int t = 0; t < T && t < WIN; ++t) issue(t);
    if (c0) lds_barrier();
    build_codes<FMT == kQ4_0, HPT, NT>(lds, xv, clen, status);
    lds_barrier();
#pragma unroll
    for (int j = 0; j < NPM; ++j) {
      const int p = p0 + 64 * j;
      const uint8_t* rec = lds + (min(p, pend - 1) - pbeg) * kW8Rec;
      uint32_t cx[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 v = reinterpret_cast<const uint4*>(rec)[i];
        cx[4 * i] = v.x; cx[4 * i + 1] = v.y; cx[4 * i + 2] = v.z; cx[4 * i + 3] = v.w;
      }
      const float4 meta = *reinterpret_cast<const float4*>(rec + 64);
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int t = j * RB + r;
        if (t + WIN < T) issue(t + WIN);
        uint32_t wl[PD];   // this lane's pair (chunked: restaged through LDS)
        if constexpr (CHUNKED) {
          uint8_t* const stage = lds + w8_stage_off(kc, NW, RB) + wave * IB;
          int q0c, nbytes;
          span(j, q0c, nbytes);
          stage_item<FMT>(stage, w[t], nbytes, lane);
          const uint32_t* rec = reinterpret_cast<const uint32_t*>(
              stage + (min(p, pend - 1) - q0c) * (2 * BB));
#pragma unroll
          for (int d = 0; d < PD; ++d) wl[d] = rec[d];
        } else {
#pragma unroll
          for (int d = 0; d < PD; ++d) wl[d] = w[t][d];
        }
        if (p < pend) {
          float t0, t1;
          pair_terms<FMT>(wl, cx, meta, t0, t1);
          *reinterpret_cast<float2*>(terms + r * (kc >> 5) + 2 * (p - pbeg)) = make_float2(t0, t1);
        }
      }
    }
    // Block-order sum of this chunk's terms (the wave's own LDS writes above
    // precede these reads in its instruction stream): fully unrolled over
    // the at most NPM * 128 terms, in groups of 16 behind a uniform guard.
    if (lane < RB) {
      const float* tr = terms + lane * (kc >> 5);
      const int nbc = clen >> 5;                  // even, <= NPM * 128
#pragma unroll
      for (int g = 0; g < NPM * 8; ++g) {
        if (16 * g + 16 <= nbc) {
          float4 v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = reinterpret_cast<const float4*>(tr + 16 * g)[i];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            total += v[i].x;
            total += v[i].y;
            total += v[i].z;
            total += v[i].w;
          }
        } else {
          for (int b = 16 * g; b < nbc; b += 2) {
            const float2 v = *reinterpret_cast<const float2*>(tr + b);
            total += v.x;
            total += v.y;
          }
          break;
        }
      }
    }
  }
  if (lane < RB && row0 + lane < n) y[row0 + lane] = total;
}

// Any K / alignment: one wavefront per row, lanes take blocks lane, lane +
// 64, ...; lane 0 adds the terms in block order.
template <int FMT>
__global__ __launch_bounds__(256) void qgemv_w8a8_generic(const uint8_t* __restrict__ W,
                                                          const float* __restrict__ x,
                                                          float* __restrict__ y, long long n,
                                                          long long k, int* status) {
  __shared__ float terms[4][64];
  constexpr int BB = Fmt<FMT>::block_bytes;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long long row = static_cast<long long>(blockIdx.x) * 4 + wave;
  const bool live = row < n;                       // wave-uniform
  const long long nb = k / 32;
  float total = 0.f;
  for (long long b0 = 0; b0 < nb; b0 += 64) {
    const long long b = b0 + lane;
    float t = 0.f;
    if (live && b < nb) {
      const float* xb = x + b * 32;
      float v[32];
      float m = 0.f;
      bool finite = true;
      for (int e = 0; e < 32; ++e) {
        v[e] = xb[e];
        m = fmaxf(m, fabsf(v[e]));
        finite = finite && isfinite(v[e]);
      }
      const float scale = m / 127.0f;
      const float inverse = scale != 0.0f ? 1.0f / scale : 0.0f;
      const uint8_t* blk = W + (row * nb + b) * BB;
      int dot = 0;
      for (int e = 0; e < 32; ++e) {
        float r = rintf(v[e] * inverse);
        r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
        const int c = finite ? static_cast<int>(r) : 0;
        const int q = FMT == kQ8_0 ? static_cast<int>(static_cast<int8_t>(blk[2 + e]))
                                   : (e < 16 ? (blk[2 + e] & 15) : (blk[2 + e - 16] >> 4)) - 8;
        dot += q * c;
      }
      const float d = half_bits_to_float(static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8));
      t = (static_cast<float>(dot) * d) * (finite ? scale : __builtin_nanf(""));
      if (!finite && status != nullptr) *status = 3;
    }
    terms[wave][lane] = t;
    if (lane == 0) {
      const long long cnt = nb - b0 < 64 ? nb - b0 : 64;
      for (int i = 0; i < cnt; ++i) total += terms[wave][i];
    }
  }
  if (live && lane == 0) y[row] = total;
}

// Load window (items in flight beyond the one being computed) by items per
// wave, T = NPM * RB, as measured on MI355X: enough to cover the load latency
// while keeping the arrival order close to the compute order.
template <int FMT, int T>
constexpr int window() {
  if constexpr (FMT == kQ4_0) return T >= 8 ? 3 : (T >= 4 ? 2 : 1);
  return T >= 8 ? 2 : 1;
}

// KIND 0: qgemv (f32 activations, exact digit dots); KIND 1: qgemv_w8a8;
// KIND 2: qgemv over a segment table (several matrices, or up/gate with the
// activation epilogue), x 16-byte aligned.
template <int KIND, int FMT, int NW, int RB, int NPM>
hipError_t launch_one(const GemvSegs& sg, const float* x, int k, int* status, hipStream_t s) {
  const int n = sg.start[sg.nseg];
  // weights held per lane: at most RB * NPM * pair dwords (<= 144 VGPRs)
  static_assert(RB * NPM * Fmt<FMT>::pair_dwords <= 144, "register budget");
  constexpr int WIN = window<FMT, NPM * RB>();
  const int kc = NPM * 4096 < k ? NPM * 4096 : k;
  const unsigned grid = static_cast<unsigned>((static_cast<long long>(n) + NW * RB - 1) / (NW * RB));
  const bool vec = reinterpret_cast<uintptr_t>(x) % 16 == 0;
  // digit records, then (chunked q8_0 items) each wave's item staging area
  const size_t dlds = chunked<FMT, NPM, RB>() ? stage_off(kc) + static_cast<size_t>(NW) * item_bytes<FMT>()
                                                 : lds_size(kc);
  if constexpr (KIND == 0) {
    if (vec)
      qgemv_dot_kernel<FMT, NW, RB, NPM, WIN, true, false><<<grid, 64 * NW, dlds, s>>>(sg, x, k, kc);
    else
      qgemv_dot_kernel<FMT, NW, RB, NPM, WIN, false, false><<<grid, 64 * NW, dlds, s>>>(sg, x, k, kc);
  } else if constexpr (KIND == 2) {
    // the caller guarantees a 16-byte aligned x
    qgemv_dot_kernel<FMT, NW, RB, NPM, WIN, true, true><<<grid, 64 * NW, dlds, s>>>(sg, x, k, kc);
  } else {
    const size_t lds = chunked<FMT, NPM, RB>()
                           ? w8_stage_off(kc, NW, RB) + static_cast<size_t>(NW) * item_bytes<FMT>()
                           : w8_lds_size(kc, NW, RB);
    if (vec)
      qgemv_w8a8_kernel<FMT, NW, RB, NPM, WIN, true><<<grid, 64 * NW, lds, s>>>(sg.w[0], x, sg.y[0], n, k, kc, status);
    else
      qgemv_w8a8_kernel<FMT, NW, RB, NPM, WIN, false><<<grid, 64 * NW, lds, s>>>(sg.w[0], x, sg.y[0], n, k, kc, status);
  }
  return hipGetLastError();
}


struct Shape {
  int nw, rb;
};

// Workgroup width (8 or 4 waves) and rows per wave: the candidate that
// minimises the rows handled by the busiest CU, among those with at most two
// workgroups per CU (which then all run together) when there are any; ties go
// to 8 waves per CU (one 8-wave or two 4-wave workgroups), then to 8-wave
// workgroups for fewer than 7 rows per wave (one digit build of x shared by
// twice the rows) and to 4-wave ones otherwise (two workgroups per CU overlap
// one's digit build with the other's loads), then to the earlier candidate.
// `forced_rb` (non-zero) restricts the choice to that many rows per wave.
Shape pick_shape(int n, const int* cand, int ncand, int forced_rb) {
  const int cus = device_cu_count();
  Shape best{8, forced_rb ? forced_rb : cand[0]};
  for (int pass = 0; pass < 2; ++pass) {
    long long best_score = -1;
    for (int nw : {8, 4}) {
      for (int i = 0; i < ncand; ++i) {
        const int rb = cand[i];
        if (forced_rb && rb != forced_rb) continue;
        const long long grid = (n + nw * rb - 1) / (nw * rb);
        const long long wpc = (grid + cus - 1) / cus;
        if (pass == 0 && wpc > 2) continue;
        const long long rows = wpc * nw * rb;
        const int not_eight = wpc * nw == 8 ? 0 : 1;
        const int not_pref = (rb >= 7) == (nw == 4) ? 0 : 1;
        const long long score = rows * 4 + not_eight * 2 + not_pref;
        if (best_score < 0 || score < best_score) {
          best = Shape{nw, rb};
          best_score = score;
        }
      }
    }
    if (best_score >= 0) break;
  }
  return best;
}

template <int KIND, int FMT, int NW, int NPM>
hipError_t launch_rb(int rb, const GemvSegs& sg, const float* x, int k, int* status,
                     hipStream_t s) {
  if constexpr (NPM == 1) {
    switch (rb) {
      case 1: return launch_one<KIND, FMT, NW, 1, 1>(sg, x, k, status, s);
      case 2: return launch_one<KIND, FMT, NW, 2, 1>(sg, x, k, status, s);
      case 4: return launch_one<KIND, FMT, NW, 4, 1>(sg, x, k, status, s);
      case 7: return launch_one<KIND, FMT, NW, 7, 1>(sg, x, k, status, s);
      case 8: return launch_one<KIND, FMT, NW, 8, 1>(sg, x, k, status, s);
      default:
        if constexpr (FMT == kQ4_0) return launch_one<KIND, FMT, NW, 14, 1>(sg, x, k, status, s);
        return launch_one<KIND, FMT, NW, 8, 1>(sg, x, k, status, s);
    }
  } else if constexpr (NPM == 2) {
    switch (rb) {
      case 1: return launch_one<KIND, FMT, NW, 1, 2>(sg, x, k, status, s);
      case 2: return launch_one<KIND, FMT, NW, 2, 2>(sg, x, k, status, s);
      case 4: return launch_one<KIND, FMT, NW, 4, 2>(sg, x, k, status, s);
      default:
        if constexpr (FMT == kQ4_0) return launch_one<KIND, FMT, NW, 7, 2>(sg, x, k, status, s);
        return launch_one<KIND, FMT, NW, 4, 2>(sg, x, k, status, s);
    }
  } else {
    switch (rb) {
      case 1: return launch_one<KIND, FMT, NW, 1, 4>(sg, x, k, status, s);
      case 2: return launch_one<KIND, FMT, NW, 2, 4>(sg, x, k, status, s);
      default:
        if constexpr (FMT == kQ4_0) return launch_one<KIND, FMT, NW, 4, 4>(sg, x, k, status, s);
        return launch_one<KIND, FMT, NW, 2, 4>(sg, x, k, status, s);
    }
  }
}

// Candidates of rows per wave: with an activation or RoPE epilogue only even
// counts (each wave holds whole (up, gate) or (d, d + half) row pairs).
template <int KIND, int FMT, int NPM>
hipError_t launch_npm(const int* cand_all, int ncand_all, const GemvSegs& sg, const float* x,
                      int k, int rb, int* status, hipStream_t s) {
  int cand[8];
  int ncand = 0;
  for (int i = 0; i < ncand_all; ++i)
    if ((sg.act < 0 && sg.half == 0) || cand_all[i] % 2 == 0) cand[ncand++] = cand_all[i];
  bool listed = false;
  for (int i = 0; i < ncand; ++i) listed = listed || cand[i] == rb;
  const Shape sh = pick_shape(sg.start[sg.nseg], cand, ncand, listed ? rb : 0);
  return sh.nw == 8 ? launch_rb<KIND, FMT, 8, NPM>(sh.rb, sg, x, k, status, s)
                    : launch_rb<KIND, FMT, 4, NPM>(sh.rb, sg, x, k, status, s);
}

template <int KIND, int FMT>
hipError_t launch_fmt(const GemvSegs& sg, const float* x, int k, int rb, int* status,
                      hipStream_t s) {
  const int npairs = k >> 6;
  if (npairs <= 64) {
    static const int q4c[] = {14, 7, 8, 4, 2, 1};
    static const int q8c[] = {8, 7, 4, 2, 1};
    return FMT == kQ4_0 ? launch_npm<KIND, FMT, 1>(q4c, 6, sg, x, k, rb, status, s)
                        : launch_npm<KIND, FMT, 1>(q8c, 5, sg, x, k, rb, status, s);
  }
  if (npairs <= 128) {
    static const int q4c[] = {7, 4, 2, 1};
    static const int q8c[] = {4, 2, 1};
    return FMT == kQ4_0 ? launch_npm<KIND, FMT, 2>(q4c, 4, sg, x, k, rb, status, s)
                        : launch_npm<KIND, FMT, 2>(q8c, 3, sg, x, k, rb, status, s);
  }
  static const int q4c[] = {4, 2, 1};
  static const int q8c[] = {2, 1};
  return FMT == kQ4_0 ? launch_npm<KIND, FMT, 4>(q4c, 3, sg, x, k, rb, status, s)
                      : launch_npm<KIND, FMT, 4>(q8c, 2, sg, x, k, rb, status, s);
}

}  // namespace

// K % 64 == 0 and W 4-byte aligned (checked by the caller).  rows_per_wave:
// 0, or a count the register budget for K does not allow, picks from the
// shape; otherwise 1, 2, 4, 7, 8 or 14 (q4_0) rows per wave.
hipError_t launch_qgemv_dot(int fmt, const void* Wv, const float* x, float* y, int n, int k,
                            int rows_per_wave, hipStream_t s) {
  GemvSegs sg{};
  sg.w[0] = static_cast<const uint8_t*>(Wv);
  sg.y[0] = y;
  sg.start[0] = 0;
  sg.start[1] = n;
  sg.nseg = 1;
  sg.act = -1;
  return fmt == kQ8_0 ? launch_fmt<0, kQ8_0>(sg, x, k, rows_per_wave, nullptr, s)
                      : launch_fmt<0, kQ4_0>(sg, x, k, rows_per_wave, nullptr, s);
}

// Several matrices over one x in one launch (K % 64 == 0, every W 4-byte
// aligned, x 16-byte aligned, checked by the caller): nseg plain segments, or
// (act >= 0) up and gate with out = activation(gate) * up.
hipError_t launch_qgemv_multi(int fmt, int nseg, const void* const* W, float* const* y,
                              const int* rows, int act, const float* x, int k, hipStream_t s) {
  GemvSegs sg{};
  sg.nseg = act >= 0 ? 1 : nseg;
  sg.act = act;
  sg.start[0] = 0;
  if (act >= 0) {
    sg.w[0] = static_cast<const uint8_t*>(W[0]);
    sg.w[1] = static_cast<const uint8_t*>(W[1]);
    sg.y[0] = y[0];
    sg.start[1] = 2 * rows[0];
  } else {
    for (int i = 0; i < nseg; ++i) {
      sg.w[i] = static_cast<const uint8_t*>(W[i]);
      sg.y[i] = y[i];
      sg.start[i + 1] = sg.start[i] + rows[i];
    }
  }
  return fmt == kQ8_0 ? launch_fmt<2, kQ8_0>(sg, x, k, 0, nullptr, s)
                      : launch_fmt<2, kQ4_0>(sg, x, k, 0, nullptr, s);
}

// Small-batch rows: passes of MB activation rows over W (m <= 8 per pass is
// the intended use).  K % 64 == 0 and W 4-byte aligned (checked by the
// caller).  One chunk of kc = 4096 columns per step (MB * lds_size(4096) of
// LDS); the rows per wave and workgroup width by the GEMV's shape rule.
template <int FMT, int NW, int RB, int MB>
hipError_t launch_rows(const uint8_t* W, const float* x, float* y, int n, int k, int m, hipStream_t s) {
  const int kc = k < 4096 ? k : 4096;
  const long long groups = (static_cast<long long>(n) + NW * RB - 1) / (NW * RB);
  const size_t lds = MB * lds_size(kc);
  // persistent grid (one chunk): as many workgroups as fit on the chip at once
  // (rounded so that every workgroup takes the same number of row groups)
  long long grid = groups;
  if (k <= kc) {
    const int per_cu = static_cast<int>(std::min<size_t>(160 * 1024 / lds, 16 / NW));
    const long long most = static_cast<long long>(device_cu_count()) * std::max(per_cu, 1);
    const long long rounds = (groups + most - 1) / most;
    grid = (groups + rounds - 1) / rounds;
  }
  const bool vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && k % 4 == 0;
  if (vec)
    qgemm_rows_kernel<FMT, NW, RB, MB, true><<<static_cast<unsigned>(grid), 64 * NW, lds, s>>>(W, x, y, n, k, m, kc);
  else
    qgemm_rows_kernel<FMT, NW, RB, MB, false><<<static_cast<unsigned>(grid), 64 * NW, lds, s>>>(W, x, y, n, k, m, kc);
  return hipGetLastError();
}

// Rows per wave: rb (1, 2 or 4) when given, else 2; 8-wave workgroups, or
// 4-wave ones when K spans several chunks and 8-wave ones would leave CUs
// idle (the GEMV's shape rule).
template <int FMT, int MB>
hipError_t launch_rows_mb(const uint8_t* W, const float* x, float* y, int n, int k, int m,
                          int rb, hipStream_t s) {
  if (rb != 1 && rb != 4) rb = 2;
  if constexpr (MB == 8) rb = rb == 4 ? 2 : rb;    // 4 rows x 8 digit sets exceed the registers
  if constexpr (MB < 8) {
    if (k > 4096) {
      static const int cand[] = {2, 1};
      const Shape sh = pick_shape(n, cand, 2, rb == 4 ? 2 : rb);
      if (sh.nw == 4)
        return sh.rb == 2 ? launch_rows<FMT, 4, 2, MB>(W, x, y, n, k, m, s)
                          : launch_rows<FMT, 4, 1, MB>(W, x, y, n, k, m, s);
      rb = sh.rb;
    }
  }
  return rb == 4 ? launch_rows<FMT, 8, 4, MB>(W, x, y, n, k, m, s)
       : rb == 2 ? launch_rows<FMT, 8, 2, MB>(W, x, y, n, k, m, s)
                 : launch_rows<FMT, 8, 1, MB>(W, x, y, n, k, m, s);
}

// y[m][n] for m rows of x in passes of at most 8 rows, each output
// bit-identical to launch_qgemv_dot of its row.
hipError_t launch_qgemm_rows(int fmt, const void* Wv, const float* x, float* y, int n, int k,
                             int m, int rows_per_wave, hipStream_t s) {
  const auto* W = static_cast<const uint8_t*>(Wv);
  for (int m0 = 0; m0 < m; m0 += 8) {
    const int mp = min(8, m - m0);
    const float* xp = x + static_cast<long long>(m0) * k;
    float* yp = y + static_cast<long long>(m0) * n;
    hipError_t e;
    if (fmt == kQ8_0)
      e = mp <= 2 ? launch_rows_mb<kQ8_0, 2>(W, xp, yp, n, k, mp, rows_per_wave, s)
        : mp <= 4 ? launch_rows_mb<kQ8_0, 4>(W, xp, yp, n, k, mp, rows_per_wave, s)
                  : launch_rows_mb<kQ8_0, 8>(W, xp, yp, n, k, mp, rows_per_wave, s);
    else
      e = mp <= 2 ? launch_rows_mb<kQ4_0, 2>(W, xp, yp, n, k, mp, rows_per_wave, s)
        : mp <= 4 ? launch_rows_mb<kQ4_0, 4>(W, xp, yp, n, k, mp, rows_per_wave, s)
                  : launch_rows_mb<kQ4_0, 8>(W, xp, yp, n, k, mp, rows_per_wave, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Q (and, kv_rows > 0, K and V) projections of one token with RoPE on Q and
// K, in one launch (K % 64 == 0, every W 4-byte aligned, x 16-byte aligned,
// checked by the caller).  q: q_rows outputs; kc / vc: the slot's kv_rows
// outputs in the key / value cache.
hipError_t launch_qgemv_qkv_rope(int fmt, const void* Wq, const void* Wk, const void* Wv,
                                 float* q, float* kc, float* vc, int q_rows, int kv_rows,
                                 int half, const float* rc, const float* rs, const float* x,
                                 int k, hipStream_t s) {
  GemvSegs sg{};
  sg.act = -1;
  sg.half = half;
  sg.rc = rc;
  sg.rs = rs;
  sg.w[0] = static_cast<const uint8_t*>(Wq);
  sg.y[0] = q;
  sg.start[0] = 0;
  sg.start[1] = q_rows;
  sg.nseg = 1;
  sg.nrope = 1;
  if (kv_rows > 0) {
    sg.w[1] = static_cast<const uint8_t*>(Wk);
    sg.w[2] = static_cast<const uint8_t*>(Wv);
    sg.y[1] = kc;
    sg.y[2] = vc;
    sg.start[2] = q_rows + kv_rows;
    sg.start[3] = q_rows + 2 * kv_rows;
    sg.nseg = 3;
    sg.nrope = 2;
  }
  return fmt == kQ8_0 ? launch_fmt<2, kQ8_0>(sg, x, k, 0, nullptr, s)
                      : launch_fmt<2, kQ4_0>(sg, x, k, 0, nullptr, s);
}

// out[h * 2 * half + d] and out[h * 2 * half + d + half] rotated in place for
// every head h < heads and d < half (the per-matrix route of the RoPE seam).
__global__ void rope_pairs_kernel(float* out, long long pairs, int half,
                                  const float* __restrict__ rc, const float* __restrict__ rs) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= pairs) return;
  const long long head = i / half;
  const int d = static_cast<int>(i - head * half);
  float* const p = out + head * 2 * half + d;
  const float a = p[0], b = p[half], c = rc[d], sn = rs[d];
  p[0] = a * c - b * sn;
  p[half] = b * c + a * sn;
}

hipError_t launch_rope_pairs(float* out, long long heads, int half, const float* rc,
                             const float* rs, hipStream_t s) {
  const long long pairs = heads * half;
  if (pairs <= 0) return hipSuccess;
  rope_pairs_kernel<<<static_cast<unsigned>((pairs + 255) / 256), 256, 0, s>>>(out, pairs, half,
                                                                               rc, rs);
  return hipGetLastError();
}

// qgemv_w8a8: the fast kernel when K/32 is even, W is 4-byte aligned and the
// sizes fit 32-bit indexing; the one-wave-per-row kernel otherwise.
hipError_t launch_qgemv_w8a8(int fmt, const void* Wv, const float* x, float* y, long long n,
                             long long k, int rows_per_wave, int* status, hipStream_t s) {
  const auto* W = static_cast<const uint8_t*>(Wv);
  const bool fast = (k >> 5) % 2 == 0 && reinterpret_cast<uintptr_t>(W) % 4 == 0 &&
                    n < (1LL << 31) && k < (1LL << 31);
  if (fast) {
    GemvSegs sg{};
    sg.w[0] = W;
    sg.y[0] = y;
    sg.start[0] = 0;
    sg.start[1] = static_cast<int>(n);
    sg.nseg = 1;
    sg.act = -1;
    return fmt == kQ8_0 ? launch_fmt<1, kQ8_0>(sg, x, (int)k, rows_per_wave, status, s)
                        : launch_fmt<1, kQ4_0>(sg, x, (int)k, rows_per_wave, status, s);
  }
  const long long grid = (n + 3) / 4;
  if (fmt == kQ8_0)
    qgemv_w8a8_generic<kQ8_0><<<static_cast<unsigned>(grid), 256, 0, s>>>(W, x, y, n, k, status);
  else
    qgemv_w8a8_generic<kQ4_0><<<static_cast<unsigned>(grid), 256, 0, s>>>(W, x, y, n, k, status);
  return hipGetLastError();
}

// out[i] = activation(out[i]) * up[i]: the per-matrix route of the fused
// up/gate activation, with the single-launch epilogue's arithmetic.
__global__ void fused_activation_kernel(float* out, const float* up, long long n, int act) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = fused_activation(out[i], act) * up[i];
}

hipError_t launch_fused_activation(float* out, const float* up, long long n, int act,
                                   hipStream_t s) {
  if (n <= 0) return hipSuccess;
  fused_activation_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(out, up, n, act);
  return hipGetLastError();
}

}  // namespace qc
