// Projections over canonical int8 weights (kInt8Symmetric / kInt8Affine of
// the reference's canonical contract): y[m][n] = sum_k x[m][k] * w(n, k) with
// w(n, k) = scale(n, g) * (code[n][k] - zero(n, g)), g = k / group_size
// (kernels/quantization/qgemm_canonical.cpp:125-176, decode_prepared_chunk).
// Activations and outputs are f32, f16 or bf16 (decoded exactly, accumulated
// in f32, rounded once at the store, kernels/common/float_storage_access.h).
//
// One launch covers up to three matrices over the same x (the prepared
// storage seams of include/quixicore_cpu/qgemm.h:32-101) with the epilogue
// fused: bias + activation, SiLU(gate) * up over interleaved gate/up rows,
// or split-half RoPE over the (d, d + half) row pairs of each head.
//
// Layout: codes row-major [rows][k] (the canonical bytes, unchanged); scales
// (and zero points) f32 [rows][groups].  The fast kernel streams each row in
// 16-byte chunks, one per lane and step (a wave covers 1024 columns of a row
// per load instruction), with the next step's chunks in flight while the
// current ones are multiplied against the f32 activations staged in LDS.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "qc_device.h"
#include "qc_digits.h"
#include "qc_int8_ring.h"
#include "qc_internal.h"

namespace qc {
namespace {

constexpr int kThreads = 256;   // 4 waves
constexpr int kWaves = kThreads / 64;

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

struct RowRef {
  int seg;    // segment of the row (mode 1: 0 = gate, 1 = up)
  int row;    // row of that segment's matrix
};

__device__ __forceinline__ RowRef logical_row(const CSegs& s, int g) {
  RowRef r;
  if (s.mode == 1) {
    r.seg = g & 1;
    r.row = g >> 1;
    return r;
  }
  r.seg = (s.nseg > 2 && g >= s.start[2]) ? 2 : (s.nseg > 1 && g >= s.start[1]) ? 1 : 0;
  r.row = g - s.start[r.seg];
  if (s.mode == 2 && r.seg < s.nrope) {
    const int j = r.row >> 1;
    const int head = j / s.half;
    r.row = head * 2 * s.half + (j - head * s.half) + (r.row & 1) * s.half;
  }
  return r;
}

// Stores the finished values of logical rows g (and g + 1 for the paired
// modes) for activation row m.  v0 / v1: their projections.
__device__ __forceinline__ void epilogue(const CSegs& s, int g, int m, float v0, float v1) {
  if (s.mode == 1) {
    const float silu = v0 / (1.0f + expf(-v0));
    store_y(s.y[0], m * s.ld[0] + (g >> 1), s.ytype[0], silu * v1);
    return;
  }
  const RowRef r = logical_row(s, g);
  if (s.mode == 2) {
    if (r.seg < s.nrope) {
      const int d = r.row % (2 * s.half);
      const float c = s.rc[d], sn = s.rs[d];
      store_y(s.y[r.seg], r.row, s.ytype[r.seg], v0 * c - v1 * sn);
      store_y(s.y[r.seg], r.row + s.half, s.ytype[r.seg], v1 * c + v0 * sn);
    } else {
      store_y(s.y[r.seg], r.row, s.ytype[r.seg], v0);
      store_y(s.y[r.seg], r.row + 1, s.ytype[r.seg], v1);
    }
    return;
  }
  float v = v0;
  if (r.seg == 0 && (s.bias != nullptr || s.act != 0)) {
    if (s.bias != nullptr) v += s.bias[r.row];
    v = linear_activation(v, s.act);
  }
  store_y(s.y[r.seg], m * s.ld[r.seg] + r.row, s.ytype[r.seg], v);
}

__device__ __forceinline__ void unpack16(const uint4& c, float* q) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int b = 0; b < 4; ++b)
      q[4 * i + b] = static_cast<float>(static_cast<int32_t>(w[i] << (24 - 8 * b)) >> 24);
  }
}

// MB activation rows per pass, RW rows per wave.  GRP: one scale per group of
// 2^gshift columns (else per row, applied once at the end); AFF: zero points.
// The activations of a K chunk (kc columns, a multiple of 1024) are staged in
// LDS as f32.  Requires k % 16 == 0 and 16-byte aligned codes.
//
// When K fits one chunk the grid is persistent: a workgroup stages x once
// and takes row groups blockIdx.x, + gridDim.x, ... (kWaves * RW logical
// rows each), the first codes of its first group in flight before the
// staging and those of the next group before the current one finishes.
// Otherwise each workgroup takes one row group and restages x per chunk.
template <int MB, int RW, bool GRP, bool AFF>
__global__ __launch_bounds__(kThreads) void cint8_kernel(const CSegs segs, const void* __restrict__ x,
                                                         int xtype, long long ldx, int m0, int mrows,
                                                         int k, int kc) {
  extern __shared__ __attribute__((aligned(16))) float xs[];   // [MB][kc]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int total = segs.start[segs.nseg];
  const int groups = (total + kWaves * RW - 1) / (kWaves * RW);

  // row pointers of row group g: codes, scales, zero points; returns its first logical row
  auto rows_of = [&](int g, const int8_t* (&w)[RW], const float* (&sp)[RW],
                     const float* (&zp)[RW]) {
    const int g0 = (g * kWaves + wave) * RW;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const RowRef rr = logical_row(segs, min(g0 + r, total - 1));
      w[r] = segs.w[rr.seg] + static_cast<long long>(rr.row) * k;
      sp[r] = segs.scale[rr.seg] + static_cast<long long>(rr.row) * segs.groups;
      zp[r] = AFF ? segs.zero[rr.seg] + static_cast<long long>(rr.row) * segs.groups : nullptr;
    }
    return g0;
  };
  // x of chunk [c0, c0 + clen) into LDS as f32: four loads in flight per
  // thread (consecutive threads, consecutive elements), then their stores
  auto stage_x = [&](int c0, int clen) {
    constexpr int kBatch = 4;
    for (int mm = 0; mm < MB; ++mm) {
      const int mrow = m0 + mm;
      const bool live = mrow < mrows;
      for (int base = 0; base < clen; base += kBatch * kThreads) {
        float v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int i = base + threadIdx.x + u * kThreads;
          v[u] = live && i < clen ? load_x(x, mrow * ldx + c0 + i, xtype) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int i = base + threadIdx.x + u * kThreads;
          if (i < clen) xs[mm * kc + i] = v[u];
        }
      }
    }
  };
  // a unit: columns [c, c + 4096) of one row (up to 4 steps of 1024), loaded
  // as one contiguous 4 KB run per wave (lane: 16 bytes per step)
  // (GRP: with the group scales and zero points of its four 16-column steps)
  struct Unit {
    uint4 c[4];
    float s[4], z[4];
  };
  auto fetch = [&](Unit& u, const int8_t* row, const float* sp, const float* zp, int c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = min(c + 16 * (lane + 64 * i), k - 16);
      u.c[i] = *reinterpret_cast<const uint4*>(row + e);
      if constexpr (GRP) {
        u.s[i] = sp[e >> segs.gshift];
        if constexpr (AFF) u.z[i] = zp[e >> segs.gshift];
      }
    }
  };
  // 16 codes of one row at column e against the staged activations; affine
  // codes enter as (q - z), the reference's decode, so an infinite x meets
  // each weight's own sign (sum q x - z sum x could give inf - inf)
  auto step = [&](const uint4& c, float sc, float zv, int c0, int e, float (&acc)[MB]) {
    float xv[MB][16];
#pragma unroll
    for (int mm = 0; mm < MB; ++mm) {
      const float4* p = reinterpret_cast<const float4*>(xs + mm * kc + (e - c0));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 t = p[i];
        xv[mm][4 * i] = t.x; xv[mm][4 * i + 1] = t.y; xv[mm][4 * i + 2] = t.z; xv[mm][4 * i + 3] = t.w;
      }
    }
    float q[16];
    unpack16(c, q);
    if constexpr (AFF) {
#pragma unroll
      for (int i = 0; i < 16; ++i) q[i] -= zv;
    }
#pragma unroll
    for (int mm = 0; mm < MB; ++mm) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) t = fmaf(q[i], xv[mm][i], t);
      if constexpr (GRP) acc[mm] = fmaf(sc, t, acc[mm]);
      else acc[mm] += t;
    }
  };
  // wave sums, returned to every lane; then lane (r * MB + mm) finishes one
  // value, or (paired modes) one row pair
  auto finish = [&](int g0, const float* const (&sp)[RW], float (&acc)[RW][MB]) {
    float tot[RW][MB];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int mm = 0; mm < MB; ++mm) {
        float v = wave_sum(acc[r][mm]);
        if constexpr (!GRP) v = sp[r][0] * v;
        tot[r][mm] = v;
      }
    if (segs.mode == 0) {
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int mm = 0; mm < MB; ++mm)
          if (lane == r * MB + mm && g0 + r < total && m0 + mm < mrows)
            epilogue(segs, g0 + r, m0 + mm, tot[r][mm], 0.f);
    } else {
#pragma unroll
      for (int r = 0; r + 1 < RW; r += 2)
#pragma unroll
        for (int mm = 0; mm < MB; ++mm)
          if (lane == r * MB + mm && g0 + r < total && m0 + mm < mrows)
            epilogue(segs, g0 + r, m0 + mm, tot[r][mm], tot[r + 1][mm]);
    }
  };

  float acc[RW][MB];
  const int8_t* w[RW];
  const float* sp[RW];
  const float* zp[RW];
  const bool single = k <= kc;
  int g = blockIdx.x;
  int g0 = rows_of(g, w, sp, zp);
  Unit cur, nxt;
  if (single) {
    fetch(cur, w[0], sp[0], zp[0], 0);
    stage_x(0, k);
    __syncthreads();
  }
  for (;;) {
    const int gn = single ? g + static_cast<int>(gridDim.x) : groups;
    const int8_t* wn[RW];
    const float* sn[RW];
    const float* zn[RW];
    const int gn0 = rows_of(min(gn, groups - 1), wn, sn, zn);
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int mm = 0; mm < MB; ++mm) acc[r][mm] = 0.f;
    for (int c0 = 0; c0 < k; c0 += kc) {
      const int clen = min(kc, k - c0);
      if (!single) {
        fetch(cur, w[0], sp[0], zp[0], c0);
        if (c0) __syncthreads();
        stage_x(c0, clen);
        __syncthreads();
      }
      // rows in order, each in 4096-column units; the next unit (of this
      // row, the next row, or the next row group's first row) is in flight
      // while the current one is computed
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        for (int c = c0; c < c0 + clen; c += 4096) {
          const int rn = r + 1 < RW ? r + 1 : r;
          if (c + 4096 < c0 + clen) fetch(nxt, w[r], sp[r], zp[r], c + 4096);
          else if (r + 1 < RW) fetch(nxt, w[rn], sp[rn], zp[rn], c0);
          else if (!single && c0 + kc < k) fetch(nxt, w[0], sp[0], zp[0], c0 + kc);
          else if (gn < groups) fetch(nxt, wn[0], sn[0], zn[0], 0);
          // affine row zero points: one per row
          const float zr = AFF && !GRP ? zp[r][0] : 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int e = c + 16 * (lane + 64 * i);
            if (e < c0 + clen) step(cur.c[i], cur.s[i], GRP ? cur.z[i] : zr, c0, e, acc[r]);
          }
          cur = nxt;
        }
      }
    }
    finish(g0, sp, acc);
    if (gn >= groups) break;
    g = gn;
    g0 = gn0;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      w[r] = wn[r];
      sp[r] = sn[r];
      zp[r] = zn[r];
    }
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

// M = 1 with exact digit dots (the GEMV's encoding of x, qc_digits.h):
// k % 64 == 0, 16-byte aligned codes, GRP groups a power of two >= 32.
// Wave w of workgroup b owns logical rows (b * kWaves + w) * RB + r; lane l
// the block pair p = l (mod 64) of each row in every chunk of up to 4096
// columns, its 64 codes in four 16-byte loads issued after the thread's x
// values and before the chunk's digit build.  Per block: f = 2^e (2^14 S0 + 2^7 S1 + S2) ~ sum_j q_j x_j
// (three v_dot4 sums per 4 codes) and, for affine weights, xs = 2^e (2^14
// D0 + 2^7 D1 + D2) ~ sum_j x_j over the same encoded x.  Group scales add
// s_g (f - z_g xs) per block; row scales finish as s (sum f - z sum xs).
template <int RB, bool GRP, bool AFF>
__global__ __launch_bounds__(kThreads) void cint8_dot_kernel(const CSegs segs,
                                                             const void* __restrict__ x,
                                                             int xtype, int k, bool xvec) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int kc = 4096;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int total = segs.start[segs.nseg];
  const int g0 = (blockIdx.x * kWaves + wave) * RB;
  const int8_t* w[RB];
  const float* sp[RB];
  const float* zp[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const RowRef rr = logical_row(segs, min(g0 + r, total - 1));
    w[r] = segs.w[rr.seg] + static_cast<long long>(rr.row) * k;
    sp[r] = segs.scale[rr.seg] + static_cast<long long>(rr.row) * segs.groups;
    zp[r] = AFF ? segs.zero[rr.seg] + static_cast<long long>(rr.row) * segs.groups : nullptr;
  }
  float acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = 0.f;
  float sxs = 0.f;   // affine row scales: this lane's sum of xs (finite blocks)
  // affine row scales with an integral zero point: (c - z) summed exactly per
  // block (affine_block), so sxs is not needed for that row
  int rzi[RB];
  bool rzint[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) rzint[r] = AFF && !GRP && integral_zero(zp[r][0], rzi[r]);
  for (int c0 = 0; c0 < k; c0 += kc) {
    const int clen = min(kc, k - c0);
    const int pbeg = c0 >> 6, pend = (c0 + clen) >> 6;
    const int p = first_pair(pbeg, lane);
    const bool live = p < pend;
    const int pc = min(p, pend - 1);
    // 1. this thread's half-block of x (16 values; past the chunk it re-reads
    // the last one, which is not built), issued before the codes so that
    // waiting for it does not wait for them (loads retire in order); no
    // branch around it, which would make the compiler wait at the join
    const int nh = clen >> 4;
    const int hx = min(static_cast<int>(threadIdx.x), nh - 1);
    float v[16];
    {
      const long long xi = c0 + 16LL * hx;
      if (xvec && xtype == QC_STORAGE_F32) {
        const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(x) + xi);
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<float4*>(&v[4 * i]) = src[i];
      } else if (xvec) {
        const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + xi);
        const uint4 a = src[0], b = src[1];
        const uint32_t wd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint16_t lo = static_cast<uint16_t>(wd[i]), hi = static_cast<uint16_t>(wd[i] >> 16);
          if (xtype == QC_STORAGE_F16) {
            v[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, lo));
            v[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, hi));
          } else {
            v[2 * i] = __uint_as_float(static_cast<uint32_t>(lo) << 16);
            v[2 * i + 1] = __uint_as_float(static_cast<uint32_t>(hi) << 16);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = load_x(x, xi + i, xtype);
      }
    }
    // 2. the codes of this lane's pair of every row (and group scales)
    uint4 cw[RB][4];
    float gs[RB][2], gz[RB][2];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        cw[r][i] = *reinterpret_cast<const uint4*>(w[r] + 64LL * pc + 16 * i);
      if constexpr (GRP) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int gi = (64 * pc + 32 * h) >> segs.gshift;
          gs[r][h] = sp[r][gi];
          gz[r][h] = AFF ? zp[r][gi] : 0.f;
        }
      }
    }
    // digits of this chunk of x (half-block h = thread; the two halves of a
    // block sit in lanes t and t ^ 1, both inside or both past the chunk)
    // 3. the chunk's digits
    if (c0) lds_barrier();
    if (static_cast<int>(threadIdx.x) < nh) build_half<AFF>(lds, v, threadIdx.x, kc);
    lds_barrier();
    if (live) {
      PairDigits g;
      read_digits<kQ8_0>(g, lds, p - pbeg, kc);
      float xs[2] = {0.f, 0.f};
      int ds[2][3] = {{0, 0, 0}, {0, 0, 0}};
      if constexpr (AFF) {
        read_digit_sums(ds, lds, p - pbeg, kc);
#pragma unroll
        for (int h = 0; h < 2; ++h) xs[h] = ldexpf(combine(ds[h][0], ds[h][1], ds[h][2]), g.e[h]);
        if constexpr (!GRP) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            if (g.gate[h] == 1.0f) sxs += xs[h];
        }
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        int sd[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint4 q4 = cw[r][i >> 2];
          const uint32_t q = (i & 3) == 0 ? q4.x : (i & 3) == 1 ? q4.y : (i & 3) == 2 ? q4.z : q4.w;
          const int hb = i >> 3;
#pragma unroll
          for (int t = 0; t < 3; ++t)
            sd[hb][t] = __builtin_amdgcn_sdot4(static_cast<int>(q), static_cast<int>(g.d[t][i]),
                                               sd[hb][t], false);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (g.gate[h] == 1.0f) {
            const float f = ldexpf(combine(sd[h][0], sd[h][1], sd[h][2]), g.e[h]);
            if constexpr (GRP && AFF) {
              int zi;
              const float t = integral_zero(gz[r][h], zi) ? affine_block(sd[h], ds[h], zi, g.e[h])
                                                          : fmaf(-gz[r][h], xs[h], f);
              acc[r] = fmaf(gs[r][h], t, acc[r]);
            } else if constexpr (GRP) {
              acc[r] = fmaf(gs[r][h], f, acc[r]);
            } else if constexpr (AFF) {
              acc[r] += rzint[r] ? affine_block(sd[h], ds[h], rzi[r], g.e[h]) : f;
            } else {
              acc[r] += f;
            }
          } else {
            const float z = AFF ? (GRP ? gz[r][h] : zp[r][0]) : 0.f;
            const float b = cint8_block_f32(w[r] + 64LL * p + 32 * h, x, c0 + 64LL * (p - pbeg) + 32 * h,
                                            xtype, z);
            acc[r] += GRP ? gs[r][h] * b : b;
          }
        }
      }
    }
  }
  // wave sums; lane r finishes row r (paired modes: lane r the pair r, r + 1)
  float tot[RB];
  const float sx = AFF && !GRP ? wave_sum(sxs) : 0.f;
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    float v = wave_sum(acc[r]);
    if constexpr (!GRP) v = sp[r][0] * (AFF && !rzint[r] ? fmaf(-zp[r][0], sx, v) : v);
    tot[r] = v;
  }
  if (segs.mode == 0) {
#pragma unroll
    for (int r = 0; r < RB; ++r)
      if (lane == r && g0 + r < total) epilogue(segs, g0 + r, 0, tot[r], 0.f);
  } else {
#pragma unroll
    for (int r = 0; r + 1 < RB; r += 2)
      if (lane == r && g0 + r < total) epilogue(segs, g0 + r, 0, tot[r], tot[r + 1]);
  }
}

// The same digit dots for several activation rows: rows m0 .. m0 + MB - 1
// (those below m) in one pass, with one digit record of x each in LDS; a
// lane's codes are loaded once and dotted with every row's digits, so each
// output row is bit-identical to the one-row kernel's.  (One row keeps its
// own kernel above: the row offset and count as arguments cost it 2-4%.)
template <int RB, bool GRP, bool AFF, int MB>
__global__ __launch_bounds__(kThreads) void cint8_dot_rows_kernel(const CSegs segs,
                                                                  const void* __restrict__ x,
                                                                  int xtype, int k, bool xvec,
                                                                  long long ldx, int m0, int m) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int kc = 4096;
  constexpr int LS = static_cast<int>(lds_size(kc));
  static_assert(MB == 2 || MB == 4, "one activation row takes cint8_dot_kernel");
  const int mrows = min(MB, m - m0);   // wave-uniform
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int total = segs.start[segs.nseg];
  const int g0 = (blockIdx.x * kWaves + wave) * RB;
  const int8_t* w[RB];
  const float* sp[RB];
  const float* zp[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const RowRef rr = logical_row(segs, min(g0 + r, total - 1));
    w[r] = segs.w[rr.seg] + static_cast<long long>(rr.row) * k;
    sp[r] = segs.scale[rr.seg] + static_cast<long long>(rr.row) * segs.groups;
    zp[r] = AFF ? segs.zero[rr.seg] + static_cast<long long>(rr.row) * segs.groups : nullptr;
  }
  float acc[RB][MB];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int mm = 0; mm < MB; ++mm) acc[r][mm] = 0.f;
  float sxs[MB];   // affine row scales: this lane's sum of xs (finite blocks)
#pragma unroll
  for (int mm = 0; mm < MB; ++mm) sxs[mm] = 0.f;
  int rzi[RB];      // integral row zero points (affine_block), as in the one-row kernel
  bool rzint[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) rzint[r] = AFF && !GRP && integral_zero(zp[r][0], rzi[r]);
  for (int c0 = 0; c0 < k; c0 += kc) {
    const int clen = min(kc, k - c0);
    const int pbeg = c0 >> 6, pend = (c0 + clen) >> 6;
    const int p = first_pair(pbeg, lane);
    const bool live = p < pend;
    const int pc = min(p, pend - 1);
    // 1. this thread's half-block of x (16 values; past the chunk it re-reads
    // the last one, which is not built), issued before the codes so that
    // waiting for it does not wait for them (loads retire in order); no
    // branch around it, which would make the compiler wait at the join
    const int nh = clen >> 4;
    const int hx = min(static_cast<int>(threadIdx.x), nh - 1);
    float v[MB][16];
#pragma unroll
    for (int mm = 0; mm < MB; ++mm) {
      // rows past m re-read row m0 (not built)
      const long long xi = static_cast<long long>(m0 + (mm < mrows ? mm : 0)) * ldx + c0 + 16LL * hx;
      if (xvec && xtype == QC_STORAGE_F32) {
        const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(x) + xi);
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<float4*>(&v[mm][4 * i]) = src[i];
      } else if (xvec) {
        const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + xi);
        const uint4 a = src[0], b = src[1];
        const uint32_t wd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint16_t lo = static_cast<uint16_t>(wd[i]), hi = static_cast<uint16_t>(wd[i] >> 16);
          if (xtype == QC_STORAGE_F16) {
            v[mm][2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, lo));
            v[mm][2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, hi));
          } else {
            v[mm][2 * i] = __uint_as_float(static_cast<uint32_t>(lo) << 16);
            v[mm][2 * i + 1] = __uint_as_float(static_cast<uint32_t>(hi) << 16);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[mm][i] = load_x(x, xi + i, xtype);
      }
    }
    // 2. the codes of this lane's pair of every row (and group scales)
    uint4 cw[RB][4];
    float gs[RB][2], gz[RB][2];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        cw[r][i] = *reinterpret_cast<const uint4*>(w[r] + 64LL * pc + 16 * i);
      if constexpr (GRP) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int gi = (64 * pc + 32 * h) >> segs.gshift;
          gs[r][h] = sp[r][gi];
          gz[r][h] = AFF ? zp[r][gi] : 0.f;
        }
      }
    }
    // digits of this chunk of x (half-block h = thread; the two halves of a
    // block sit in lanes t and t ^ 1, both inside or both past the chunk)
    // 3. the chunk's digits
    if (c0) lds_barrier();
#pragma unroll
    for (int mm = 0; mm < MB; ++mm)
      if (mm < mrows && static_cast<int>(threadIdx.x) < nh)
        build_half<AFF>(lds + mm * LS, v[mm], threadIdx.x, kc);
    lds_barrier();
#pragma unroll
    for (int mm = 0; mm < MB; ++mm) {
      if (!live || mm >= mrows) continue;
      const uint8_t* const rec = lds + mm * LS;
      const long long xrow = static_cast<long long>(m0 + mm) * ldx;
      PairDigits g;
      read_digits<kQ8_0>(g, rec, p - pbeg, kc);
      float xs[2] = {0.f, 0.f};
      int ds[2][3] = {{0, 0, 0}, {0, 0, 0}};
      if constexpr (AFF) {
        read_digit_sums(ds, rec, p - pbeg, kc);
#pragma unroll
        for (int h = 0; h < 2; ++h) xs[h] = ldexpf(combine(ds[h][0], ds[h][1], ds[h][2]), g.e[h]);
        if constexpr (!GRP) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            if (g.gate[h] == 1.0f) sxs[mm] += xs[h];
        }
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        int sd[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint4 q4 = cw[r][i >> 2];
          const uint32_t q = (i & 3) == 0 ? q4.x : (i & 3) == 1 ? q4.y : (i & 3) == 2 ? q4.z : q4.w;
          const int hb = i >> 3;
#pragma unroll
          for (int t = 0; t < 3; ++t)
            sd[hb][t] = __builtin_amdgcn_sdot4(static_cast<int>(q), static_cast<int>(g.d[t][i]),
                                               sd[hb][t], false);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (g.gate[h] == 1.0f) {
            const float f = ldexpf(combine(sd[h][0], sd[h][1], sd[h][2]), g.e[h]);
            if constexpr (GRP && AFF) {
              int zi;
              const float t = integral_zero(gz[r][h], zi) ? affine_block(sd[h], ds[h], zi, g.e[h])
                                                          : fmaf(-gz[r][h], xs[h], f);
              acc[r][mm] = fmaf(gs[r][h], t, acc[r][mm]);
            } else if constexpr (GRP) {
              acc[r][mm] = fmaf(gs[r][h], f, acc[r][mm]);
            } else if constexpr (AFF) {
              acc[r][mm] += rzint[r] ? affine_block(sd[h], ds[h], rzi[r], g.e[h]) : f;
            } else {
              acc[r][mm] += f;
            }
          } else {
            const float z = AFF ? (GRP ? gz[r][h] : zp[r][0]) : 0.f;
            const float b = cint8_block_f32(w[r] + 64LL * p + 32 * h, x,
                                            xrow + c0 + 64LL * (p - pbeg) + 32 * h, xtype, z);
            acc[r][mm] += GRP ? gs[r][h] * b : b;
          }
        }
      }
    }
  }
  // wave sums; lane r finishes row r (paired modes: lane r the pair r, r + 1)
#pragma unroll
  for (int mm = 0; mm < MB; ++mm) {
    if (mm >= mrows) continue;
    float tot[RB];
    const float sx = AFF && !GRP ? wave_sum(sxs[mm]) : 0.f;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float v = wave_sum(acc[r][mm]);
      if constexpr (!GRP) v = sp[r][0] * (AFF && !rzint[r] ? fmaf(-zp[r][0], sx, v) : v);
      tot[r] = v;
    }
    if (segs.mode == 0) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
        if (lane == r && g0 + r < total) epilogue(segs, g0 + r, m0 + mm, tot[r], 0.f);
    } else {
#pragma unroll
      for (int r = 0; r + 1 < RB; r += 2)
        if (lane == r && g0 + r < total) epilogue(segs, g0 + r, m0 + mm, tot[r], tot[r + 1]);
    }
  }
}

// Any layout: one wave per (logical row, activation row), element by
// element with the reference's decode value = scale * (code - zero), into
// f32 scratch [m][total] (the epilogue kernel then finishes it).
__global__ __launch_bounds__(kThreads) void cint8_generic(const CSegs segs, const void* __restrict__ x,
                                                          int xtype, long long ldx, int mrows, int k,
                                                          float* __restrict__ out) {
  const int total = segs.start[segs.nseg];
  const long long item = static_cast<long long>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (item >= static_cast<long long>(total) * mrows) return;
  const int g = static_cast<int>(item % total);
  const int mrow = static_cast<int>(item / total);
  const RowRef rr = logical_row(segs, g);
  const int8_t* w = segs.w[rr.seg] + static_cast<long long>(rr.row) * k;
  const float* sc = segs.scale[rr.seg] + static_cast<long long>(rr.row) * segs.groups;
  const float* zp = segs.zero[rr.seg] == nullptr
                        ? nullptr
                        : segs.zero[rr.seg] + static_cast<long long>(rr.row) * segs.groups;
  float acc = 0.f;
  for (int e = threadIdx.x & 63; e < k; e += 64) {
    const int grp = segs.groups > 1 ? e / segs.gsize : 0;
    const float z = zp == nullptr ? 0.f : zp[grp];
    const float v = sc[grp] * (static_cast<float>(w[e]) - z);
    acc = fmaf(load_x(x, mrow * ldx + e, xtype), v, acc);
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) out[item] = acc;
}

__global__ __launch_bounds__(kThreads) void cint8_finish(const CSegs segs, const float* __restrict__ p,
                                                         int mrows) {
  const int total = segs.start[segs.nseg];
  const int step = segs.mode == 0 ? 1 : 2;
  const long long units = static_cast<long long>(total / step) * mrows;
  const long long u = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (u >= units) return;
  const int g = static_cast<int>(u % (total / step)) * step;
  const int mrow = static_cast<int>(u / (total / step));
  const float* row = p + static_cast<long long>(mrow) * total;
  epilogue(segs, g, mrow, row[g], step == 2 ? row[g + 1] : 0.f);
}

template <int MB, int RW, bool GRP, bool AFF>
hipError_t launch_fast(const CSegs& sg, const void* x, int xtype, long long ldx, int m, int k,
                       hipStream_t s) {
  const int total = sg.start[sg.nseg];
  const int kc = min(((k + 1023) / 1024) * 1024, 16384 / MB);
  const long long groups = (total + kWaves * RW - 1) / (kWaves * RW);
  const size_t lds = sizeof(float) * MB * kc;
  // one chunk: a persistent grid of what fits on the chip at once, rounded
  // so that every workgroup takes the same number of row groups
  long long g = groups;
  if (k <= kc) {
    const long long per_cu = std::max<long long>(1, std::min<long long>(160 * 1024 / lds, 8));
    const long long most = static_cast<long long>(device_cu_count()) * per_cu;
    const long long rounds = (groups + most - 1) / most;
    g = (groups + rounds - 1) / rounds;
  }
  const unsigned grid = static_cast<unsigned>(g);
  for (int m0 = 0; m0 < m; m0 += MB) {
    cint8_kernel<MB, RW, GRP, AFF><<<grid, kThreads, lds, s>>>(sg, x, xtype, ldx, m0, m, k, kc);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <int RB, bool GRP, bool AFF, int MB>
hipError_t launch_dot(const CSegs& sg, const void* x, int xtype, long long ldx, int m, int k,
                      hipStream_t s) {
  const int total = sg.start[sg.nseg];
  const unsigned grid = static_cast<unsigned>((total + kWaves * RB - 1) / (kWaves * RB));
  // x read in 16-byte pieces when every row starts 16-byte aligned (every
  // half-block then is: k % 64 == 0)
  const long long row_bytes = ldx * (xtype == QC_STORAGE_F32 ? 4 : 2);
  const bool xvec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && (m == 1 || row_bytes % 16 == 0);
  if constexpr (MB == 1) {
    cint8_dot_kernel<RB, GRP, AFF><<<grid, kThreads, lds_size(4096), s>>>(sg, x, xtype, k, xvec);
    return hipGetLastError();
  } else {
    for (int m0 = 0; m0 < m; m0 += MB) {
      cint8_dot_rows_kernel<RB, GRP, AFF, MB><<<grid, kThreads, MB * lds_size(4096), s>>>(
          sg, x, xtype, k, xvec, ldx, m0, m);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
}

template <bool GRP, bool AFF>
hipError_t launch_dot_rb(const CSegs& sg, const void* x, int xtype, long long ldx, int m, int k,
                         int rb, hipStream_t s) {
  if (m > 1)   // passes of up to 4 activation rows, two weight rows per wave
    return m == 2 ? launch_dot<2, GRP, AFF, 2>(sg, x, xtype, ldx, m, k, s)
                  : launch_dot<2, GRP, AFF, 4>(sg, x, xtype, ldx, m, k, s);
  switch (rb) {
    case 8: return launch_dot<8, GRP, AFF, 1>(sg, x, xtype, ldx, m, k, s);
    case 4: return launch_dot<4, GRP, AFF, 1>(sg, x, xtype, ldx, m, k, s);
    default: return launch_dot<2, GRP, AFF, 1>(sg, x, xtype, ldx, m, k, s);
  }
}

template <int MB, int RW>
hipError_t launch_mb(const CSegs& sg, bool grp, bool aff, const void* x, int xtype, long long ldx,
                     int m, int k, hipStream_t s) {
  if (grp)
    return aff ? launch_fast<MB, RW, true, true>(sg, x, xtype, ldx, m, k, s)
               : launch_fast<MB, RW, true, false>(sg, x, xtype, ldx, m, k, s);
  return aff ? launch_fast<MB, RW, false, true>(sg, x, xtype, ldx, m, k, s)
             : launch_fast<MB, RW, false, false>(sg, x, xtype, ldx, m, k, s);
}

}  // namespace

// ---- Row-plane route: two or more activation rows, one scale per weight row
// (or three or more, with scale groups of a multiple of 128 columns)
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

constexpr int kPlanesMaxK = 16384;
constexpr int kPlanesChunkM = 1024;     // activation rows per pass: bounds the scratch
// N = 14336, K = 4096 at M = 2: row scales 22.9 us on the digit-dot kernel,
// 18.8 here; groups of 128 22.0 there, 26.5 here (M = 3: 34.6 there, 26.4 here)
constexpr int kPlanesMinM = 2;
constexpr int kPlanesMinMGrouped = 3;
constexpr int kPlanesNonfinite = 0x40000000;

// The prep kernel: 1024 threads per activation row, each holding up to 16 of
// its values (four groups of four, K <= 16384) in registers, so the row is
// read once with every load in flight.
constexpr int kPrepThreads = 1024;
constexpr int kPrepWaves = kPrepThreads / 64;
constexpr int kPrepGroups = kPlanesMaxK / (4 * kPrepThreads);

__device__ __forceinline__ float block_max(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kPrepWaves; ++w) r = fmaxf(r, red[w]);
  return r;
}

__device__ __forceinline__ void block_sum3(int (&v)[3], int (*red)[kPrepWaves]) {
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    for (int off = 32; off > 0; off >>= 1) v[t] += __shfl_xor(v[t], off);
    if ((threadIdx.x & 63) == 0) red[t][threadIdx.x >> 6] = v[t];
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    int r = red[t][0];
#pragma unroll
    for (int w = 1; w < kPrepWaves; ++w) r += red[t][w];
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
// over each group g of gsize columns (GROUPED: gsize a multiple of 128, so
// the 128 columns of a half wave's loads lie in one group), else over the
// row (ngroups = 1).
constexpr int kPlanesMaxGroups = kPlanesMaxK / 128;
template <bool GROUPED>
__global__ __launch_bounds__(kPrepThreads) void cint8_planes_prep(
    const void* __restrict__ x, int xtype, long long ldx, int k, bool vec, int gsize,
    int ngroups, int8_t* __restrict__ planes, int* __restrict__ rexp, int* __restrict__ dsum) {
  __shared__ float fred[kPrepWaves];
  __shared__ int ired[3][kPrepWaves];
  __shared__ int gsum[GROUPED ? 3 * kPlanesMaxGroups : 1];
  if constexpr (GROUPED) {
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
    if constexpr (GROUPED) {
      // the half wave's 128 columns: one group
#pragma unroll
      for (int t = 0; t < 3; ++t)
        for (int off = 16; off > 0; off >>= 1) sum[t] += __shfl_xor(sum[t], off);
      if ((threadIdx.x & 31) == 0) {
        const int grp = c / gsize;
#pragma unroll
        for (int t = 0; t < 3; ++t) atomicAdd(&gsum[3 * grp + t], sum[t]);
      }
    }
  }
  if constexpr (GROUPED) {
    __syncthreads();
    if (threadIdx.x == 0) rexp[m] = bad ? kPlanesNonfinite : e;
    for (int i = threadIdx.x; i < 3 * ngroups; i += kPrepThreads)
      dsum[3LL * m * ngroups + i] = gsum[i];
  } else {
    block_sum3(sum, ired);
    if (threadIdx.x == 0) {
      rexp[m] = bad ? kPlanesNonfinite : e;
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
// that step's group, the scales (lanes 0-31) and zero points (lanes 32-63;
// the scales again when there are none) of each 32-row block of the tile's
// B rows (slots 0..TS-1), then the digit sums S_0..S_2 of 16 activation rows
// per slot (lanes 0-47).  Slots past those repeat the first scale.  Each
// wave issues kLoads slots; read() keeps, at a group's last step (ready),
// what the wave's fragments need.
template <int TN, int TM, int WGN, int WGM, bool SWIGLU>
struct GroupSide {
  static constexpr int NW = WGN * WGM;
  static constexpr int FN = TN / WGN / 32, FM = TM / WGM / 32;
  static constexpr int TS = TM / 32, TD = (TN / 4 + 15) / 16, T = TS + TD;
  static constexpr int kLoads = (T + NW - 1) / NW;
  const int8_t* src[kLoads];   // this lane's address for group 0
  int stride[kLoads];          // bytes per group (wave-uniform)
  int spg, rleft, wn, wm;
  bool ready;
  float sc[FM], zr[FM];
  int sx[FN][4][3];

  __device__ void init(const PlaneOut& o, const int* dsum, int mc, int tn, int tm, int wave,
                       int wn_, int wm_) {
    const int lane = threadIdx.x & 63;
    spg = o.gsize / 128;
    rleft = spg;
    ready = false;
    wn = wn_;
    wm = wm_;
#pragma unroll
    for (int q = 0; q < kLoads; ++q) {
      const int t = wave * kLoads + q;          // wave-uniform
      if (t < TS) {
        const long long c = static_cast<long long>(tm) * (TM / 32) + t;   // B block
        const bool second = SWIGLU && (c & 1);
        long long n = (SWIGLU ? (c >> 1) * 32 : c * 32) + (lane & 31);
        n = n < o.rows ? n : o.rows - 1;
        const float* scale = second ? o.scale2 : o.scale;
        const float* zero = second ? o.zero2 : o.zero;
        zero = zero != nullptr ? zero : scale;
        src[q] = reinterpret_cast<const int8_t*>(pick(scale, zero, lane >= 32) + n * o.groups);
        stride[q] = 4;
      } else if (t < T) {
        const int l = lane < 48 ? lane : lane - 48;
        int r = tn * (TN / 4) + 16 * (t - TS) + l / 3;
        r = r < mc ? r : mc - 1;
        src[q] = reinterpret_cast<const int8_t*>(dsum + static_cast<long long>(r) * o.groups * 3 +
                                                 l % 3);
        stride[q] = 12;
      } else {
        src[q] = reinterpret_cast<const int8_t*>(o.scale);
        stride[q] = 0;
      }
    }
  }
  __device__ void issue(int step, int wave, int8_t* base) const {
    const int grp = step / spg;
#pragma unroll
    for (int q = 0; q < kLoads; ++q)
      load_lds4(src[q] + grp * stride[q], base + (wave * kLoads + q) * 256);
  }
  __device__ void read(int, const int8_t* base) {
    ready = --rleft == 0;
    if (!ready) return;
    rleft = spg;
    const int lane = threadIdx.x & 63;
    const float* f = reinterpret_cast<const float*>(base);
    const int* v = reinterpret_cast<const int*>(base);
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int bj = wm / 32 + j;
      sc[j] = f[bj * 64 + (lane & 31)];
      zr[j] = f[bj * 64 + 32 + (lane & 31)];
    }
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row = wn / 4 + 8 * i + 2 * g + (lane >> 5);
        const int off = (TS + row / 16) * 64 + (row % 16) * 3;
#pragma unroll
        for (int t = 0; t < 3; ++t) sx[i][g][t] = v[off + t];
      }
  }
};

// The fused form: planes [4 mc][k] (operand A, TN rows per tile) against the
// weight codes (operand B, TM rows per tile), then for each (activation row,
// weight row n) the combination and the shared epilogue, stored as
// y[(m0 + r) * ld + n].  Lanes 0-31 of a store hold 32 consecutive n.  With
// SWIGLU the B tiles pair gate and up blocks (PairedRows): in a wave tile of
// 64 B rows (FM even), fragments j and j + 1 hold gate and up of the same n.
// GROUPED (gsize a multiple of the 128-column K step): at the end of each
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
template <int TN, int TM, int S, int WGN, int WGM, bool SWIGLU, bool GROUPED>
__global__ __launch_bounds__(64 * WGN * WGM) void cint8_planes_gemm(
    const int8_t* __restrict__ planes, int mc, const PlaneOut o, const int* __restrict__ rexp,
    const int* __restrict__ dsum, const void* __restrict__ x, int xtype, long long ldx, int m0,
    int k, int tiles_n, int tiles_m) {
  using R = Int8Ring<TN, TM, S, WGN, WGM, 128>;
  using Side = std::conditional_t<GROUPED, GroupSide<TN, TM, WGN, WGM, SWIGLU>, Int8NoSide>;
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
  auto fold = [&](int, v16i (&a)[R::FN][R::FM]) {
    if constexpr (GROUPED) {
      if (!side.ready) return;                  // uniform: not the group's last step
#pragma unroll
      for (int j = 0; j < R::FM; ++j) {
        // zi: the integral zero point the int32 form subtracts (0 for none,
        // a fractional one or one beyond zlim); zf: the zero point the f32
        // form subtracts (0 for none or an integral one within zlim)
        const float sg = side.sc[j];
        const float z = has_zero ? side.zr[j] : 0.0f;
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
            const int* sx = side.sx[i][g];     // (zi = 0 without zero points)
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
                const int* sx = side.sx[i][g];
                fv[i][g] = fmaf(-zf, combine(sx[0], sx[1], sx[2]), fv[i][g]);
              }
          }
          if (__any(wide)) {                    // integral beyond zlim: exact in int64
#pragma unroll
            for (int i = 0; i < R::FN; ++i)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const int* sx = side.sx[i][g];
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
        // plane row 3 of every activation row is zero: its sums stay 0
#pragma unroll
        for (int i = 0; i < R::FN; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if ((e & 3) != 3) a[i][j][e] = 0;
      }
    }
  };
  if constexpr (SWIGLU)
    R::run_rows(planes, PairedRows{o.w, o.w2, o.rows, k}, 4 * mc, k,
                static_cast<long long>(tn) * TN, static_cast<long long>(tm) * TM, ring, acc, fold,
                &side);
  else
    R::run_rows(planes, Int8Rows{o.w, o.rows, k}, 4 * mc, k, static_cast<long long>(tn) * TN,
                static_cast<long long>(tm) * TM, ring, acc, fold, &side);
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

template <int TN, int TM, int S, int WGN, int WGM, bool SWIGLU, bool GROUPED>
hipError_t launch_planes_gemm(const int8_t* planes, int mc, const PlaneOut& o, const int* rexp,
                              const int* dsum, const void* x, int xtype, long long ldx, int m0,
                              int k, hipStream_t s) {
  const int tiles_n = (4 * mc + TN - 1) / TN;
  // SwiGLU: 64 B rows per 32 output rows
  const long long brows = SWIGLU ? 64LL * ((o.rows + 31) / 32) : o.rows;
  const int tiles_m = static_cast<int>((brows + TM - 1) / TM);
  cint8_planes_gemm<TN, TM, S, WGN, WGM, SWIGLU, GROUPED><<<tiles_n * tiles_m, 64 * WGN * WGM, 0, s>>>(
      planes, mc, o, rexp, dsum, x, xtype, ldx, m0, k, tiles_n, tiles_m);
  return hipGetLastError();
}

// Tile by plane rows: up to 64 activation rows the whole plane matrix in one
// A tile and 64 output rows per workgroup (224 workgroups at N = 14336): 64
// weight rows, or 64 gate and 64 up rows in wave tiles of 64 B rows; up to
// 128 rows two A tiles of 256 by 128 B rows (224 workgroups at N = 14336, where
// 448 of 256 x 64 took 1.4x as long); above, the W8A8 kernel's 256 x 256 tile.
template <bool SWIGLU, bool GROUPED>
hipError_t launch_fused(const int8_t* planes, int mc, const PlaneOut& o, const int* rexp,
                        const int* dsum, const void* x, int xtype, long long ldx, int m0, int k,
                        hipStream_t s) {
  constexpr int TM = SWIGLU ? 128 : 64;
#define QC_PLANES(TN_, TM_, S_, WGN_, WGM_, SW_) \
  launch_planes_gemm<TN_, TM_, S_, WGN_, WGM_, SW_, GROUPED>(planes, mc, o, rexp, dsum, x, xtype, \
                                                             ldx, m0, k, s)
  // (grouped SwiGLU: 5 stages, as its side loads would take 6 past the vmcnt range)
  if (mc <= 8) return QC_PLANES(32, TM, SWIGLU ? (GROUPED ? 5 : 6) : 8, 1, 2, SWIGLU);
  if (mc <= 16) return QC_PLANES(64, TM, SWIGLU ? 4 : 6, 1, 2, SWIGLU);
  if (mc <= 32) return QC_PLANES(128, TM, 4, 2, 2, SWIGLU);
  if (mc <= 64) {
    if constexpr (SWIGLU) return QC_PLANES(256, TM, 3, 4, 2, true);
    else return QC_PLANES(256, TM, 3, 4, 1, false);
  }
  // group sums in registers beside 256 x 256 tiles would spill: 256 x 128 above 64 rows
  if constexpr (GROUPED) {
    return QC_PLANES(256, 128, 3, 4, 2, SWIGLU);
  } else {
    if (mc <= 128) return QC_PLANES(256, 128, 3, 4, 2, SWIGLU);
    return QC_PLANES(256, 256, 2, 4, 2, SWIGLU);
  }
#undef QC_PLANES
}

size_t up256(size_t b) { return (b + 255) / 256 * 256; }

// The call's scratch: buffer 0 of its stream's cache entry, whose call lock
// `hold` keeps until the caller's last launch.
hipError_t call_scratch(hipStream_t s, size_t bytes, std::unique_lock<std::mutex>& hold,
                        void** out) {
  StreamWorkspace* ws = nullptr;
  const hipError_t e = stream_workspace(s, &ws);
  if (e != hipSuccess) return e;
  hold = std::unique_lock<std::mutex>(ws->call);
  return stream_buffer(ws, s, bytes, 0, out);
}

// All checks done by the caller, which routes only 16-byte aligned codes here
// and, with groups, group sizes that are multiples of 128 columns.
template <bool GROUPED>
hipError_t launch_planes(const CSegs& sg, const CInt8Launch& L, int m, int k, hipStream_t s) {
  const int nmat = L.mode == 1 ? 2 : L.nw;
  const size_t es = L.xtype == QC_STORAGE_F32 ? 4 : 2;
  const bool vec = L.xtype == QC_STORAGE_F32 && reinterpret_cast<uintptr_t>(L.x) % 16 == 0 &&
                   L.ldx % 4 == 0;
  const int ngroups = GROUPED ? sg.groups : 1;
  const int gsize = GROUPED ? sg.gsize : k;
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
                                                           ngroups, planes, rexp, dsum);
    e = hipGetLastError();
    if (e == hipSuccess && L.mode == 1) {
      const PlaneOut o{sg.w[0], sg.scale[0], sg.zero[0], sg.w[1], sg.scale[1], sg.zero[1],
                       sg.y[0], sg.ld[0], sg.ytype[0], static_cast<int>(L.w[0].rows),
                       nullptr, 0, 0, ngroups, gsize};
      e = launch_fused<true, GROUPED>(planes, mc, o, rexp, dsum, L.x, L.xtype, L.ldx, m0, k, s);
      continue;
    }
    for (int i = 0; i < nmat && e == hipSuccess; ++i) {
      const PlaneOut o{sg.w[i], sg.scale[i], sg.zero[i], nullptr, nullptr, nullptr, sg.y[i],
                       sg.ld[i], sg.ytype[i], static_cast<int>(L.w[i].rows), sg.bias, sg.act,
                       i == 0 && (sg.bias != nullptr || sg.act != 0) ? 1 : 0, ngroups, gsize};
      e = launch_fused<false, GROUPED>(planes, mc, o, rexp, dsum, L.x, L.xtype, L.ldx, m0, k, s);
    }
  }
  return e;
}

}  // namespace

// Host entry (all checks done by the caller): see CInt8Launch in qc_internal.h.
hipError_t launch_cint8(const CInt8Launch& L, hipStream_t s) {
  CSegs sg{};
  int total = 0;
  sg.nseg = L.mode == 1 ? 1 : L.nw;
  sg.start[0] = 0;
  for (int i = 0; i < L.nw; ++i) {
    sg.w[i] = L.w[i].codes;
    sg.scale[i] = L.w[i].scales;
    sg.zero[i] = L.w[i].zero_points;
    sg.y[i] = L.y[i];
    sg.ytype[i] = L.ytype[i];
    sg.ld[i] = L.mode == 1 ? L.w[0].rows : L.w[i].rows;
  }
  if (L.mode == 1) {
    total = static_cast<int>(2 * L.w[0].rows);
    sg.start[1] = total;
  } else {
    for (int i = 0; i < L.nw; ++i) sg.start[i + 1] = sg.start[i] + static_cast<int>(L.w[i].rows);
    total = sg.start[L.nw];
  }
  sg.mode = L.mode;
  sg.groups = static_cast<int>(L.w[0].groups);
  sg.gsize = static_cast<int>(L.w[0].cols / L.w[0].groups);
  sg.gshift = 0;
  if (sg.groups > 1)
    while ((1 << sg.gshift) < sg.gsize) ++sg.gshift;
  sg.bias = L.bias;
  sg.act = L.act;
  sg.half = L.half;
  sg.nrope = L.nrope;
  sg.rc = L.rope_cos;
  sg.rs = L.rope_sin;
  const int k = static_cast<int>(L.w[0].cols);
  const int m = static_cast<int>(L.m);
  const bool aff = L.w[0].zero_points != nullptr;
  const bool grp = sg.groups > 1;
  bool fast = k % 16 == 0 && (!grp || (sg.gsize >= 16 && (1 << sg.gshift) == sg.gsize));
  for (int i = 0; i < L.nw; ++i)
    fast = fast && reinterpret_cast<uintptr_t>(L.w[i].codes) % 16 == 0;
  // Two or more activation rows with row scales, or three or more with scale
  // groups of a multiple of 128 columns: the digit planes on the int8 MFMA
  // GEMM (row-plane route above).
  if (fast && L.dot == 0 && L.mode != 2 && m >= kPlanesMinM && k % 32 == 0 &&
      k <= kPlanesMaxK) {
    if (!grp) return launch_planes<false>(sg, L, m, k, s);
    if (sg.gsize % 128 == 0 && m >= kPlanesMinMGrouped)
      return launch_planes<true>(sg, L, m, k, s);
  }
  // Exact digit dots over 64-column block pairs, two rows per wave, passes of
  // up to four activation rows
  // (M = 1, K=4096, 14336 rows: 13.9 us against 15.3 / 16.6 us with 4 / 8
  // rows; SwiGLU over 2 x 14336 rows 22.3 against 23.7 / 27.3 us; M = 2 / 4 /
  // 8: 22 / 41 / 82 us against 37 / 61 / 121 us on the f32 kernel).
  if (fast && k % 64 == 0 && (!grp || sg.gsize >= 32) && L.dot >= 0) {
    int rb = 2;
    if (L.rows_per_wave == 2 || L.rows_per_wave == 4 || L.rows_per_wave == 8) rb = L.rows_per_wave;
    if (grp)
      return aff ? launch_dot_rb<true, true>(sg, L.x, L.xtype, L.ldx, m, k, rb, s)
                 : launch_dot_rb<true, false>(sg, L.x, L.xtype, L.ldx, m, k, rb, s);
    return aff ? launch_dot_rb<false, true>(sg, L.x, L.xtype, L.ldx, m, k, rb, s)
               : launch_dot_rb<false, false>(sg, L.x, L.xtype, L.ldx, m, k, rb, s);
  }
  if (fast) {
    const int cus = device_cu_count();
    const bool four = L.rows_per_wave == 2 || L.rows_per_wave == 4
                          ? L.rows_per_wave == 4
                          : (total + kWaves * 4 - 1) / (kWaves * 4) >= 2 * cus;
    if (m == 1)
      return four ? launch_mb<1, 4>(sg, grp, aff, L.x, L.xtype, L.ldx, m, k, s)
                  : launch_mb<1, 2>(sg, grp, aff, L.x, L.xtype, L.ldx, m, k, s);
    if (m == 2)
      return four ? launch_mb<2, 4>(sg, grp, aff, L.x, L.xtype, L.ldx, m, k, s)
                  : launch_mb<2, 2>(sg, grp, aff, L.x, L.xtype, L.ldx, m, k, s);
    return four ? launch_mb<4, 4>(sg, grp, aff, L.x, L.xtype, L.ldx, m, k, s)
                : launch_mb<4, 2>(sg, grp, aff, L.x, L.xtype, L.ldx, m, k, s);
  }
  float* p = nullptr;
  const size_t bytes = sizeof(float) * static_cast<size_t>(total) * m;
  std::unique_lock<std::mutex> hold;
  hipError_t e = call_scratch(s, bytes, hold, reinterpret_cast<void**>(&p));
  if (e != hipSuccess) return e;
  const long long items = static_cast<long long>(total) * m;
  cint8_generic<<<static_cast<unsigned>((items + kWaves - 1) / kWaves), kThreads, 0, s>>>(
      sg, L.x, L.xtype, L.ldx, m, k, p);
  e = hipGetLastError();
  if (e == hipSuccess) {
    const long long units = items / (L.mode == 0 ? 1 : 2);
    cint8_finish<<<static_cast<unsigned>((units + kThreads - 1) / kThreads), kThreads, 0, s>>>(sg, p, m);
    e = hipGetLastError();
  }
  return e;
}

// ---- Decode and storage conversion (model load / inspection, not the
// projection path) -------------------------------------------------------

namespace {

// out[r][c] = scale(r, g) * (float(code[r][c]) - zero(r, g)): the int code
// converted exactly, the zero point subtracted and the scale applied, each
// rounded in f32 (kernels/quantization/quant_import_ref.cpp:753-770);
// g = gidx[c] when a group index is given, else c / gsize.
__global__ __launch_bounds__(kThreads) void cint8_dequant_kernel(
    const int8_t* __restrict__ codes, const float* __restrict__ scales,
    const float* __restrict__ zeros, const int* __restrict__ gidx, long long rows, long long cols,
    long long groups, long long gsize, float* __restrict__ out) {
  const long long total = rows * cols;
  const long long step = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += step) {
    const long long r = i / cols, c = i - r * cols;
    const long long si = r * groups + (gidx != nullptr ? gidx[c] : c / gsize);
    const float z = zeros != nullptr ? zeros[si] : 0.0f;
    out[i] = scales[si] * (static_cast<float>(codes[i]) - z);
  }
}

// f16 / bf16 / f32 storage to f32, exactly (float_storage_to_f32 of
// kernels/utils/float_storage_ref.cpp).
__global__ __launch_bounds__(kThreads) void storage_to_f32_kernel(const void* __restrict__ x,
                                                                  int type, long long count,
                                                                  float* __restrict__ out) {
  const long long step = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += step)
    out[i] = load_x(x, i, type);
}

// y[m][n] = sum_c w(n, c) * a(m, c), each operand decoded as
// scale * (float(code) - zero) in f32, the products accumulated per lane with
// explicit FMAs and summed across the wave: the general canonical int8 x
// int8 projection (group scales, affine weights, activation zero points that
// are not integers), one wave per output.
__global__ __launch_bounds__(kThreads) void cint8_dual_generic(
    const int8_t* __restrict__ wc, const float* __restrict__ ws, const float* __restrict__ wz,
    long long wgroups, const int8_t* __restrict__ ac, const float* __restrict__ as,
    const float* __restrict__ az, long long agroups, long long m, long long n, long long k,
    float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const long long waves = static_cast<long long>(gridDim.x) * kWaves;
  const long long wgs = k / wgroups, ags = k / agroups;
  for (long long o = static_cast<long long>(blockIdx.x) * kWaves + (threadIdx.x >> 6); o < m * n;
       o += waves) {
    const long long mi = o / n, ni = o - mi * n;
    const int8_t* wr = wc + ni * k;
    const int8_t* ar = ac + mi * k;
    float acc = 0.0f;
    for (long long c = lane; c < k; c += 64) {
      const long long gw = ni * wgroups + c / wgs, ga = mi * agroups + c / ags;
      const float wv = ws[gw] * (static_cast<float>(wr[c]) - (wz != nullptr ? wz[gw] : 0.0f));
      const float av = as[ga] * (static_cast<float>(ar[c]) - (az != nullptr ? az[ga] : 0.0f));
      acc = fmaf(wv, av, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[o] = acc;
  }
}

// out[r] = sum_c codes[r][c] in int32 (exact for cols < 2^24), one wave per row.
__global__ __launch_bounds__(kThreads) void cint8_row_sums(const int8_t* __restrict__ codes,
                                                           long long rows, long long cols,
                                                           int32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const long long waves = static_cast<long long>(gridDim.x) * kWaves;
  for (long long r = static_cast<long long>(blockIdx.x) * kWaves + (threadIdx.x >> 6); r < rows;
       r += waves) {
    const int8_t* row = codes + r * cols;
    int sum = 0;
    for (long long c = lane; c < cols; c += 64) sum += row[c];
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if (lane == 0) out[r] = sum;
  }
}

unsigned elementwise_grid(long long count) {
  const long long blocks = (count + kThreads - 1) / kThreads;
  return static_cast<unsigned>(std::min<long long>(std::max<long long>(blocks, 1), 256LL * 16));
}

}  // namespace

hipError_t launch_cint8_dequant(const int8_t* codes, const float* scales, const float* zeros,
                                const int* group_index, long long rows, long long cols,
                                long long groups, long long group_size, float* out,
                                hipStream_t s) {
  cint8_dequant_kernel<<<elementwise_grid(rows * cols), kThreads, 0, s>>>(
      codes, scales, zeros, group_index, rows, cols, groups, group_size, out);
  return hipGetLastError();
}

hipError_t launch_cint8_dual(const qc_cint8_weights& w, const qc_cint8_weights& a,
                             const int* a_int_zero_points, float* y, int int8_route,
                             hipStream_t s) {
  const long long m = a.rows, n = w.rows, k = w.cols;
  const bool mfma = w.zero_points == nullptr && w.groups == 1 && a.groups == 1 &&
                    (a.zero_points == nullptr || a_int_zero_points != nullptr);
  if (!mfma) {
    const long long waves = m * n;
    const unsigned grid = static_cast<unsigned>(
        std::min<long long>((waves + kWaves - 1) / kWaves, 256LL * 64));
    cint8_dual_generic<<<grid, kThreads, 0, s>>>(w.codes, w.scales, w.zero_points, w.groups,
                                                 a.codes, a.scales, a.zero_points, a.groups, m,
                                                 n, k, y);
    return hipGetLastError();
  }
  if (a.zero_points == nullptr)
    return launch_int8_gemm(w.codes, a.codes, w.scales, a.scales, nullptr, nullptr, y, nullptr,
                            m, n, k, false, nullptr, s, int8_route);
  // affine activations: dot - z * row_sum(w), the weights' row sums summed here
  int32_t* sums = nullptr;
  std::unique_lock<std::mutex> hold;
  hipError_t e = call_scratch(s, sizeof(int32_t) * n, hold, reinterpret_cast<void**>(&sums));
  if (e != hipSuccess) return e;
  const unsigned grid = static_cast<unsigned>(std::min<long long>((n + kWaves - 1) / kWaves, 4096));
  cint8_row_sums<<<grid, kThreads, 0, s>>>(w.codes, n, k, sums);
  e = hipGetLastError();
  if (e == hipSuccess)
    e = launch_int8_gemm(w.codes, a.codes, w.scales, a.scales, sums, a_int_zero_points, y,
                         nullptr, m, n, k, true, nullptr, s, int8_route);
  return e;
}

hipError_t launch_storage_to_f32(const void* x, int type, long long count, float* out,
                                 hipStream_t s) {
  storage_to_f32_kernel<<<elementwise_grid(count), kThreads, 0, s>>>(x, type, count, out);
  return hipGetLastError();
}

}  // namespace qc
