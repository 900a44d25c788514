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

#include "qc_cint8.h"
#include "qc_device.h"
#include "qc_digits.h"
#include "qc_internal.h"

namespace qc {
namespace {

constexpr int kThreads = 256;   // 4 waves
constexpr int kWaves = kThreads / 64;

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

// M = 1 with exact digit dots (the GEMV's encoding of x, qc_digits.h):
// k % 64 == 0, 16-byte aligned codes, GRP groups a power of two >= 32.
// Wave w of workgroup b owns logical rows (b * kWaves + w) * RB + r; lane l
// the block pair p = l (mod 64) of each row in every chunk of up to 4096
// columns, its 64 codes in four 16-byte loads issued after the thread's x
// values and before the chunk's digit build.  Per block: f = 2^e (2^14 S0 + 2^7 S1 + S2) ~ sum_j q_j x_j
// (three v_dot4 sums per 4 codes) and, for affine weights, xs = 2^e (2^14
// D0 + 2^7 D1 + D2) ~ sum_j x_j over the same encoded x.  Group scales add
// s_g (f - z_g xs) per block; row scales finish as s (sum f - z sum xs).
//
// WL (K above 4096): each row's 4 KB of a chunk is read in whole lines --
// lane l takes bytes 16 l + 1024 i, non-temporal -- and handed to the lanes
// through a 4 KB staging area per wave (lanes past a short last chunk re-read
// its last bytes).  A lane's own 64-byte pair is half a line: per-lane loads
// re-request lines, and with the hint fetch them twice.
template <int RB, bool GRP, bool AFF, bool WL = false>
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
    const int cbytes = 64 * (pend - pbeg);   // this chunk's bytes of a row (WL)
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (WL) {
          const int off = min(16 * lane + 1024 * i, cbytes - 16);
          const u32x4nt t = __builtin_nontemporal_load(
              reinterpret_cast<const u32x4nt*>(w[r] + 64LL * pbeg + off));
          cw[r][i] = make_uint4(t.x, t.y, t.z, t.w);
        } else {
          cw[r][i] = *reinterpret_cast<const uint4*>(w[r] + 64LL * pc + 16 * i);
        }
      }
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
    if constexpr (WL) {
      // each row's chunk through the wave's staging area, then this lane's pair
      // (wave_lds_sync orders the previous reads before the stores, and the
      // stores before the reads; lanes with a clamped offset store the same
      // bytes as the lane that owns them)
      uint8_t* const stage = lds + (lds_size(kc) + 15) / 16 * 16 + wave * 4096;
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<uint4*>(stage + min(16 * lane + 1024 * i, cbytes - 16)) = cw[r][i];
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 4; ++i)
          cw[r][i] = *reinterpret_cast<const uint4*>(stage + 64 * (pc - pbeg) + 16 * i);
      }
    }
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
    if (k > 4096)
      cint8_dot_kernel<RB, GRP, AFF, true>
          <<<grid, kThreads, (lds_size(4096) + 15) / 16 * 16 + kWaves * 4096, s>>>(sg, x, xtype, k,
                                                                               xvec);
    else
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

hipError_t call_scratch(hipStream_t s, size_t bytes, std::unique_lock<std::mutex>& hold,
                        void** out) {
  StreamWorkspace* ws = nullptr;
  const hipError_t e = stream_workspace(s, &ws);
  if (e != hipSuccess) return e;
  hold = std::unique_lock<std::mutex>(ws->call);
  return stream_buffer(ws, s, bytes, 0, out);
}

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
  // Two or more activation rows with row scales, three or more with scale
  // groups of 64 or a multiple of 128 columns, five or more with groups of
  // 32: the digit planes on the int8 MFMA GEMM (the row-plane route,
  // canonical_planes.hip).
  if (fast && L.dot == 0 && L.mode != 2 && m >= kPlanesMinM && k % 32 == 0 &&
      k <= kPlanesMaxK) {
    if (!grp) return launch_cint8_planes(sg, L, m, k, false, s);
    if ((sg.gsize % 128 == 0 || sg.gsize == 64) && k % 128 == 0 && m >= kPlanesMinMGrouped)
      return launch_cint8_planes(sg, L, m, k, true, s);
    if (sg.gsize == 32 && k % 128 == 0 && m >= kPlanesMinMGroups32)
      return launch_cint8_planes(sg, L, m, k, true, s);
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
