// Producers of the W8A8 GEMM's activations on gfx950: residual add + RMSNorm +
// dynamic int8 quantization, and per-row asymmetric int8 quantization (with
// its dequantization).
//
// rms_norm_add_quant_int8 restates kernels/norms/norm_quant_ref.cpp of the
// reference as its x86-64 build runs it, bit for bit:
//   value = x + residual (f32), stored to residual_out                (82-86)
//   sumsq = sum of double(value)^2 in element order                   (82-86)
//   inverse = float(1 / sqrt(sumsq / hidden + eps)) in double         (88-89)
//   normalized = (value * inverse) * weight (f32)                       (103)
//   per group: scale = max|normalized| / 127, inv = scale > 0 ? 1/scale : 0,
//   code = clamp(rint(normalized * inv), -127, 127); a group holding a
//   non-finite normalized value is skipped (no scale, no codes) and the call
//   reports kInvalidArgument                                   (150-168, 283-290)
// The squares are exact in double and non-negative, so a parallel sum of
// them lies within a factor (1 +- 3 hidden 2^-53) of the element-order sum,
// and f(S) = float(1 / sqrt(S / hidden + eps)) is monotone in S (every step is
// a correctly rounded monotone operation).  When f takes one value at both
// ends of that interval around the parallel sum, it is the reference's
// value; otherwise (a row on a float rounding boundary) the workgroup replays
// the element-order sum.  Double division and sqrt are IEEE correctly rounded
// on this target, f32 division too, and the file is built with
// -ffp-contract=off.
//
// quantize_int8_asymmetric restates kernels/quantization/quantization_ref.cpp:
// 190-226 in double, with static_cast<int> of an out-of-range double giving
// INT_MIN and int additions wrapping, as the reference's x86-64 build does.
// Each code's rint(x / scale) comes from an f32 product wherever that provably
// equals the double quotient's rounding (asym_fast), else from the division.
#include "qc_device.h"
#include "qc_internal.h"

namespace qc {
namespace {

__device__ __forceinline__ int8_t code127(float v, float inv) {
  int q = static_cast<int>(rintf(v * inv));
  q = q < -127 ? -127 : (q > 127 ? 127 : q);
  return static_cast<int8_t>(q);
}

__device__ __forceinline__ uint32_t codes4(float4 v, float inv) {
  const uint32_t a = static_cast<uint8_t>(code127(v.x, inv));
  const uint32_t b = static_cast<uint8_t>(code127(v.y, inv));
  const uint32_t c = static_cast<uint8_t>(code127(v.z, inv));
  const uint32_t d = static_cast<uint8_t>(code127(v.w, inv));
  return a | (b << 8) | (c << 16) | (d << 24);
}

__device__ __forceinline__ bool finite4(float4 v) {
  return isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w);
}

__device__ __forceinline__ float absmax4(float4 v, float m) {
  return fmaxf(fmaxf(fmaxf(m, fabsf(v.x)), fmaxf(fabsf(v.y), fabsf(v.z))), fabsf(v.w));
}

__device__ __forceinline__ double sumsq4(float4 v, double s) {
  s += static_cast<double>(v.x) * v.x;
  s += static_cast<double>(v.y) * v.y;
  s += static_cast<double>(v.z) * v.z;
  s += static_cast<double>(v.w) * v.w;
  return s;
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ float4 normalize4(float4 v, float inv, float4 w) {
  return make_float4((v.x * inv) * w.x, (v.y * inv) * w.y, (v.z * inv) * w.z,
                     (v.w * inv) * w.w);
}

__device__ __forceinline__ float rms_inverse(double sumsq, double hidden, double eps) {
  return static_cast<float>(1.0 / sqrt(sumsq / hidden + eps));
}

// inverse from a sum taken in any order, when provably equal to the
// element-order sum's (see the header).  A non-finite sum (an inf or NaN
// value) is the same in every order: no double overflow is possible for
// squares of floats.
__device__ __forceinline__ bool settled_inverse(double s, double hidden, double eps, float* inv) {
  if (!(s <= 1.7976931348623157e308)) {
    *inv = rms_inverse(s, hidden, eps);
    return true;
  }
  const double d = 3.0 * hidden * 0x1p-53;
  const float a = rms_inverse(s * (1.0 - d), hidden, eps);
  const float b = rms_inverse(s * (1.0 + d), hidden, eps);
  *inv = a;
  return __float_as_uint(a) == __float_as_uint(b);
}

// Workgroup sum of a double, returned to every thread (any order).
template <int NT>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double s = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) s += red[w];
  return s;
}

// Workgroup max of non-negative floats and OR of a flag, returned to every thread.
template <int NT>
__device__ __forceinline__ void block_max_any(float& m, int& bad, float* smax, int* sbad) {
  m = wave_max_nonneg(m);
  bad = __any(bad) ? 1 : 0;
  if ((threadIdx.x & 63) == 0) {
    smax[threadIdx.x >> 6] = m;
    sbad[threadIdx.x >> 6] = bad;
  }
  __syncthreads();
  m = smax[0];
  bad = sbad[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) {
    m = fmaxf(m, smax[w]);
    bad |= sbad[w];
  }
}

// One workgroup of NT threads per row, the row in registers (V float4 per
// thread; float4 index t + i * NT).  G4 = group size / 4 for groups of 4..256
// columns (a group is G4 adjacent lanes), 0 for one group per row.  Requires
// hidden % 4 == 0, 4 <= hidden <= 4 * NT * V, 16-byte aligned x / residual /
// weight / residual_out and 4-byte aligned codes.  residual_out may alias x
// or residual (each element is read before it is written, by one thread).
template <int V, int NT, int G4>
__global__ __launch_bounds__(NT) void rms_norm_quant_rows(
    const float* x, const float* residual, const float* __restrict__ weight, int8_t* codes,
    float* residual_out, float* __restrict__ scales, int hidden, float eps, int force_seq,
    int* status) {
  __shared__ double red[NT / 64];
  __shared__ float smax[NT / 64];
  __shared__ int sbad[NT / 64];
  __shared__ float4 stage[NT];
  __shared__ float sinv;
  const long long base = static_cast<long long>(blockIdx.x) * hidden;
  const float4* x4 = reinterpret_cast<const float4*>(x + base);
  const float4* r4 = reinterpret_cast<const float4*>(residual + base);
  const float4* w4 = reinterpret_cast<const float4*>(weight);
  float4* o4 = reinterpret_cast<float4*>(residual_out + base);
  uint32_t* c4 = reinterpret_cast<uint32_t*>(codes + base);
  const int n4 = hidden >> 2;
  const int t = threadIdx.x;

  // Every lane issues all 2V loads (a lane past the row re-reads the row's
  // last float4 and ignores it), so they are in flight together: a load
  // inside `if (idx < n4)` was waited for before the next one was issued.
  float4 v[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = t + i * NT;
    const int li = idx < n4 ? idx : n4 - 1;
    v[i] = add4(x4[li], r4[li]);
  }
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = t + i * NT;
    if (idx < n4) {
      o4[idx] = v[i];
      ss = sumsq4(v[i], ss);
    }
  }
  const double hd = static_cast<double>(hidden), ed = static_cast<double>(eps);
  float inv = 0.f;
  const bool settled = settled_inverse(block_sum_f64<NT>(ss, red), hd, ed, &inv) && !force_seq;
  if (!settled) {
    // element-order replay: chunk i of the row is v[i] of every thread
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      if (i * NT < n4) {
        __syncthreads();
        if (t + i * NT < n4) stage[t] = v[i];
        __syncthreads();
        if (t == 0) {
          const int cnt = min(NT, n4 - i * NT);
          for (int j = 0; j < cnt; ++j) s = sumsq4(stage[j], s);
        }
      }
    }
    if (t == 0) sinv = rms_inverse(s, hd, ed);
    __syncthreads();
    inv = sinv;
  }

#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = t + i * NT;
    if (idx < n4) v[i] = normalize4(v[i], inv, w4[idx]);
  }
  const int groups = G4 == 0 ? 1 : n4 / G4;
  if constexpr (G4 == 0) {
    float m = 0.f;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      if (t + i * NT < n4) {
        bad |= !finite4(v[i]);
        m = absmax4(v[i], m);
      }
    }
    block_max_any<NT>(m, bad, smax, sbad);
    if (bad) {
      if (t == 0) *status = 3;
      return;
    }
    const float scale = m / 127.0f;
    const float qinv = scale > 0.f ? 1.0f / scale : 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int idx = t + i * NT;
      if (idx < n4) c4[idx] = codes4(v[i], qinv);
    }
    if (t == 0) scales[blockIdx.x] = scale;
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int idx = t + i * NT;
      // G4 divides 64 and NT, so a group is G4 adjacent lanes of one wave and
      // idx < n4 holds for all of them or none (n4 is a multiple of G4)
      float m = idx < n4 ? absmax4(v[i], 0.f) : 0.f;
      int bad = idx < n4 ? !finite4(v[i]) : 0;
#pragma unroll
      for (int o = 1; o < G4; o <<= 1) {
        m = fmaxf(m, __shfl_xor(m, o));
        bad |= __shfl_xor(bad, o);
      }
      if (idx < n4) {
        if (bad) {
          if (idx % G4 == 0) *status = 3;
        } else {
          const float scale = m / 127.0f;
          const float qinv = scale > 0.f ? 1.0f / scale : 0.f;
          c4[idx] = codes4(v[i], qinv);
          if (idx % G4 == 0) scales[static_cast<long long>(blockIdx.x) * groups + idx / G4] = scale;
        }
      }
    }
  }
}

// Any layout: one workgroup per row, element loops over global memory (the
// normalized values are recomputed from residual_out, which this workgroup
// wrote before a barrier), one wavefront per group.
constexpr int kGenThreads = 256;

__global__ __launch_bounds__(kGenThreads) void rms_norm_quant_generic(
    const float* x, const float* residual, const float* __restrict__ weight, int8_t* codes,
    float* residual_out, float* __restrict__ scales, long long hidden, long long group,
    float eps, int force_seq, int* status) {
  __shared__ double red[kGenThreads / 64];
  __shared__ float stage[kGenThreads];
  __shared__ float sinv;
  const long long base = static_cast<long long>(blockIdx.x) * hidden;
  const int t = threadIdx.x;
  double ss = 0.0;
  for (long long i = t; i < hidden; i += kGenThreads) {
    const float v = x[base + i] + residual[base + i];
    residual_out[base + i] = v;
    ss += static_cast<double>(v) * v;
  }
  const double hd = static_cast<double>(hidden), ed = static_cast<double>(eps);
  float inv = 0.f;
  const bool settled =
      settled_inverse(block_sum_f64<kGenThreads>(ss, red), hd, ed, &inv) && !force_seq;
  if (!settled) {
    double s = 0.0;
    for (long long c = 0; c < hidden; c += kGenThreads) {
      __syncthreads();
      if (c + t < hidden) stage[t] = residual_out[base + c + t];
      __syncthreads();
      if (t == 0) {
        const long long cnt = min(static_cast<long long>(kGenThreads), hidden - c);
        for (long long j = 0; j < cnt; ++j) s += static_cast<double>(stage[j]) * stage[j];
      }
    }
    if (t == 0) sinv = rms_inverse(s, hd, ed);
  }
  __syncthreads();   // residual_out complete (and sinv) for the whole workgroup
  if (!settled) inv = sinv;

  const int lane = t & 63;
  const long long groups = hidden / group;
  for (long long g = t >> 6; g < groups; g += kGenThreads / 64) {
    const long long g0 = base + g * group;
    float m = 0.f;
    int bad = 0;
    for (long long j = lane; j < group; j += 64) {
      const float n = (residual_out[g0 + j] * inv) * weight[g * group + j];
      bad |= !isfinite(n);
      m = fmaxf(m, fabsf(n));
    }
    m = wave_max_nonneg(m);
    if (__any(bad)) {
      if (lane == 0) *status = 3;
      continue;
    }
    const float scale = m / 127.0f;
    const float qinv = scale > 0.f ? 1.0f / scale : 0.f;
    for (long long j = lane; j < group; j += 64)
      codes[g0 + j] = code127((residual_out[g0 + j] * inv) * weight[g * group + j], qinv);
    if (lane == 0) scales[static_cast<long long>(blockIdx.x) * groups + g] = scale;
  }
}

// ------------------------------------------------- asymmetric int8 ---

// static_cast<int>(double) as an x86-64 build executes it (cvttsd2si):
// truncation, and INT_MIN for NaN or a value outside the int range.
__device__ __forceinline__ int x86_int(double d) {
  return (d > -2147483649.0 && d < 2147483648.0) ? static_cast<int>(d) : INT_MIN;
}

// rint(v / sv) as the reference rounds it (the IEEE double quotient, half to
// even), mostly without a division.  With rs = f32(RN(1 / sv)), the f32
// product t = v * rs is (v / sv)(1 + e) with |e| <= 2^-23 (1 + 2^-22) (two f32
// roundings and one double), and the double quotient D is (v / sv)(1 + e')
// with |e'| <= 2^-53, so |t - D| < 2^-22.9 |t|.  Where t lies farther than
// 2^-21 |t| from every half-integer, no half-integer separates t from D and
// rintf(t) == rint(D); below |t| = 1/8 both round to zero.  Exact ties
// (v / sv = k + 1/2), |t| >= 2^21 and a non-finite t (1 / sv beyond the f32
// range) fail the test and take the division.  f32 denormals are kept on
// this target, so subnormal v and t stay within the bound.
__device__ __forceinline__ bool asym_fast(float v, float rs, int& q) {
  const float t = v * rs;
  const float r = rintf(t);
  const bool ok = fabsf(t - r) < 0.5f - fabsf(t) * 0x1p-21f;
  q = ok ? static_cast<int>(r) : 0;
  return ok;
}

__device__ __forceinline__ int asym_exact(float v, double sv) {
  return x86_int(rint(static_cast<double>(v) / sv));
}

// The code of rounded quotient q: q + zero with 32-bit wrap, saturated to int8.
__device__ __forceinline__ uint32_t asym_byte(int q, int zero) {
  int c = static_cast<int>(static_cast<uint32_t>(q) + static_cast<uint32_t>(zero));
  c = c < -128 ? -128 : (c > 127 ? 127 : c);
  return static_cast<uint8_t>(static_cast<int8_t>(c));
}

__device__ __forceinline__ int8_t asym_code(float v, double sv, float rs, int zero) {
  int q;
  if (!asym_fast(v, rs, q)) q = asym_exact(v, sv);
  return static_cast<int8_t>(asym_byte(q, zero));
}

__device__ __forceinline__ uint32_t asym_codes4(float4 v, double sv, float rs, int zero) {
  return static_cast<uint32_t>(static_cast<uint8_t>(asym_code(v.x, sv, rs, zero))) |
         (static_cast<uint32_t>(static_cast<uint8_t>(asym_code(v.y, sv, rs, zero))) << 8) |
         (static_cast<uint32_t>(static_cast<uint8_t>(asym_code(v.z, sv, rs, zero))) << 16) |
         (static_cast<uint32_t>(static_cast<uint8_t>(asym_code(v.w, sv, rs, zero))) << 24);
}

constexpr int kAsymThreads = 256;

// One workgroup per row: min / max (exact in any order), the row's affine
// parameters in double, then the codes.  A row holding a non-finite value is
// left unwritten and sets *status (asynchronous form; the synchronous form
// rejects such input before launching).
template <bool VEC>
__global__ __launch_bounds__(kAsymThreads) void quantize_asym_rows(
    const float* __restrict__ x, int8_t* __restrict__ codes, float* __restrict__ scales,
    int* __restrict__ zero_points, long long dim, int* status) {
  __shared__ float slo[kAsymThreads / 64], shi[kAsymThreads / 64];
  __shared__ int sbad[kAsymThreads / 64];
  const long long row = blockIdx.x;
  const float* xr = x + row * dim;
  const int t = threadIdx.x;
  float lo = INFINITY, hi = -INFINITY;
  int bad = 0;
  if constexpr (VEC) {
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    for (long long i = t; i < dim / 4; i += kAsymThreads) {
      const float4 v = x4[i];
      bad |= !finite4(v);
      lo = fminf(fminf(lo, v.x), fminf(v.y, fminf(v.z, v.w)));
      hi = fmaxf(fmaxf(hi, v.x), fmaxf(v.y, fmaxf(v.z, v.w)));
    }
  } else {
    for (long long i = t; i < dim; i += kAsymThreads) {
      const float v = xr[i];
      bad |= !isfinite(v);
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, o));
    hi = fmaxf(hi, __shfl_xor(hi, o));
  }
  bad = __any(bad) ? 1 : 0;
  if ((t & 63) == 0) {
    slo[t >> 6] = lo;
    shi[t >> 6] = hi;
    sbad[t >> 6] = bad;
  }
  __syncthreads();
  lo = slo[0];
  hi = shi[0];
  bad = sbad[0];
#pragma unroll
  for (int w = 1; w < kAsymThreads / 64; ++w) {
    lo = fminf(lo, slo[w]);
    hi = fmaxf(hi, shi[w]);
    bad |= sbad[w];
  }
  if (bad) {
    if (t == 0 && status != nullptr) *status = 3;
    return;
  }
  // The sign of a zero minimum or maximum changes none of the values below.
  const double minimum = lo, maximum = hi;
  const double range = maximum - minimum;
  double sv;
  if (range > 0.0) {
    sv = range / 255.0;
  } else {
    const double a = fabs(minimum) / 127.0;
    sv = a < 1e-7 ? 1e-7 : a;
  }
  const int zero = x86_int(rint(-128.0 - minimum / sv));
  const float rs = static_cast<float>(1.0 / sv);
  if (t == 0) {
    scales[row] = static_cast<float>(sv);
    zero_points[row] = zero;
  }
  int8_t* cr = codes + row * dim;
  if constexpr (VEC) {
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    uint32_t* c4 = reinterpret_cast<uint32_t*>(cr);
    for (long long i = t; i < dim / 4; i += kAsymThreads) {
      const float4 v = x4[i];
      c4[i] = asym_codes4(v, sv, rs, zero);
    }
  } else {
    for (long long i = t; i < dim; i += kAsymThreads) cr[i] = asym_code(xr[i], sv, rs, zero);
  }
}


// The same with the row held in registers (V float4 per thread): one read
// of x.  Requires dim % 4 == 0, 4 <= dim <= 4 * NT * V, x 16-byte and codes
// 4-byte aligned.
template <int V, int NT>
__global__ __launch_bounds__(NT) void quantize_asym_rows_regs(
    const float* __restrict__ x, int8_t* __restrict__ codes, float* __restrict__ scales,
    int* __restrict__ zero_points, int dim, int* status) {
  __shared__ float slo[NT / 64], shi[NT / 64];
  __shared__ int sbad[NT / 64];
  const long long row = blockIdx.x;
  const float4* x4 = reinterpret_cast<const float4*>(x + row * dim);
  uint32_t* c4 = reinterpret_cast<uint32_t*>(codes + row * dim);
  const int n4 = dim >> 2;
  const int t = threadIdx.x;
  float4 v[V];
  float lo = INFINITY, hi = -INFINITY;
  int bad = 0;
  // All V loads in flight together, as in quantize_rows_regs (a lane past the
  // row re-reads its last float4 and ignores it); x is read once and the
  // codes written once: non-temporal loads and stores.
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = t + i * NT;
    const u32x4nt u = __builtin_nontemporal_load(reinterpret_cast<const u32x4nt*>(x4) +
                                                 (idx < n4 ? idx : n4 - 1));
    v[i] = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                       __uint_as_float(u.w));
  }
#pragma unroll
  for (int i = 0; i < V; ++i) {
    if (t + i * NT < n4) {
      bad |= !finite4(v[i]);
      lo = fminf(fminf(lo, v[i].x), fminf(v[i].y, fminf(v[i].z, v[i].w)));
      hi = fmaxf(fmaxf(hi, v[i].x), fmaxf(v[i].y, fmaxf(v[i].z, v[i].w)));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, o));
    hi = fmaxf(hi, __shfl_xor(hi, o));
  }
  bad = __any(bad) ? 1 : 0;
  if ((t & 63) == 0) {
    slo[t >> 6] = lo;
    shi[t >> 6] = hi;
    sbad[t >> 6] = bad;
  }
  __syncthreads();
  lo = slo[0];
  hi = shi[0];
  bad = sbad[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) {
    lo = fminf(lo, slo[w]);
    hi = fmaxf(hi, shi[w]);
    bad |= sbad[w];
  }
  if (bad) {
    if (t == 0 && status != nullptr) *status = 3;
    return;
  }
  const double minimum = lo, maximum = hi;
  const double range = maximum - minimum;
  double sv;
  if (range > 0.0) {
    sv = range / 255.0;
  } else {
    const double a = fabs(minimum) / 127.0;
    sv = a < 1e-7 ? 1e-7 : a;
  }
  const int zero = x86_int(rint(-128.0 - minimum / sv));
  const float rs = static_cast<float>(1.0 / sv);
  if (t == 0) {
    scales[row] = static_cast<float>(sv);
    zero_points[row] = zero;
  }
  // The f32 estimate for every value first; the few that fail its test (one
  // bit each in slow) take the division in one branch per thread.
  int q[V][4];
  uint32_t slow = 0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    q[i][0] = q[i][1] = q[i][2] = q[i][3] = 0;
    if (t + i * NT < n4) {
      slow |= (asym_fast(v[i].x, rs, q[i][0]) ? 0u : 1u) << (4 * i);
      slow |= (asym_fast(v[i].y, rs, q[i][1]) ? 0u : 2u) << (4 * i);
      slow |= (asym_fast(v[i].z, rs, q[i][2]) ? 0u : 4u) << (4 * i);
      slow |= (asym_fast(v[i].w, rs, q[i][3]) ? 0u : 8u) << (4 * i);
    }
  }
  if (slow != 0) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      if (slow & (1u << (4 * i))) q[i][0] = asym_exact(v[i].x, sv);
      if (slow & (2u << (4 * i))) q[i][1] = asym_exact(v[i].y, sv);
      if (slow & (4u << (4 * i))) q[i][2] = asym_exact(v[i].z, sv);
      if (slow & (8u << (4 * i))) q[i][3] = asym_exact(v[i].w, sv);
    }
  }
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = t + i * NT;
    if (idx < n4)
      __builtin_nontemporal_store(asym_byte(q[i][0], zero) | (asym_byte(q[i][1], zero) << 8) |
                                      (asym_byte(q[i][2], zero) << 16) |
                                      (asym_byte(q[i][3], zero) << 24),
                                  c4 + idx);
  }
}

// out = scale[row] * float(int(code) - zero_point[row]) (wrapping subtraction).
__global__ __launch_bounds__(256) void dequantize_asym(const int8_t* __restrict__ codes,
                                                       const float* __restrict__ scales,
                                                       const int* __restrict__ zero_points,
                                                       float* __restrict__ out, long long rows,
                                                       long long dim) {
  const long long total = rows * dim;
  const long long stride = static_cast<long long>(gridDim.x) * 256;
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += stride) {
    const long long r = i / dim;
    const int d = static_cast<int>(static_cast<uint32_t>(static_cast<int>(codes[i])) -
                                   static_cast<uint32_t>(zero_points[r]));
    out[i] = scales[r] * static_cast<float>(d);
  }
}

template <int V, int NT>
hipError_t launch_rows_v(int g4, unsigned grid, const float* x, const float* r, const float* w,
                         int8_t* c, float* ro, float* sc, int hidden, float eps, int force,
                         int* status, hipStream_t s) {
  switch (g4) {
    case 0: rms_norm_quant_rows<V, NT, 0><<<grid, NT, 0, s>>>(x, r, w, c, ro, sc, hidden, eps, force, status); break;
    case 1: rms_norm_quant_rows<V, NT, 1><<<grid, NT, 0, s>>>(x, r, w, c, ro, sc, hidden, eps, force, status); break;
    case 2: rms_norm_quant_rows<V, NT, 2><<<grid, NT, 0, s>>>(x, r, w, c, ro, sc, hidden, eps, force, status); break;
    case 4: rms_norm_quant_rows<V, NT, 4><<<grid, NT, 0, s>>>(x, r, w, c, ro, sc, hidden, eps, force, status); break;
    case 8: rms_norm_quant_rows<V, NT, 8><<<grid, NT, 0, s>>>(x, r, w, c, ro, sc, hidden, eps, force, status); break;
    case 16: rms_norm_quant_rows<V, NT, 16><<<grid, NT, 0, s>>>(x, r, w, c, ro, sc, hidden, eps, force, status); break;
    case 32: rms_norm_quant_rows<V, NT, 32><<<grid, NT, 0, s>>>(x, r, w, c, ro, sc, hidden, eps, force, status); break;
    default: rms_norm_quant_rows<V, NT, 64><<<grid, NT, 0, s>>>(x, r, w, c, ro, sc, hidden, eps, force, status); break;
  }
  return hipGetLastError();
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

hipError_t launch_rms_norm_add_quant_int8(const float* x, const float* residual,
                                          const float* weight, int8_t* codes,
                                          float* residual_out, float* scales, long long rows,
                                          long long hidden, float eps, long long group,
                                          bool force_sequential, int* status, hipStream_t s) {
  const int force = force_sequential ? 1 : 0;
  // groups of 4..256 columns that are a power of two, or one group per row
  const long long g4 = group == hidden ? 0 : group / 4;
  const bool small_group = group % 4 == 0 && g4 >= 1 && g4 <= 64 && (g4 & (g4 - 1)) == 0;
  const bool fast = hidden % 4 == 0 && hidden >= 4 && hidden <= 32768 &&
                    (group == hidden || small_group) &&
                    aligned16(x) && aligned16(residual) && aligned16(weight) &&
                    aligned16(residual_out) && reinterpret_cast<uintptr_t>(codes) % 4 == 0 &&
                    rows <= 0x7FFFFFFFLL;
  if (fast) {
    const unsigned grid = static_cast<unsigned>(rows);
    const int h = static_cast<int>(hidden), g = static_cast<int>(g4);
    if (hidden <= 1024)
      return launch_rows_v<1, 256>(g, grid, x, residual, weight, codes, residual_out, scales, h, eps, force, status, s);
    if (hidden <= 2048)
      return launch_rows_v<2, 256>(g, grid, x, residual, weight, codes, residual_out, scales, h, eps, force, status, s);
    if (hidden <= 4096)
      return launch_rows_v<4, 256>(g, grid, x, residual, weight, codes, residual_out, scales, h, eps, force, status, s);
    if (hidden <= 8192)
      return launch_rows_v<8, 256>(g, grid, x, residual, weight, codes, residual_out, scales, h, eps, force, status, s);
    if (hidden <= 16384)
      return launch_rows_v<8, 512>(g, grid, x, residual, weight, codes, residual_out, scales, h, eps, force, status, s);
    return launch_rows_v<8, 1024>(g, grid, x, residual, weight, codes, residual_out, scales, h, eps, force, status, s);
  }
  if (rows > 0x7FFFFFFFLL) return hipErrorInvalidValue;
  rms_norm_quant_generic<<<static_cast<unsigned>(rows), kGenThreads, 0, s>>>(
      x, residual, weight, codes, residual_out, scales, hidden, group, eps, force, status);
  return hipGetLastError();
}

hipError_t launch_quantize_int8_asymmetric(const float* x, int8_t* codes, float* scales,
                                           int* zero_points, long long rows, long long dim,
                                           int* status, hipStream_t s) {
  if (rows > 0x7FFFFFFFLL) return hipErrorInvalidValue;
  const unsigned grid = static_cast<unsigned>(rows);
  const bool vec = dim % 4 == 0 && aligned16(x) && reinterpret_cast<uintptr_t>(codes) % 4 == 0;
  if (vec && dim >= 4 && dim <= 32768) {
    const int d = static_cast<int>(dim);
    if (dim <= 1024)
      quantize_asym_rows_regs<1, 256><<<grid, 256, 0, s>>>(x, codes, scales, zero_points, d, status);
    else if (dim <= 2048)
      quantize_asym_rows_regs<2, 256><<<grid, 256, 0, s>>>(x, codes, scales, zero_points, d, status);
    else if (dim <= 4096)
      quantize_asym_rows_regs<4, 256><<<grid, 256, 0, s>>>(x, codes, scales, zero_points, d, status);
    else if (dim <= 8192)
      quantize_asym_rows_regs<8, 256><<<grid, 256, 0, s>>>(x, codes, scales, zero_points, d, status);
    else if (dim <= 16384)
      quantize_asym_rows_regs<8, 512><<<grid, 512, 0, s>>>(x, codes, scales, zero_points, d, status);
    else
      quantize_asym_rows_regs<8, 1024><<<grid, 1024, 0, s>>>(x, codes, scales, zero_points, d, status);
    return hipGetLastError();
  }
  if (vec)
    quantize_asym_rows<true><<<grid, kAsymThreads, 0, s>>>(x, codes, scales, zero_points, dim, status);
  else
    quantize_asym_rows<false><<<grid, kAsymThreads, 0, s>>>(x, codes, scales, zero_points, dim, status);
  return hipGetLastError();
}

hipError_t launch_dequantize_int8_asymmetric(const int8_t* codes, const float* scales,
                                             const int* zero_points, float* out, long long rows,
                                             long long dim, hipStream_t s) {
  long long blocks = (rows * dim + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  dequantize_asym<<<static_cast<unsigned>(blocks), 256, 0, s>>>(codes, scales, zero_points, out,
                                                                rows, dim);
  return hipGetLastError();
}

}  // namespace qc
