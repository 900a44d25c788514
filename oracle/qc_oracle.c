/*
 * CPU oracle for the quantized-matmul hot path -- TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, and only as the checker.  The product library never links it.
 *
 * Restates, in plain C, the reference algorithms of QuixiAI/QuixiCore-CPU
 * (paths relative to the reference root).  Compiled with -ffp-contract=off.
 */
#include "qc_oracle.h"

#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 --- */

/* IEEE binary16 -> binary32, exact for every code (subnormals, +-0, inf,
 * NaN payload shifted into the f32 mantissa).
 * Follows kernels/common/fp16.h:11-37; written via ldexpf, not bit-renormalization. */
float qco_fp16_to_fp32(uint16_t h) {
  const int exponent = (h >> 10) & 31;
  const uint32_t mantissa = h & 1023u;
  if (exponent == 31) {
    uint32_t bits = ((uint32_t)(h & 0x8000u) << 16) | 0x7F800000u | (mantissa << 13);
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
  }
  const float magnitude = exponent == 0
                              ? ldexpf((float)mantissa, -24)
                              : ldexpf((float)(mantissa | 1024u), exponent - 25);
  return (h & 0x8000u) ? -magnitude : magnitude;
}

/* binary32 -> binary16, round to nearest even, overflow -> inf, NaN -> 0x7E00
 * with the sign kept.  Follows kernels/common/fp16.h:39-75; computed through
 * an exact double scaling and rint (RNE), not the reference's bit shifts. */
uint16_t qco_fp32_to_fp16(float f) {
  uint32_t bits;
  memcpy(&bits, &f, sizeof bits);
  const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  const uint32_t magnitude_bits = bits & 0x7FFFFFFFu;
  if (magnitude_bits > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (magnitude_bits == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
  const double a = fabs((double)f);
  if (a == 0.0) return sign;
  int e2 = 0;
  const double v = frexp(a, &e2); /* a = v * 2^e2, v in [0.5, 1) */
  int field = e2 + 14;            /* biased half exponent of a = 1.m * 2^(e2-1) */
  if (field >= 1) {
    double q = rint(ldexp(v, 11)); /* 11 significant bits, in [1024, 2048] */
    if (q == 2048.0) {
      q = 1024.0;
      ++field;
    }
    if (field >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (uint16_t)(field << 10) | (uint16_t)((uint32_t)q - 1024u));
  }
  /* half subnormal: units of 2^-24; 1024 units is the smallest normal 0x0400 */
  const double q = rint(ldexp(a, 24));
  return (uint16_t)(sign | (uint16_t)q);
}

/* ------------------------------------------------------------- formats --- */

/* gguf_format_info: kernels/quantization/gguf_ref.cpp:509-510 (q8_0 32/34, q4_0 32/18). */
static int block_bytes_of(int format) {
  return format == QCO_Q8_0 ? 34 : (format == QCO_Q4_0 ? 18 : 0);
}

/* validate + packed_size: src/dispatch/qgemv.cpp:125-164. */
static int validate_shape(int format, long long n, long long k) {
  if (block_bytes_of(format) == 0) return QCO_UNSUPPORTED_FORMAT;
  if (n <= 0 || k <= 0 || k % 32 != 0) return QCO_INVALID_SHAPE;
  if (n > LLONG_MAX / k || n > LLONG_MAX / (k / 32)) return QCO_INVALID_SHAPE;
  return QCO_OK;
}

int qco_packed_size(int format, long long n, long long k, size_t* size) {
  const int status = validate_shape(format, n, k);
  if (status != QCO_OK) return status;
  if (size == NULL) return QCO_INVALID_ARGUMENT;
  const size_t blocks_per_row = (size_t)(k / 32);
  const size_t bytes = (size_t)block_bytes_of(format);
  if ((size_t)n > SIZE_MAX / blocks_per_row) return QCO_INVALID_SHAPE;
  const size_t blocks = (size_t)n * blocks_per_row;
  if (blocks > SIZE_MAX / bytes) return QCO_INVALID_SHAPE;
  *size = blocks * bytes;
  return QCO_OK;
}

/* q8_0 block pack: kernels/quantization/qgemv_ref.cpp:14-41.  amax by fmax,
 * d = amax/127 in f32, multiply by the f32 reciprocal, round half to even,
 * clamp +-127, store fp16(d).  Non-finite input stops with an error. */
static int pack_q8_0(const float* w, long long n, long long k, uint8_t* out) {
  const long long nb = k / 32;
  for (long long r = 0; r < n; ++r) {
    for (long long b = 0; b < nb; ++b) {
      const float* src = w + r * k + b * 32;
      uint8_t* blk = out + (r * nb + b) * 34;
      float amax = 0.0f;
      for (int j = 0; j < 32; ++j) {
        if (!isfinite(src[j])) return 0;
        amax = fmaxf(amax, fabsf(src[j]));
      }
      const float d = amax / 127.0f;
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
      const uint16_t dh = qco_fp32_to_fp16(d);
      memcpy(blk, &dh, 2);
      for (int j = 0; j < 32; ++j) {
        float q = nearbyintf(src[j] * id);
        if (q < -127.0f) q = -127.0f;
        if (q > 127.0f) q = 127.0f;
        blk[2 + j] = (uint8_t)(int8_t)q;
      }
    }
  }
  return 1;
}

/* q4_0 block pack: kernels/quantization/qgemv_w8a8_ref.cpp:45-77.  vmax is the
 * first element of strictly largest magnitude (signed), d = vmax / -8,
 * q = clamp(lround(w*id) + 8, 0, 15) (half away from zero); byte j holds
 * element j in the low nibble and element j+16 in the high nibble. */
static int pack_q4_0(const float* w, long long n, long long k, uint8_t* out) {
  const long long nb = k / 32;
  for (long long r = 0; r < n; ++r) {
    for (long long b = 0; b < nb; ++b) {
      const float* src = w + r * k + b * 32;
      uint8_t* blk = out + (r * nb + b) * 18;
      float amax = 0.0f, vmax = 0.0f;
      for (int j = 0; j < 32; ++j) {
        if (!isfinite(src[j])) return 0;
        if (fabsf(src[j]) > amax) {
          amax = fabsf(src[j]);
          vmax = src[j];
        }
      }
      const float d = vmax / -8.0f;
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
      const uint16_t dh = qco_fp32_to_fp16(d);
      memcpy(blk, &dh, 2);
      for (int j = 0; j < 16; ++j) {
        long lo = lroundf(src[j] * id) + 8;
        long hi = lroundf(src[j + 16] * id) + 8;
        lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
        hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
        blk[2 + j] = (uint8_t)(lo | (hi << 4));
      }
    }
  }
  return 1;
}

/* qgemv_pack_weighted for q8_0/q4_0: src/dispatch/qgemv.cpp:215-275. */
int qco_pack(int format, const float* w, long long n, long long k, void* packed) {
  const int status = validate_shape(format, n, k);
  if (status != QCO_OK) return status;
  size_t ignored = 0;
  if (qco_packed_size(format, n, k, &ignored) != QCO_OK) return QCO_INVALID_SHAPE;
  if (w == NULL || packed == NULL) return QCO_INVALID_ARGUMENT;
  const int ok = format == QCO_Q8_0 ? pack_q8_0(w, n, k, (uint8_t*)packed)
                                    : pack_q4_0(w, n, k, (uint8_t*)packed);
  return ok ? QCO_OK : QCO_INVALID_ARGUMENT;
}

static float block_scale(const uint8_t* blk) {
  uint16_t dh;
  memcpy(&dh, blk, 2);
  return qco_fp16_to_fp32(dh);
}

/* Dequantize element j of a block.  q8_0: d * q (qgemv_ref.cpp:43-56);
 * q4_0: (nibble - 8) * d (qgemv_w8a8_ref.cpp:79-93).  Both products are exact
 * in f32 (<= 11 + 8 significant bits). */
static float dequant_elem(int format, const uint8_t* blk, int j) {
  const float d = block_scale(blk);
  if (format == QCO_Q8_0) return d * (float)(int8_t)blk[2 + j];
  const int nib = j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4);
  return (float)(nib - 8) * d;
}

/* qgemv_unpack: src/dispatch/qgemv.cpp:277-297. */
int qco_unpack(int format, const void* packed, long long n, long long k, float* w) {
  const int status = validate_shape(format, n, k);
  if (status != QCO_OK) return status;
  if (packed == NULL || w == NULL) return QCO_INVALID_ARGUMENT;
  const int bb = block_bytes_of(format);
  const long long nb = k / 32;
  const uint8_t* p = (const uint8_t*)packed;
  for (long long r = 0; r < n; ++r)
    for (long long b = 0; b < nb; ++b)
      for (int j = 0; j < 32; ++j)
        w[r * k + b * 32 + j] = dequant_elem(format, p + (r * nb + b) * bb, j);
  return QCO_OK;
}

/* ---------------------------------------------------------------- GEMV --- */

/* q8_0 x86 route gemv_rows_ref: kernels/quantization/qgemv_ref.cpp:62-83.
 * Per row: acc = 0; per block sum = sum + float(q_j) * x_j (sequential);
 * acc = acc + d * sum. */
void qco_q8_0_gemv(const void* packed, const float* x, float* y, long long n, long long k) {
  const long long nb = k / 32;
  const uint8_t* p = (const uint8_t*)packed;
  for (long long r = 0; r < n; ++r) {
    float acc = 0.0f;
    for (long long b = 0; b < nb; ++b) {
      const uint8_t* blk = p + (r * nb + b) * 34;
      const float d = block_scale(blk);
      float sum = 0.0f;
      for (int j = 0; j < 32; ++j) sum += (float)(int8_t)blk[2 + j] * x[b * 32 + j];
      acc += d * sum;
    }
    y[r] = acc;
  }
}

/* Portable q4_0 row kernel: kernels/quantization/qgemv_w8a8_ref.cpp:95-118.
 * Low and high nibble products interleaved in one block sum. */
void qco_q4_0_gemv_ref(const void* packed, const float* x, float* y, long long n, long long k) {
  const long long nb = k / 32;
  const uint8_t* p = (const uint8_t*)packed;
  for (long long r = 0; r < n; ++r) {
    float sum = 0.0f;
    for (long long b = 0; b < nb; ++b) {
      const uint8_t* blk = p + (r * nb + b) * 18;
      const float* xb = x + b * 32;
      float block_sum = 0.0f;
      for (int e = 0; e < 16; ++e) {
        block_sum += (float)((blk[2 + e] & 15) - 8) * xb[e];
        block_sum += (float)((blk[2 + e] >> 4) - 8) * xb[e + 16];
      }
      sum += block_scale(blk) * block_sum;
    }
    y[r] = sum;
  }
}

/* One dot_i8x16_f32 of kernels/quantization/qgemv_gguf_avx2.cpp:19-36 in
 * scalar form: two 8-lane products, lane-wise sum, then the 256->128 fold and
 * two horizontal adds.  fuse_pair: the lane-wise sum is evaluated as
 * fma(v[i], x[i], v[8+i]*x[8+i]) -- GCC contracts the mul+add of the vector
 * intrinsics under -mfma, rounding the second product and fusing the first
 * (pinned bit-exactly against oracle/_ref). */
static float dot16_avx2order(const int* v, const float* xin, int fuse_pair) {
  float s[8];
  for (int i = 0; i < 8; ++i) {
    const float p1 = (float)v[8 + i] * xin[8 + i];
    s[i] = fuse_pair ? fmaf((float)v[i], xin[i], p1) : (float)v[i] * xin[i] + p1;
  }
  float t[4];
  for (int i = 0; i < 4; ++i) t[i] = s[i] + s[i + 4];
  return (t[0] + t[1]) + (t[2] + t[3]);
}

/* x86 AVX2 q4_0 route q4_rows: kernels/quantization/qgemv_gguf_avx2.cpp:295-320.
 * flags bit 0: total += d * dot as one FMA; bit 1: fused pair sum (above). */
void qco_q4_0_gemv_avx2order(const void* packed, const float* x, float* y, long long n,
                             long long k, int flags) {
  const long long nb = k / 32;
  const uint8_t* p = (const uint8_t*)packed;
  for (long long r = 0; r < n; ++r) {
    float total = 0.0f;
    for (long long b = 0; b < nb; ++b) {
      const uint8_t* blk = p + (r * nb + b) * 18;
      int lo[16], hi[16];
      for (int j = 0; j < 16; ++j) {
        lo[j] = (blk[2 + j] & 15) - 8;
        hi[j] = ((blk[2 + j] >> 4) & 15) - 8;
      }
      const float dot = dot16_avx2order(lo, x + b * 32, flags & 2) +
                        dot16_avx2order(hi, x + b * 32 + 16, flags & 2);
      const float d = block_scale(blk);
      total = (flags & 1) ? fmaf(d, dot, total) : total + d * dot;
    }
    y[r] = total;
  }
}

/* Fused decode seam qgemv_qkv_rope_kv: kernels/quantization/qgemv_fused_ref.cpp:
 * 342-443, with packed_row_dot (:151-160) on the x86 build: q8_0_row_dot (:131-149,
 * the order of qco_q8_0_gemv) and q4_0_row_dot (:57-83, the interleaved order of
 * qco_q4_0_gemv_ref).  Validation as :348-391.  Per head and d < half, with
 * first = row d and second = row d + half: out[d] = first * c - second * s,
 * out[d + half] = second * c + first * s, c / s from row `position` of the
 * [max_position][half] tables; V rows are stored as projected. */
static int product_ok(const long long* dims, int count) {
  long long product = 1;
  for (int i = 0; i < count; ++i) {
    if (dims[i] <= 0 || product > LLONG_MAX / dims[i]) return 0;
    product *= dims[i];
  }
  return 1;
}

static float row_dot(int format, const uint8_t* row, const float* x, long long k) {
  float y = 0.0f;
  if (format == QCO_Q8_0)
    qco_q8_0_gemv(row, x, &y, 1, k);
  else
    qco_q4_0_gemv_ref(row, x, &y, 1, k);
  return y;
}

int qco_qgemv_qkv_rope_kv(int format, const void* packed_q, const void* packed_k,
                          const void* packed_v, const float* x, const float* cosine,
                          const float* sine, float* q, float* key_cache, float* value_cache,
                          long long query_heads, long long kv_heads, long long head_dim,
                          long long input_dim, long long slots, long long max_position,
                          int position, int slot) {
  const long long qdims[3] = {query_heads, head_dim, input_dim};
  const long long kdims[3] = {slots, kv_heads, head_dim};
  if (!product_ok(qdims, 3) || !product_ok(kdims, 3) || head_dim % 2 != 0 || position < 0 ||
      position >= max_position || slot < -1 || slot >= slots)
    return QCO_INVALID_SHAPE;
  if (!packed_q || !packed_k || !packed_v || !x || !cosine || !sine || !q || !key_cache ||
      !value_cache)
    return QCO_INVALID_ARGUMENT;
  const long long query_dim = query_heads * head_dim, kv_dim = kv_heads * head_dim;
  size_t bytes = 0;
  int st = qco_packed_size(format, query_dim, input_dim, &bytes);
  if (st != QCO_OK) return st;
  if (qco_packed_size(format, kv_dim, input_dim, &bytes) != QCO_OK) return QCO_INVALID_SHAPE;
  const long long row_bytes = (input_dim / 32) * block_bytes_of(format);
  const long long half = head_dim / 2;
  const float* c = cosine + (long long)position * half;
  const float* sn = sine + (long long)position * half;
  const uint8_t* wq = (const uint8_t*)packed_q;
  const uint8_t* wk = (const uint8_t*)packed_k;
  const uint8_t* wv = (const uint8_t*)packed_v;
  for (long long h = 0; h < query_heads; ++h)
    for (long long d = 0; d < half; ++d) {
      const long long r0 = h * head_dim + d, r1 = r0 + half;
      const float first = row_dot(format, wq + r0 * row_bytes, x, input_dim);
      const float second = row_dot(format, wq + r1 * row_bytes, x, input_dim);
      q[r0] = first * c[d] - second * sn[d];
      q[r1] = second * c[d] + first * sn[d];
    }
  if (slot < 0) return QCO_OK;
  float* kc = key_cache + (long long)slot * kv_dim;
  float* vc = value_cache + (long long)slot * kv_dim;
  for (long long h = 0; h < kv_heads; ++h)
    for (long long d = 0; d < half; ++d) {
      const long long r0 = h * head_dim + d, r1 = r0 + half;
      const float first = row_dot(format, wk + r0 * row_bytes, x, input_dim);
      const float second = row_dot(format, wk + r1 * row_bytes, x, input_dim);
      kc[r0] = first * c[d] - second * sn[d];
      kc[r1] = second * c[d] + first * sn[d];
    }
  for (long long r = 0; r < kv_dim; ++r) vc[r] = row_dot(format, wv + r * row_bytes, x, input_dim);
  return QCO_OK;
}

/* f64 contract oracle ("THE qgemv contract oracle"):
 * tests/correctness/test_qgemv.cpp:278-303 -- double accumulation over the
 * exactly dequantized weights.  Also returns ||w_hat_row||_2 for the
 * normalised tolerance |y - y64| <= tol * ||x||_2 * ||w_hat_row||_2. */
int qco_qgemv_f64(int format, const void* packed, const float* x, double* y64,
                  double* wnorm, long long n, long long k) {
  const int status = validate_shape(format, n, k);
  if (status != QCO_OK) return status;
  const int bb = block_bytes_of(format);
  const long long nb = k / 32;
  const uint8_t* p = (const uint8_t*)packed;
  for (long long r = 0; r < n; ++r) {
    double acc = 0.0, sq = 0.0;
    for (long long b = 0; b < nb; ++b) {
      const uint8_t* blk = p + (r * nb + b) * bb;
      for (int j = 0; j < 32; ++j) {
        const double w = (double)dequant_elem(format, blk, j);
        acc += w * (double)x[b * 32 + j];
        sq += w * w;
      }
    }
    y64[r] = acc;
    if (wnorm) wnorm[r] = sqrt(sq);
  }
  return QCO_OK;
}

/* ------------------------------------------------------ quantize_int8 --- */

/* kernels/quantization/quantization_ref.cpp:17-21 (quant_shape), 66-68
 * (rounded_int = nearbyint), 143-168 (quantize_int8).  Whole-input finite
 * check before any write; per group: max = max(max, |x|), scale = max/127,
 * inv = scale > 0 ? 1/scale : 0, code = clamp(nearbyint(x*inv), -127, 127). */
int qco_quantize_int8(const float* x, int8_t* codes, float* scales, long long rows,
                      long long dim, long long group_size) {
  if (rows <= 0 || dim <= 0 || rows > LLONG_MAX / dim) return QCO_INVALID_SHAPE;
  if (group_size == 0) group_size = dim;
  if (group_size <= 0 || dim % group_size != 0) return QCO_INVALID_SHAPE;
  if (x == NULL || codes == NULL || scales == NULL) return QCO_INVALID_ARGUMENT;
  for (long long i = 0; i < rows * dim; ++i)
    if (!isfinite(x[i])) return QCO_INVALID_ARGUMENT;
  const long long groups = dim / group_size;
  for (long long r = 0; r < rows; ++r) {
    for (long long g = 0; g < groups; ++g) {
      const long long base = r * dim + g * group_size;
      float maximum = 0.0f;
      for (long long i = 0; i < group_size; ++i) {
        const float a = fabsf(x[base + i]);
        if (maximum < a) maximum = a;
      }
      const float scale = maximum / 127.0f;
      scales[r * groups + g] = scale;
      const float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
      for (long long i = 0; i < group_size; ++i) {
        int q = (int)nearbyintf(x[base + i] * inverse);
        q = q < -127 ? -127 : (q > 127 ? 127 : q);
        codes[base + i] = (int8_t)q;
      }
    }
  }
  return QCO_OK;
}

/* ------------------------------------------------------- qgemv_w8a8 --- */

/* Per-32-block int8 activations: kernels/quantization/qgemv_w8a8_ref.cpp:18-41
 * (max = fmax(max, |x|), scale = max / 127, inverse = scale != 0 ? 1/scale
 * : 0, code = clamp(nearbyint(x * inverse), -127, 127)); x is finite here. */
static void quantize_blocks32(const float* x, long long k, int8_t* qx, float* dx) {
  for (long long b = 0; b < k / 32; ++b) {
    const float* in = x + b * 32;
    float maximum = 0.0f;
    for (int e = 0; e < 32; ++e) maximum = fmaxf(maximum, fabsf(in[e]));
    const float scale = maximum / 127.0f;
    const float inverse = scale != 0.0f ? 1.0f / scale : 0.0f;
    dx[b] = scale;
    for (int e = 0; e < 32; ++e) {
      const float v = nearbyintf(in[e] * inverse);
      qx[b * 32 + e] = (int8_t)(v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v));
    }
  }
}

/* qgemv_w8a8: validation src/dispatch/qgemv_w8a8.cpp:99-105,130-143 (format,
 * then shape, then nulls, then a non-finite x); rows
 * kernels/quantization/qgemv_w8a8_ref.cpp:120-145 (q4_0: integer dot of
 * (nibble - 8) with the codes, low nibbles against elements 0..15 and high
 * against 16..31) and 147-177 (q8_0).  Per row, in block order:
 * sum = sum + (float(dot) * d_w) * d_x. */
int qco_qgemv_w8a8(int format, const void* packed, const float* x, float* y, long long n,
                   long long k) {
  const int status = validate_shape(format, n, k);
  if (status != QCO_OK) return status;
  if (packed == NULL || x == NULL || y == NULL) return QCO_INVALID_ARGUMENT;
  for (long long e = 0; e < k; ++e)
    if (!isfinite(x[e])) return QCO_INVALID_ARGUMENT;
  const long long nb = k / 32;
  int8_t* qx = (int8_t*)malloc((size_t)k);
  float* dx = (float*)malloc((size_t)nb * sizeof(float));
  if (qx == NULL || dx == NULL) {
    free(qx);
    free(dx);
    return QCO_OUT_OF_MEMORY;
  }
  quantize_blocks32(x, k, qx, dx);
  const uint8_t* p = (const uint8_t*)packed;
  const int bb = block_bytes_of(format);
  for (long long r = 0; r < n; ++r) {
    float sum = 0.0f;
    for (long long b = 0; b < nb; ++b) {
      const uint8_t* blk = p + (r * nb + b) * bb;
      const int8_t* in = qx + b * 32;
      int dot = 0;
      if (format == QCO_Q4_0) {
        for (int j = 0; j < 16; ++j) {
          dot += ((blk[2 + j] & 0x0F) - 8) * in[j];
          dot += ((blk[2 + j] >> 4) - 8) * in[j + 16];
        }
      } else {
        for (int e = 0; e < 32; ++e) dot += (int)(int8_t)blk[2 + e] * in[e];
      }
      sum += (float)dot * block_scale(blk) * dx[b];
    }
    y[r] = sum;
  }
  free(qx);
  free(dx);
  return QCO_OK;
}

/* ---------------------------------------------------------- int8 GEMM --- */

/* Public validation src/dispatch/int8_gemm.cpp:67-94 and the exact int64
 * kernel kernels/quantization/int8_gemm_ref.cpp:9-32:
 * y[m,n] = (float(dot) * ws[n]) * as[m], dot -= zp[m]*row_sum[n] if asymmetric. */
int qco_int8_gemm(const int8_t* w, const int8_t* x, const float* ws, const float* as,
                  const int32_t* row_sum, const int* zp, float* y, long long m,
                  long long n, long long k, int asymmetric) {
  if (m <= 0 || n <= 0 || k <= 0 || m > LLONG_MAX / n || m * n > LLONG_MAX / k)
    return QCO_INVALID_SHAPE;
  if (!w || !x || !ws || !as || !y || (asymmetric && (!row_sum || !zp)))
    return QCO_INVALID_ARGUMENT;
  for (long long i = 0; i < n; ++i)
    if (!isfinite(ws[i])) return QCO_INVALID_ARGUMENT;
  for (long long i = 0; i < m; ++i)
    if (!isfinite(as[i])) return QCO_INVALID_ARGUMENT;
  for (long long r = 0; r < m; ++r) {
    for (long long c = 0; c < n; ++c) {
      int64_t dot = 0;
      for (long long i = 0; i < k; ++i) dot += (int)w[c * k + i] * (int)x[r * k + i];
      if (asymmetric) dot -= (int64_t)zp[r] * row_sum[c];
      y[r * n + c] = (float)dot * ws[c] * as[r];
    }
  }
  return QCO_OK;
}

void qco_int8_gemm_entries(const int8_t* w, const int8_t* x, const float* ws,
                           const float* as, const long long* rows, const long long* cols,
                           long long count, long long k, int64_t* acc64, float* y) {
  for (long long e = 0; e < count; ++e) {
    const long long r = rows[e], c = cols[e];
    int64_t dot = 0;
    for (long long i = 0; i < k; ++i) dot += (int)w[c * k + i] * (int)x[r * k + i];
    acc64[e] = dot;
    y[e] = (float)dot * ws[c] * as[r];
  }
}

/* ------------------------------------------- rms_norm_add_quant_int8 --- */

/* kernels/norms/norm_quant_ref.cpp:106-114 (valid_dynamic_shape: rows x
 * hidden product, finite eps >= 0, group 0 -> hidden, hidden % group == 0),
 * 117-130 (shape, then nulls), 33-92 (add_and_measure, RMS branch; the
 * x86-64 build runs the plain loop at 82-89: value = x + residual stored to
 * residual_out, sumsq += double(value) * value in element order, inverse =
 * float(1 / sqrt(sumsq / hidden + eps)) in double), 94-104 (normalized_at:
 * (residual_out * inverse) * weight in f32), 150-168 and 224-290 (per group:
 * maximum = max(maximum, |value|), a non-finite value marks the group
 * invalid and skips it; scale = maximum / 127, inverse = scale > 0 ? 1 /
 * scale : 0, code = clamp(nearbyint(value * inverse), -127, 127)).  Every
 * row is processed; an invalid group leaves its scale and codes unwritten
 * and the call returns kInvalidArgument at the end. */
int qco_rms_norm_add_quant_int8(const float* x, const float* residual, const float* weight,
                                int8_t* codes, float* residual_out, float* scales,
                                long long rows, long long hidden, float eps,
                                long long group_size) {
  if (rows <= 0 || hidden <= 0 || rows > LLONG_MAX / hidden || !isfinite(eps) || eps < 0.0f)
    return QCO_INVALID_SHAPE;
  if (group_size == 0) group_size = hidden;
  if (group_size <= 0 || hidden % group_size != 0) return QCO_INVALID_SHAPE;
  if (!x || !residual || !weight || !codes || !residual_out || !scales)
    return QCO_INVALID_ARGUMENT;
  float* values = (float*)malloc((size_t)group_size * sizeof(float));
  if (values == NULL) return QCO_OUT_OF_MEMORY;
  const long long groups = hidden / group_size;
  int invalid = 0;
  for (long long r = 0; r < rows; ++r) {
    const long long base = r * hidden;
    double sumsq = 0.0;
    for (long long i = 0; i < hidden; ++i) {
      const float value = x[base + i] + residual[base + i];
      residual_out[base + i] = value;
      sumsq += (double)value * value;
    }
    const float inverse = (float)(1.0 / sqrt(sumsq / (double)hidden + (double)eps));
    for (long long g = 0; g < groups; ++g) {
      float maximum = 0.0f;
      int bad = 0;
      for (long long i = 0; i < group_size; ++i) {
        const long long col = g * group_size + i;
        const float value = (residual_out[base + col] * inverse) * weight[col];
        values[i] = value;
        if (!isfinite(value)) bad = 1;
        const float a = fabsf(value);
        if (maximum < a) maximum = a;
      }
      if (bad) {
        invalid = 1;
        continue;
      }
      const float scale = maximum / 127.0f;
      scales[r * groups + g] = scale;
      const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
      for (long long i = 0; i < group_size; ++i) {
        int q = (int)nearbyintf(values[i] * inv);
        q = q < -127 ? -127 : (q > 127 ? 127 : q);
        codes[base + g * group_size + i] = (int8_t)q;
      }
    }
  }
  free(values);
  return invalid ? QCO_INVALID_ARGUMENT : QCO_OK;
}

/* ------------------------------------------ quantize_int8_asymmetric --- */

/* static_cast<int>(double) as the reference's x86-64 build executes it
 * (cvttsd2si / cvttpd2dq): truncation toward zero, and INT_MIN for NaN or a
 * value outside the int range.  int + int and int - int wrap. */
static int x86_double_to_int(double d) {
  if (!(d > -2147483649.0 && d < 2147483648.0)) return INT_MIN;
  return (int)d;
}
static int wrap_add(int a, int b) { return (int)((uint32_t)a + (uint32_t)b); }
static int wrap_sub(int a, int b) { return (int)((uint32_t)a - (uint32_t)b); }

/* kernels/quantization/quantization_ref.cpp:190-226.  Whole-input finite
 * check first; per row, in double: range = max - min, scale_value = range > 0
 * ? range / 255 : max(|min| / 127, 1e-7), scale = float(scale_value), zero =
 * int(nearbyint(-128 - min / scale_value)), code = clamp(int(nearbyint(x /
 * scale_value)) + zero, -128, 127). */
int qco_quantize_int8_asymmetric(const float* x, int8_t* codes, float* scales,
                                 int* zero_points, long long rows, long long dim) {
  if (rows <= 0 || dim <= 0 || rows > LLONG_MAX / dim) return QCO_INVALID_SHAPE;
  if (!x || !codes || !scales || !zero_points) return QCO_INVALID_ARGUMENT;
  for (long long i = 0; i < rows * dim; ++i)
    if (!isfinite(x[i])) return QCO_INVALID_ARGUMENT;
  for (long long r = 0; r < rows; ++r) {
    const float* in = x + r * dim;
    float lo = in[0], hi = in[0];
    for (long long i = 1; i < dim; ++i) {
      if (in[i] < lo) lo = in[i];
      if (hi < in[i]) hi = in[i];
    }
    const double minimum = (double)lo, maximum = (double)hi;
    const double range = maximum - minimum;
    double scale_value;
    if (range > 0.0) {
      scale_value = range / 255.0;
    } else {
      const double a = fabs(minimum) / 127.0;
      scale_value = a < 1e-7 ? 1e-7 : a;
    }
    const int zero = x86_double_to_int(nearbyint(-128.0 - minimum / scale_value));
    scales[r] = (float)scale_value;
    zero_points[r] = zero;
    for (long long i = 0; i < dim; ++i) {
      int q = wrap_add(x86_double_to_int(nearbyint((double)in[i] / scale_value)), zero);
      q = q < -128 ? -128 : (q > 127 ? 127 : q);
      codes[r * dim + i] = (int8_t)q;
    }
  }
  return QCO_OK;
}

/* kernels/quantization/quantization_ref.cpp:228-244: out = scale[row] *
 * float(int(code) - zero_point[row]). */
int qco_dequantize_int8_asymmetric(const int8_t* codes, const float* scales,
                                   const int* zero_points, float* out, long long rows,
                                   long long dim) {
  if (rows <= 0 || dim <= 0 || rows > LLONG_MAX / dim) return QCO_INVALID_SHAPE;
  if (!codes || !scales || !zero_points || !out) return QCO_INVALID_ARGUMENT;
  for (long long r = 0; r < rows; ++r)
    for (long long i = 0; i < dim; ++i)
      out[r * dim + i] = scales[r] * (float)wrap_sub((int)codes[r * dim + i], zero_points[r]);
  return QCO_OK;
}
