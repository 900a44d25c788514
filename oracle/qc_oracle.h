/*
 * CPU oracle for the quantized-matmul hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference algorithms (QuixiAI/QuixiCore-CPU),
 * used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
 * the checker.  The product library (libquixicore_hip.so) never links, loads
 * or calls anything in this directory.
 *
 * Every function cites the reference file:line it follows.  Built with
 * -ffp-contract=off so every f32 operation rounds exactly where the C source
 * says it does (the reference's baseline x86-64 translation units have no FMA
 * instructions available, so they round the same way).
 *
 * Pinning of each function (how a plausible mistake would be caught) is
 * listed in tests/test_oracle.py; functions with no independent check would
 * be marked "parity unpinned" here -- currently there are none.
 */
#ifndef QC_ORACLE_H
#define QC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status integers in the reference order (include/quixicore_cpu/status.h:5-11). */
enum {
  QCO_OK = 0,
  QCO_INVALID_SHAPE = 1,
  QCO_UNSUPPORTED_FORMAT = 2,
  QCO_INVALID_ARGUMENT = 3,
  QCO_OUT_OF_MEMORY = 4
};

/* QuantFormat values used on this path (include/quixicore_cpu/qgemv.h:10-13). */
enum { QCO_Q8_0 = 0, QCO_Q4_0 = 1 };

float qco_fp16_to_fp32(uint16_t h);
uint16_t qco_fp32_to_fp16(float f);

int qco_packed_size(int format, long long n, long long k, size_t* size);
int qco_pack(int format, const float* w, long long n, long long k, void* packed);
int qco_unpack(int format, const void* packed, long long n, long long k, float* w);

/* f32 GEMV in the summation order of the reference's x86 routes. */
void qco_q8_0_gemv(const void* packed, const float* x, float* y, long long n, long long k);
void qco_q4_0_gemv_ref(const void* packed, const float* x, float* y, long long n, long long k);
void qco_q4_0_gemv_avx2order(const void* packed, const float* x, float* y, long long n,
                             long long k, int fused_scale_add);

/* One decode token's Q/K/V projections (the reference's x86 row orders) with
 * split-half RoPE on Q and K and K/V stored into cache slot `slot`. */
int qco_qgemv_qkv_rope_kv(int format, const void* packed_q, const void* packed_k,
                          const void* packed_v, const float* x, const float* cosine,
                          const float* sine, float* q, float* key_cache, float* value_cache,
                          long long query_heads, long long kv_heads, long long head_dim,
                          long long input_dim, long long slots, long long max_position,
                          int position, int slot);

/* f64 contract oracle: y64 = dequant(W) . x in double, plus ||w_hat_row||_2. */
int qco_qgemv_f64(int format, const void* packed, const float* x, double* y64,
                  double* wnorm, long long n, long long k);

int qco_quantize_int8(const float* x, int8_t* codes, float* scales, long long rows,
                      long long dim, long long group_size);

/* Activation-quantizing GEMV: x quantized per 32-element block to int8, integer
 * block dots, y[r] = sum_b (float(dot) * d_w) * d_x in block order. */
int qco_qgemv_w8a8(int format, const void* packed, const float* x, float* y, long long n,
                   long long k);

int qco_int8_gemm(const int8_t* w, const int8_t* x, const float* ws, const float* as,
                  const int32_t* row_sum, const int* zp, float* y, long long m,
                  long long n, long long k, int asymmetric);
/* Selected entries only: acc64[i] and y[i] for (rows[i], cols[i]). */
void qco_int8_gemm_entries(const int8_t* w, const int8_t* x, const float* ws,
                           const float* as, const long long* rows, const long long* cols,
                           long long count, long long k, int64_t* acc64, float* y);

/* Residual add + RMSNorm + dynamic int8 quantization (per row, or per group
 * of group_size columns); status 3 after all rows if a group's normalized
 * values are not finite (that group's scale and codes are left unwritten). */
int qco_rms_norm_add_quant_int8(const float* x, const float* residual, const float* weight,
                                int8_t* codes, float* residual_out, float* scales,
                                long long rows, long long hidden, float eps,
                                long long group_size);

/* Per-row asymmetric int8: codes in [-128, 127], value ~ scale * (code - zero). */
int qco_quantize_int8_asymmetric(const float* x, int8_t* codes, float* scales,
                                 int* zero_points, long long rows, long long dim);
int qco_dequantize_int8_asymmetric(const int8_t* codes, const float* scales,
                                   const int* zero_points, float* out, long long rows,
                                   long long dim);

#ifdef __cplusplus
}
#endif

#endif
