// extern "C" wrappers over the reference's own hot-path functions, compiled
// from the unmodified sources under /root/reference by oracle/Makefile (target
// `ref`) into oracle/_ref/libqcref.so.  TEST INFRASTRUCTURE ONLY: used by
// tests/ to pin the C oracle, and by bench.py's cpu_baseline leg.
//
// Each wrapper calls the function the reference's x86 dispatch selects:
//   q8_0 qgemv  -> quant::q8_0_gemv_ref     (src/dispatch/qgemv.cpp:73-79,350-351)
//   q4_0 qgemv  -> quant::gguf_gemv_avx2    (src/dispatch/qgemv.cpp:59-60,104-123,352-363)
//   qgemm       -> one qgemv per row        (kernels/quantization/qgemm_ref.cpp:156-162)
//   int8_gemm   -> the public dispatcher    (src/dispatch/int8_gemm.cpp:67-94)
//   quantize_int8 -> the public function    (kernels/quantization/quantization_ref.cpp:143-168)
//   qgemv_w8a8  -> quant::q{4,8}_0_gemv_w8a8_ref (src/dispatch/qgemv_w8a8.cpp:27-34,66-73)
//   rms_norm_add_quant_int8, quantize_int8_asymmetric, dequantize_int8_asymmetric
//               -> the public functions  (kernels/norms/norm_quant_ref.cpp:1060-1068;
//                                          kernels/quantization/quantization_ref.cpp:190-244)
#include <cstddef>
#include <cstdint>

#include "kernels/quantization/gguf_ref.h"
#include "kernels/quantization/qgemv.h"
#include "kernels/quantization/qgemv_w8a8.h"
#include "quixicore_cpu/qgemm.h"
#include "quixicore_cpu/quantization.h"
#include "quixicore_cpu/threading.h"

namespace qc = quixicore_cpu;

extern "C" {

int qcref_q8_0_pack(const float* w, long long n, long long k, void* out) {
  return qc::quant::q8_0_pack_ref(w, n, k, static_cast<qc::quant::BlockQ8_0*>(out)) ? 0 : 3;
}

int qcref_q4_0_pack(const float* w, long long n, long long k, void* out) {
  return qc::quant::q4_0_pack_ref(w, n, k, static_cast<qc::quant::BlockQ4_0*>(out)) ? 0 : 3;
}

void qcref_q8_0_gemv(const void* packed, const float* x, float* y, long long n, long long k) {
  qc::quant::q8_0_gemv_ref(static_cast<const qc::quant::BlockQ8_0*>(packed), x, y, n, k);
}

void qcref_q4_0_gemv_avx2(const void* packed, const float* x, float* y, long long n,
                          long long k) {
  qc::quant::gguf_gemv_avx2(qc::QuantFormat::kQ4_0, packed, x, y, n, k);
}

void qcref_q4_0_gemv_portable(const void* packed, const float* x, float* y, long long n,
                              long long k) {
  qc::quant::q4_0_gemv_ref(static_cast<const qc::quant::BlockQ4_0*>(packed), x, y, n, k);
}

// The x86 qgemm: M independent qgemv calls over the same packed weights.
void qcref_qgemm(int format, const void* packed, const float* x, float* y, long long m,
                 long long n, long long k) {
  for (long long row = 0; row < m; ++row) {
    if (format == 0) {
      qcref_q8_0_gemv(packed, x + row * k, y + row * n, n, k);
    } else {
      qcref_q4_0_gemv_avx2(packed, x + row * k, y + row * n, n, k);
    }
  }
}

int qcref_quantize_int8(const float* x, std::int8_t* codes, float* scales, long long rows,
                        long long dim, long long group_size) {
  return static_cast<int>(qc::quantize_int8(x, codes, scales, rows, dim, group_size));
}

int qcref_int8_gemm(const std::int8_t* w, const std::int8_t* x, const float* ws,
                    const float* as, const std::int32_t* row_sum, const int* zp, float* y,
                    long long m, long long n, long long k, int asymmetric) {
  return static_cast<int>(
      qc::int8_gemm(w, x, ws, as, row_sum, zp, y, m, n, k, asymmetric != 0));
}

// qgemv_w8a8 -> the x86 variant the dispatcher resolves, the portable ref
// (src/dispatch/qgemv_w8a8.cpp:27-34,66-73; the dotprod variants are aarch64).
void qcref_q4_0_gemv_w8a8(const void* packed, const float* x, float* y, long long n,
                          long long k) {
  qc::quant::q4_0_gemv_w8a8_ref(static_cast<const qc::quant::BlockQ4_0*>(packed), x, y, n, k);
}

void qcref_q8_0_gemv_w8a8(const void* packed, const float* x, float* y, long long n,
                          long long k) {
  qc::quant::q8_0_gemv_w8a8_ref(static_cast<const qc::quant::BlockQ8_0*>(packed), x, y, n, k);
}

const char* qcref_int8_gemm_variant() { return qc::int8_gemm_variant(); }

int qcref_rms_norm_add_quant_int8(const float* x, const float* residual, const float* weight,
                                  std::int8_t* codes, float* residual_out, float* scales,
                                  long long rows, long long hidden, float eps,
                                  long long group_size) {
  return static_cast<int>(qc::rms_norm_add_quant_int8(x, residual, weight, codes, residual_out,
                                                      scales, rows, hidden, eps, group_size));
}

int qcref_quantize_int8_asymmetric(const float* x, std::int8_t* codes, float* scales,
                                   int* zero_points, long long rows, long long dim) {
  return static_cast<int>(qc::quantize_int8_asymmetric(x, codes, scales, zero_points, rows, dim));
}

int qcref_dequantize_int8_asymmetric(const std::int8_t* codes, const float* scales,
                                     const int* zero_points, float* out, long long rows,
                                     long long dim) {
  return static_cast<int>(qc::dequantize_int8_asymmetric(codes, scales, zero_points, out, rows,
                                                        dim));
}

void qcref_set_num_threads(int n) { qc::set_num_threads(n); }
int qcref_num_threads() { return qc::num_threads(); }

}  // extern "C"
