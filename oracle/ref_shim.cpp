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
//   qgemv_qkv_rope_kv -> the public function (kernels/quantization/qgemv_fused_ref.cpp:342-443)
//   qgemm_prepacked_*_storage -> the public functions (kernels/quantization/qgemm_canonical.cpp),
//               run over tests/cpp/storage_scenarios.h
//   quantize_canonical / dequantize_canonical -> the public functions
//               (kernels/quantization/quant_import_ref.cpp), run over
//               tests/cpp/canonical_quant_scenarios.h
//   CpuPackedWeights::prepare (both overloads), info(), panel_data()
//               -> src/memory/packed_weights.cpp:197-412
#include <cstddef>
#include <cstdint>

#include "kernels/quantization/gguf_ref.h"
#include "kernels/quantization/qgemv.h"
#include "kernels/quantization/qgemv_w8a8.h"
#include <cstring>

#include "quixicore_cpu/packed_weights.h"
#include "quixicore_cpu/qgemm.h"
#include "quixicore_cpu/quant_import.h"
#include "quixicore_cpu/quantization.h"
#include "quixicore_cpu/threading.h"
#include "../tests/cpp/storage_scenarios.h"
#include "../tests/cpp/canonical_quant_scenarios.h"

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

// info fields of a prepared weight as 24 integers (the order the tests read).
static void dump_info(const qc::CpuPackedWeightsInfo& i, long long* out) {
  const long long v[] = {static_cast<long long>(i.layout), i.rows, i.columns, i.row_tile,
                         i.block_size, i.blocks_per_row, static_cast<long long>(i.block_bytes),
                         static_cast<long long>(i.contract_bytes),
                         static_cast<long long>(i.panel_bytes), i.prepared_version,
                         static_cast<long long>(i.required_isa), i.column_tile,
                         static_cast<long long>(i.panel_alignment),
                         static_cast<long long>(i.prepared_bytes),
                         static_cast<long long>(i.logical_bytes), i.has_canonical_layout,
                         static_cast<long long>(i.canonical_layout),
                         static_cast<long long>(i.scale_table_offset),
                         static_cast<long long>(i.zero_point_table_offset),
                         static_cast<long long>(i.activation_scale_offset),
                         static_cast<long long>(i.activation_zero_point_offset),
                         static_cast<long long>(i.row_sum_table_offset),
                         static_cast<long long>(i.format),
                         static_cast<long long>(i.memory_amplification * 1e6)};
  std::memcpy(out, v, sizeof(v));
}

// Status of prepare; on kOk the panel (prepared_bytes, at most cap) and info.
int qcref_prepare_gguf(int format, const void* bytes, long long rows, long long columns,
                       int layout, void* panel, long long cap, long long* info) {
  qc::CpuPackedWeights w;
  const qc::Status s = w.prepare(static_cast<qc::QuantFormat>(format), bytes, rows, columns,
                                 static_cast<qc::CpuPanelLayout>(layout));
  if (s != qc::Status::kOk) return static_cast<int>(s);
  const qc::CpuPackedWeightsInfo i = w.info();
  dump_info(i, info);
  const long long n = static_cast<long long>(i.prepared_bytes);
  std::memcpy(panel, w.panel_data(), static_cast<size_t>(n < cap ? n : cap));
  return 0;
}

// A kInt8Symmetric / kInt8Affine tensor with row, channel or group scales,
// optional zero points, activation scales / zero points and row sums.
int qcref_prepare_canonical_int8(int affine, long long rows, long long columns,
                                 long long group_size, int scale_mode, const int8_t* data,
                                 const float* scales, long long nscales, const float* zps,
                                 const float* act_scales, long long nact, const int* act_zps,
                                 const int32_t* row_sums, int layout, void* panel,
                                 long long cap, long long* info) {
  qc::CanonicalQuantTensor t;
  t.metadata.layout = affine ? qc::CanonicalQuantLayout::kInt8Affine
                             : qc::CanonicalQuantLayout::kInt8Symmetric;
  t.metadata.logical_rows = rows;
  t.metadata.logical_columns = columns;
  t.metadata.group_size = group_size;
  t.metadata.scale_mode = static_cast<qc::QuantScaleMode>(scale_mode);
  t.metadata.scale_encoding = qc::QuantScaleEncoding::kFP32;
  t.metadata.scale_count = static_cast<size_t>(nscales);
  const auto* d = reinterpret_cast<const uint8_t*>(data);
  t.data.assign(d, d + rows * columns);
  t.scales.assign(scales, scales + nscales);
  if (affine) {
    t.metadata.zero_point_mode = qc::QuantZeroPointMode::kInteger;
    t.metadata.zero_point_count = static_cast<size_t>(nscales);
    t.zero_points.assign(zps, zps + nscales);
  }
  if (nact > 0) t.activation_scales.assign(act_scales, act_scales + nact);
  if (nact > 0 && act_zps != nullptr) t.activation_zero_points.assign(act_zps, act_zps + nact);
  if (row_sums != nullptr) t.row_sums.assign(row_sums, row_sums + rows);
  qc::CpuPackedWeights w;
  const qc::Status s = w.prepare(t, static_cast<qc::CpuPanelLayout>(layout));
  if (s != qc::Status::kOk) return static_cast<int>(s);
  const qc::CpuPackedWeightsInfo i = w.info();
  dump_info(i, info);
  const long long n = static_cast<long long>(i.prepared_bytes);
  std::memcpy(panel, w.panel_data(), static_cast<size_t>(n < cap ? n : cap));
  return 0;
}

// import_smoothquant_w8a8 (row sums computed by the importer), then prepare.
int qcref_prepare_smoothquant(const int8_t* w, const float* ws, long long rows, long long columns,
                              const float* act_scales, long long nact, const int* act_zps,
                              int layout, void* panel, long long cap, long long* info) {
  qc::SmoothQuantW8A8Source src;
  src.weights = w;
  src.weight_count = static_cast<size_t>(rows * columns);
  src.weight_scales = ws;
  src.weight_scale_count = static_cast<size_t>(rows);
  src.activation_scales = act_scales;
  src.activation_scale_count = static_cast<size_t>(nact);
  src.activation_zero_points = act_zps;
  src.activation_zero_point_count = act_zps != nullptr ? static_cast<size_t>(nact) : 0;
  src.rows = rows;
  src.columns = columns;
  qc::CanonicalQuantTensor t;
  qc::Status s = qc::import_smoothquant_w8a8(src, &t);
  if (s != qc::Status::kOk) return 100 + static_cast<int>(s);
  qc::CpuPackedWeights pw;
  s = pw.prepare(t, static_cast<qc::CpuPanelLayout>(layout));
  if (s != qc::Status::kOk) return static_cast<int>(s);
  const qc::CpuPackedWeightsInfo i = pw.info();
  dump_info(i, info);
  const long long n = static_cast<long long>(i.prepared_bytes);
  std::memcpy(panel, pw.panel_data(), static_cast<size_t>(n < cap ? n : cap));
  return 0;
}

int qcref_qgemv_qkv_rope_kv(int format, const void* packed_q, const void* packed_k,
                            const void* packed_v, const float* x, const float* cosine,
                            const float* sine, float* q, float* key_cache, float* value_cache,
                            long long query_heads, long long kv_heads, long long head_dim,
                            long long input_dim, long long slots, long long max_position,
                            int position, int slot) {
  return static_cast<int>(qc::qgemv_qkv_rope_kv(
      static_cast<qc::QuantFormat>(format), packed_q, packed_k, packed_v, x, cosine, sine, q,
      key_cache, value_cache, query_heads, kv_heads, head_dim, input_dim, slots, max_position,
      position, slot));
}

// The prepared storage projection scenarios (tests/cpp/storage_scenarios.h)
// through the reference's own CpuPackedWeights and qgemm_prepacked_*_storage.
int qcref_storage_scenarios(const char* dir) {
  storage_scenarios::Sink sink(dir);
  if (sink.manifest == nullptr) return 1;
  storage_scenarios::run(sink);
  return 0;
}

// The quantize_canonical / dequantize_canonical scenarios
// (tests/cpp/canonical_quant_scenarios.h) through the reference's functions
// (kernels/quantization/quant_import_ref.cpp:552-681,717-838).
int qcref_canonical_quant_scenarios(const char* dir) {
  storage_scenarios::Sink sink(dir);
  if (sink.manifest == nullptr) return 2;
  canonical_quant_scenarios::run(sink);
  return 0;
}

void qcref_set_num_threads(int n) { qc::set_num_threads(n); }
int qcref_num_threads() { return qc::num_threads(); }

}  // extern "C"
