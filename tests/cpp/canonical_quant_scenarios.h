// quantize_canonical / dequantize_canonical scenarios -- TEST INFRASTRUCTURE
// ONLY.  One list, compiled twice against the same C++ API
// (include/quixicore_cpu/quant_import.h:42-45,53-54): into oracle/_ref with
// the reference's own headers and library (oracle/ref_shim.cpp,
// qcref_canonical_quant_scenarios) and into tests/cpp/canonical_quant_check.cpp
// with this repository's drop-in and libquixicore_hip.so.  Both write every
// status and every int8 tensor table / decoded output under a directory;
// tests/test_gpu_canonical_quant.py compares the two runs byte for byte.
//
// Names starting with "other_" use layouts this GPU path does not compute:
// only their statuses are written (the reference's validation results must
// match; where the reference computes, this path returns kUnsupportedFormat).
// Names starting with "proj_" are qgemm_prepacked_quantized /
// qgemv_prepacked_quantized outputs (f32 sums, not bit-identical across the
// two libraries) and the decoded operands they are checked against.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "quixicore_cpu/float_storage.h"
#include "quixicore_cpu/packed_weights.h"
#include "quixicore_cpu/qgemm.h"
#include "quixicore_cpu/qgemv.h"
#include "quixicore_cpu/quant_import.h"
#include "storage_scenarios.h"

namespace canonical_quant_scenarios {

namespace qc = quixicore_cpu;
using storage_scenarios::Sink;
using L = qc::CanonicalQuantLayout;

// Rows of xorshift values in [-1, 1) scaled by 2^(r % 24 - 12); row 5 is all
// zeros and row 7 holds one outlier 1000 times its row's scale.
inline std::vector<float> matrix(uint32_t seed, long long rows, long long cols) {
  std::vector<float> v(static_cast<size_t>(rows * cols));
  uint32_t s = seed | 1u;
  for (long long r = 0; r < rows; ++r)
    for (long long c = 0; c < cols; ++c) {
      const float u = static_cast<float>(storage_scenarios::next(&s) >> 8) * (2.0f / 16777216.0f) - 1.0f;
      v[r * cols + c] = r == 5 ? 0.0f : std::ldexp(u, static_cast<int>(r % 24) - 12);
    }
  if (rows > 7) v[7 * cols + 3] = std::ldexp(1000.0f, 7 % 24 - 12);
  return v;
}

// Finite f16 bit patterns: sign, exponent field 3..26, random mantissa.
inline std::vector<uint16_t> f16_matrix(uint32_t seed, size_t n) {
  std::vector<uint16_t> v(n);
  uint32_t s = seed | 1u;
  for (auto& e : v) {
    const uint32_t z = storage_scenarios::next(&s);
    e = static_cast<uint16_t>((z & 0x8000u) | ((3u + (z >> 16) % 24u) << 10) | (z & 0x3ffu));
  }
  return v;
}

// bf16 values: the upper halves of f32 matrix values.
inline std::vector<uint16_t> bf16_matrix(const std::vector<float>& f) {
  std::vector<uint16_t> v(f.size());
  for (size_t i = 0; i < f.size(); ++i) v[i] = storage_scenarios::bf16_bits(f[i]);
  return v;
}

inline void put_tensor(Sink& sink, const std::string& name, const qc::CanonicalQuantTensor& t) {
  const qc::QuantTensorMetadata& md = t.metadata;
  const long long meta[] = {static_cast<long long>(md.layout), md.logical_rows,
                            md.logical_columns, md.group_size,
                            static_cast<long long>(md.scale_mode),
                            static_cast<long long>(md.scale_encoding),
                            static_cast<long long>(md.zero_point_mode),
                            static_cast<long long>(md.scale_count),
                            static_cast<long long>(md.zero_point_count),
                            static_cast<long long>(t.provenance),
                            static_cast<long long>(t.scale_codes.size()),
                            static_cast<long long>(t.row_sums.size())};
  sink.data(name + "_meta", meta, sizeof(meta), "i64");
  sink.data(name + "_codes", t.data.data(), t.data.size(), "i8");
  sink.data(name + "_scales", t.scales.data(), t.scales.size() * 4, "f32");
  sink.data(name + "_zeros", t.zero_points.data(), t.zero_points.size() * 4, "f32");
}

// quantize, record the tensor, decode it again and record that.
inline void round_trip(Sink& sink, const std::string& name, qc::FloatStorageInput in,
                       long long rows, long long cols, L layout, long long group) {
  qc::CanonicalQuantTensor t;
  sink.status(name, qc::quantize_canonical(in, rows, cols, layout, group, &t));
  put_tensor(sink, name, t);
  std::vector<float> out(static_cast<size_t>(rows * cols), 7.0f);
  sink.status(name + "_dequant", qc::dequantize_canonical(t, out.data(), rows * cols));
  sink.data(name + "_dequant", out.data(), out.size() * 4, "f32");
}

// qgemm_prepacked_quantized / qgemv_prepacked_quantized
// (qgemm_canonical.cpp:5415-5507): int8 weights (symmetric rows, symmetric
// groups of 128, affine rows) against int8 activations (symmetric rows,
// symmetric groups of 64, affine rows), every pair, plus the validation cases.
inline void projections(Sink& sink) {
  const long long n = 96, k = 512, m = 5;
  const std::vector<float> wf = matrix(0x77, n, k);
  const std::vector<float> af = matrix(0x99, m, k);
  struct Op {
    const char* name;
    L layout;
    long long group;
  };
  const Op wops[] = {{"wsym", L::kInt8Symmetric, 0}, {"wsymg", L::kInt8Symmetric, 128},
                     {"waff", L::kInt8Affine, 0}};
  const Op aops[] = {{"asym", L::kInt8Symmetric, 0}, {"asymg", L::kInt8Symmetric, 64},
                     {"aaff", L::kInt8Affine, 0}};
  qc::CpuPackedWeights prepared[3];
  qc::CanonicalQuantTensor acts[3];
  for (int i = 0; i < 3; ++i) {
    qc::CanonicalQuantTensor t;
    const std::string nm = std::string("proj_") + wops[i].name;
    sink.status(nm, qc::quantize_canonical({wf.data(), qc::FloatStorageType::kF32, n * k}, n, k,
                                           wops[i].layout, wops[i].group, &t));
    std::vector<float> dec(static_cast<size_t>(n * k));
    sink.status(nm + "_dequant", qc::dequantize_canonical(t, dec.data(), n * k));
    sink.data(nm + "_dequant", dec.data(), dec.size() * 4, "f32");
    sink.status(nm + "_prepare", prepared[i].prepare(t));
  }
  for (int j = 0; j < 3; ++j) {
    const std::string nm = std::string("proj_") + aops[j].name;
    sink.status(nm, qc::quantize_canonical({af.data(), qc::FloatStorageType::kF32, m * k}, m, k,
                                           aops[j].layout, aops[j].group, &acts[j]));
    std::vector<float> dec(static_cast<size_t>(m * k));
    sink.status(nm + "_dequant", qc::dequantize_canonical(acts[j], dec.data(), m * k));
    sink.data(nm + "_dequant", dec.data(), dec.size() * 4, "f32");
  }
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      const std::string nm = std::string("proj_") + wops[i].name + "_" + aops[j].name;
      std::vector<float> y(static_cast<size_t>(m * n), 7.0f);
      sink.status(nm, qc::qgemm_prepacked_quantized(prepared[i], acts[j], y.data()));
      sink.data(nm + "_y", y.data(), y.size() * 4, "f32");
    }
  // M = 1: the first activation row alone
  for (int j = 0; j < 3; ++j) {
    qc::CanonicalQuantTensor one;
    const std::string nm = std::string("proj_gemv_") + aops[j].name;
    sink.status(nm + "_source", qc::quantize_canonical({af.data(), qc::FloatStorageType::kF32, k},
                                                       1, k, aops[j].layout, aops[j].group, &one));
    std::vector<float> y(static_cast<size_t>(n), 7.0f);
    sink.status(nm, qc::qgemv_prepacked_quantized(prepared[0], one, y.data()));
    sink.data(nm + "_y", y.data(), y.size() * 4, "f32");
  }
  // validation: rows for the GEMV form, K, output, readiness, GGUF weights
  std::vector<float> y(static_cast<size_t>(m * n), 7.0f);
  sink.status("proj_gemv_rows5", qc::qgemv_prepacked_quantized(prepared[0], acts[0], y.data()));
  qc::CanonicalQuantTensor narrow;
  sink.status("proj_narrow_source",
              qc::quantize_canonical({af.data(), qc::FloatStorageType::kF32, m * 256}, m, 256,
                                     L::kInt8Symmetric, 0, &narrow));
  sink.status("proj_k_mismatch", qc::qgemm_prepacked_quantized(prepared[0], narrow, y.data()));
  sink.status("proj_null_y", qc::qgemm_prepacked_quantized(prepared[0], acts[0], nullptr));
  qc::CpuPackedWeights empty;
  sink.status("proj_unprepared", qc::qgemm_prepacked_quantized(empty, acts[0], y.data()));
  std::size_t bytes = 0;
  (void)qc::qgemv_packed_size(qc::QuantFormat::kQ8_0, n, k, &bytes);
  std::vector<uint8_t> gguf(bytes);
  sink.status("proj_gguf_pack", qc::qgemv_pack(qc::QuantFormat::kQ8_0, wf.data(), n, k, gguf.data()));
  qc::CpuPackedWeights gw;
  sink.status("proj_gguf_prepare", gw.prepare(qc::QuantFormat::kQ8_0, gguf.data(), n, k));
  sink.status("proj_gguf_weights", qc::qgemm_prepacked_quantized(gw, acts[0], y.data()));
  qc::CanonicalQuantTensor bad = acts[0];
  bad.scales.pop_back();
  sink.status("proj_invalid_activation", qc::qgemm_prepacked_quantized(prepared[0], bad, y.data()));
  sink.data("proj_untouched", y.data(), y.size() * 4, "f32");
  // an fp8 activation tensor (one tensor scale): computed by the reference only
  qc::CanonicalQuantTensor f8;
  f8.metadata.layout = L::kFP8E4M3FN;
  f8.metadata.logical_rows = m;
  f8.metadata.logical_columns = k;
  f8.metadata.scale_mode = qc::QuantScaleMode::kTensor;
  f8.metadata.scale_encoding = qc::QuantScaleEncoding::kFP32;
  f8.metadata.scale_count = 1;
  f8.data.assign(static_cast<size_t>(m * k), 0x38);
  f8.scales.assign(1, 0.5f);
  sink.status("other_proj_fp8_activation", qc::qgemm_prepacked_quantized(prepared[0], f8, y.data()));
}

inline void run(Sink& sink) {
  projections(sink);

  const long long rows = 48, cols = 256;
  const size_t n = static_cast<size_t>(rows * cols);
  const std::vector<float> x = matrix(0x5eed, rows, cols);
  const std::vector<uint16_t> xh = f16_matrix(0xf16, n);
  const std::vector<uint16_t> xb = bf16_matrix(x);
  const qc::FloatStorageInput f32{x.data(), qc::FloatStorageType::kF32, rows * cols};
  const qc::FloatStorageInput f16{xh.data(), qc::FloatStorageType::kF16, rows * cols};
  const qc::FloatStorageInput bf16{xb.data(), qc::FloatStorageType::kBF16, rows * cols};

  // kInt8Symmetric: per row (group 0 and group = cols), groups, 16-bit inputs
  round_trip(sink, "sym_row_f32", f32, rows, cols, L::kInt8Symmetric, 0);
  round_trip(sink, "sym_gcols_f32", f32, rows, cols, L::kInt8Symmetric, cols);
  round_trip(sink, "sym_g64_f32", f32, rows, cols, L::kInt8Symmetric, 64);
  round_trip(sink, "sym_g32_f16", f16, rows, cols, L::kInt8Symmetric, 32);
  round_trip(sink, "sym_g128_bf16", bf16, rows, cols, L::kInt8Symmetric, 128);
  // kInt8Affine: per row only (group 0 or cols)
  round_trip(sink, "aff_row_f32", f32, rows, cols, L::kInt8Affine, 0);
  round_trip(sink, "aff_gcols_bf16", bf16, rows, cols, L::kInt8Affine, cols);
  round_trip(sink, "aff_row_f16", f16, rows, cols, L::kInt8Affine, 0);

  // validation order: tensor, shape, input count, finiteness, then the layout's shape
  qc::CanonicalQuantTensor t;
  sink.status("null_tensor", qc::quantize_canonical(f32, rows, cols, L::kInt8Symmetric, 0, nullptr));
  sink.status("rows0", qc::quantize_canonical(f32, 0, cols, L::kInt8Symmetric, 0, &t));
  sink.status("cols_neg", qc::quantize_canonical(f32, rows, -4, L::kInt8Symmetric, 0, &t));
  qc::FloatStorageInput short_in = f32;
  short_in.count -= 1;
  sink.status("count_mismatch", qc::quantize_canonical(short_in, rows, cols, L::kInt8Symmetric, 0, &t));
  qc::FloatStorageInput null_in = f32;
  null_in.data = nullptr;
  sink.status("null_input", qc::quantize_canonical(null_in, rows, cols, L::kInt8Affine, 0, &t));
  std::vector<float> bad = x;
  bad[3 * cols + 17] = std::numeric_limits<float>::quiet_NaN();
  const qc::FloatStorageInput badin{bad.data(), qc::FloatStorageType::kF32, rows * cols};
  sink.status("nonfinite", qc::quantize_canonical(badin, rows, cols, L::kInt8Symmetric, 0, &t));
  sink.status("nonfinite_bad_group",
              qc::quantize_canonical(badin, rows, cols, L::kInt8Symmetric, 100, &t));
  sink.status("nonfinite_affine", qc::quantize_canonical(badin, rows, cols, L::kInt8Affine, 0, &t));
  std::vector<uint16_t> hinf = xh;
  hinf[99] = 0x7c00;   // +inf in f16
  const qc::FloatStorageInput hinfin{hinf.data(), qc::FloatStorageType::kF16, rows * cols};
  sink.status("nonfinite_f16", qc::quantize_canonical(hinfin, rows, cols, L::kInt8Symmetric, 32, &t));
  sink.status("bad_group", qc::quantize_canonical(f32, rows, cols, L::kInt8Symmetric, 100, &t));
  sink.status("neg_group", qc::quantize_canonical(f32, rows, cols, L::kInt8Symmetric, -32, &t));
  sink.status("affine_group", qc::quantize_canonical(f32, rows, cols, L::kInt8Affine, 64, &t));

  // layouts other than int8: statuses only
  sink.status("other_int4_g32", qc::quantize_canonical(f32, rows, cols, L::kInt4Symmetric, 32, &t));
  sink.status("other_int4_g0", qc::quantize_canonical(f32, rows, cols, L::kInt4Symmetric, 0, &t));
  sink.status("other_uint4_g64", qc::quantize_canonical(f32, rows, cols, L::kUInt4Affine, 64, &t));
  sink.status("other_uint4_g48", qc::quantize_canonical(f32, rows, cols, L::kUInt4Affine, 48, &t));
  sink.status("other_fp8_row", qc::quantize_canonical(f32, rows, cols, L::kFP8E4M3FN, 0, &t));
  sink.status("other_fp8_g100", qc::quantize_canonical(f32, rows, cols, L::kFP8E5M2, 100, &t));
  sink.status("other_fp4_g32", qc::quantize_canonical(f32, rows, cols, L::kFP4E2M1, 32, &t));
  sink.status("other_mxfp8", qc::quantize_canonical(f32, rows, cols, L::kMXFP8E4M3E8M0, 0, &t));
  sink.status("other_mxfp4_cols48",
              qc::quantize_canonical({x.data(), qc::FloatStorageType::kF32, rows * 48}, rows, 48,
                                     L::kMXFP4E2M1E8M0, 0, &t));
  sink.status("other_nvfp4", qc::quantize_canonical(f32, rows, cols, L::kNVFP4E2M1E4M3, 0, &t));
  sink.status("other_nvfp4_cols40",
              qc::quantize_canonical({x.data(), qc::FloatStorageType::kF32, rows * 40}, rows, 40,
                                     L::kNVFP4E2M1E4M3, 0, &t));
  sink.status("other_bitnet_g0", qc::quantize_canonical(f32, rows, cols, L::kBitNetTernary, 0, &t));
  sink.status("other_bitnet_g48", qc::quantize_canonical(f32, rows, cols, L::kBitNetTernary, 48, &t));
  sink.status("other_turbo_key", qc::quantize_canonical(f32, rows, cols, L::kTurboQuantKey, 0, &t));
  sink.status("other_nonfinite_fp8", qc::quantize_canonical(badin, rows, cols, L::kFP8E4M3FN, 0, &t));

  // dequantize_canonical: output, tensor validation, then the count
  qc::CanonicalQuantTensor good;
  sink.status("deq_source", qc::quantize_canonical(f32, rows, cols, L::kInt8Affine, 0, &good));
  std::vector<float> out(n + 1, 7.0f);
  sink.status("deq_null_out", qc::dequantize_canonical(good, nullptr, rows * cols));
  sink.status("deq_count_high", qc::dequantize_canonical(good, out.data(), rows * cols + 1));
  sink.status("deq_count_zero", qc::dequantize_canonical(good, out.data(), 0));
  qc::CanonicalQuantTensor broken = good;
  broken.scales.pop_back();
  sink.status("deq_invalid_tensor", qc::dequantize_canonical(broken, out.data(), rows * cols));
  sink.data("deq_untouched", out.data(), out.size() * 4, "f32");
  // a kFP8E4M3FN tensor with one tensor scale (valid in the contract)
  qc::CanonicalQuantTensor f8;
  f8.metadata.layout = L::kFP8E4M3FN;
  f8.metadata.logical_rows = rows;
  f8.metadata.logical_columns = cols;
  f8.metadata.scale_mode = qc::QuantScaleMode::kTensor;
  f8.metadata.scale_encoding = qc::QuantScaleEncoding::kFP32;
  f8.metadata.scale_count = 1;
  f8.data.assign(n, 0x38);
  f8.scales.assign(1, 0.5f);
  sink.status("other_deq_fp8", qc::dequantize_canonical(f8, out.data(), rows * cols));
}

}  // namespace canonical_quant_scenarios
