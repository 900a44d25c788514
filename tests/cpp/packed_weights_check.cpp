// CpuPackedWeights through the C++ drop-in API, as the reference's
// tests/correctness/test_packed_weights.cpp exercises it (:33-118 per format
// and layout, :250-265 invalid calls), plus canonical int8 tensors
// (src/memory/packed_weights.cpp:280-412).  Checks run in this program
// (REQUIRE) and every prepared panel and info record is written under argv[1]
// so that tests/test_gpu_packed_weights.py can compare them, byte for byte,
// with the reference's own CpuPackedWeights (oracle/_ref).
//
// Output: <dir>/manifest.txt with lines "<case> <status>" and, per prepared
// case, <case>.panel (prepared_bytes), <case>.info (24 int64, the order of
// oracle/ref_shim.cpp's dump_info) and <case>.in (the input bytes).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "quixicore_cpu/packed_weights.h"
#include "quixicore_cpu/qgemm.h"
#include "quixicore_cpu/qgemv.h"
#include "quixicore_cpu/quant_import.h"
#include "quixicore_cpu/workspace.h"

namespace qc = quixicore_cpu;

#define REQUIRE(c)                                                            \
  do {                                                                        \
    if (!(c)) {                                                               \
      std::fprintf(stderr, "FAILED: %s at %s:%d\n", #c, __FILE__, __LINE__); \
      return false;                                                           \
    }                                                                         \
  } while (0)

namespace {

std::string g_dir;
FILE* g_manifest = nullptr;

uint32_t next(uint32_t* s) {
  *s ^= *s << 13;
  *s ^= *s >> 17;
  *s ^= *s << 5;
  return *s;
}

void write(const std::string& name, const void* p, size_t n) {
  FILE* f = std::fopen((g_dir + "/" + name).c_str(), "wb");
  if (f == nullptr) return;
  if (n) std::fwrite(p, 1, n, f);
  std::fclose(f);
}

void dump(const std::string& name, const qc::CpuPackedWeights& w, const void* in, size_t in_bytes) {
  const qc::CpuPackedWeightsInfo i = w.info();
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
  write(name + ".info", v, sizeof(v));
  write(name + ".panel", w.panel_data(), i.prepared_bytes);
  write(name + ".in", in, in_bytes);
  std::fprintf(g_manifest, "%s 0\n", name.c_str());
}

const qc::CpuPanelLayout kLayouts[] = {qc::CpuPanelLayout::kPortableRows1,
                                       qc::CpuPanelLayout::kNeonRows4,
                                       qc::CpuPanelLayout::kAvx2Rows8,
                                       qc::CpuPanelLayout::kAvx512Rows16};

// tests/correctness/test_packed_weights.cpp:33-118
bool run_format(qc::QuantFormat format, const char* fname) {
  constexpr long long n = 19, k = 64;
  uint32_t state = 0xA341316Cu;
  std::vector<float> dense(n * k);
  for (float& v : dense) v = static_cast<float>(next(&state) >> 8) / 8388608.0f - 1.0f;
  size_t bytes = 0;
  REQUIRE(qc::qgemv_packed_size(format, n, k, &bytes) == qc::Status::kOk);
  std::vector<uint8_t> packed(bytes);
  REQUIRE(qc::qgemv_pack(format, dense.data(), n, k, packed.data()) == qc::Status::kOk);
  for (qc::CpuPanelLayout layout : kLayouts) {
    qc::CpuPackedWeights w;
    REQUIRE(w.prepare(format, packed.data(), n, k, layout) == qc::Status::kOk);
    REQUIRE(w.ready());
    const qc::CpuPackedWeightsInfo info = w.info();
    REQUIRE(info.layout == layout);
    REQUIRE(info.rows == n && info.columns == k);
    REQUIRE(info.contract_bytes == bytes);
    REQUIRE(info.prepared_version == 1);
    REQUIRE(info.column_tile == info.block_size);
    REQUIRE(info.panel_alignment == 64);
    REQUIRE(info.prepared_bytes == info.panel_bytes);
    REQUIRE(info.memory_amplification >= 1.0);
    REQUIRE(std::string(qc::cpu_prepared_isa_name(info.required_isa)) != "unknown");
    REQUIRE(!info.has_canonical_layout);
    REQUIRE(std::memcmp(w.contract_data(), packed.data(), bytes) == 0);
    REQUIRE(reinterpret_cast<uintptr_t>(w.panel_data()) % 64 == 0);
    dump(std::string(fname) + "_" + qc::cpu_panel_layout_name(layout), w, packed.data(), bytes);

    for (long long m : {1LL, 3LL, 17LL, 65LL}) {
      std::vector<float> x(m * k), want(m * n), got(m * n);
      for (float& v : x) v = static_cast<float>(next(&state) >> 8) / 8388608.0f - 1.0f;
      REQUIRE(qc::qgemm(format, packed.data(), x.data(), want.data(), m, n, k) ==
              qc::Status::kOk);
      qc::Workspace ws;
      REQUIRE(qc::qgemm_prepacked(w, x.data(), got.data(), m, &ws) == qc::Status::kOk);
      for (size_t i = 0; i < got.size(); ++i)
        REQUIRE(std::fabs(want[i] - got[i]) <= 3e-5f * (1.0f + std::fabs(want[i])));
      REQUIRE(ws.used() == 0);
      if (m >= 64) {
        const size_t capacity = ws.capacity();
        REQUIRE(capacity != 0);
        REQUIRE(qc::qgemm_prepacked(w, x.data(), got.data(), m, &ws) == qc::Status::kOk);
        REQUIRE(ws.capacity() == capacity);
        REQUIRE(ws.used() == 0);
      }
    }
  }
  // kAuto resolves from this host's CPU (compared with the reference's choice)
  qc::CpuPackedWeights a;
  REQUIRE(a.prepare(format, packed.data(), n, k) == qc::Status::kOk);
  dump(std::string(fname) + "_auto", a, packed.data(), bytes);
  return true;
}

// tests/correctness/test_packed_weights.cpp:250-265
bool run_invalid() {
  qc::CpuPackedWeights w;
  uint8_t byte = 0;
  REQUIRE(w.prepare(qc::QuantFormat::kQ4_0, nullptr, 1, 32) == qc::Status::kInvalidArgument);
  REQUIRE(w.prepare(qc::QuantFormat::kQ4_0, &byte, 1, 31) == qc::Status::kInvalidShape);
  REQUIRE(w.prepare(qc::QuantFormat::kQ4_0, &byte, 1, 32, static_cast<qc::CpuPanelLayout>(99)) ==
          qc::Status::kInvalidArgument);
  float v = 0.0f;
  REQUIRE(qc::qgemm_prepacked(w, &v, &v, 1) == qc::Status::kInvalidArgument);
  REQUIRE(!w.ready());
  REQUIRE(w.info().rows == 0 && w.panel_data() == nullptr && w.contract_data() == nullptr);
  return true;
}

// Canonical int8 tensors: SmoothQuant import (channel scales, row sums
// computed, activation scales and zero points) and an affine tensor with
// group scales, each in every layout.
bool run_canonical() {
  constexpr long long n = 19, k = 64;
  uint32_t state = 0x12345u;
  std::vector<int8_t> wq(n * k);
  for (int8_t& v : wq) v = static_cast<int8_t>(static_cast<int>(next(&state) >> 24) - 128);
  wq[0] = -128;
  std::vector<float> ws(n), as(3);
  for (float& v : ws) v = static_cast<float>(next(&state) >> 8) / 1e9f;
  for (float& v : as) v = static_cast<float>(next(&state) >> 8) / 1e8f;
  const int azp[3] = {-3, 0, 7};
  qc::SmoothQuantW8A8Source src;
  src.weights = wq.data();
  src.weight_count = wq.size();
  src.weight_scales = ws.data();
  src.weight_scale_count = ws.size();
  src.activation_scales = as.data();
  src.activation_scale_count = as.size();
  src.activation_zero_points = azp;
  src.activation_zero_point_count = 3;
  src.rows = n;
  src.columns = k;
  write("canon_w.in", wq.data(), wq.size());
  write("canon_ws.in", ws.data(), ws.size() * sizeof(float));
  write("canon_as.in", as.data(), as.size() * sizeof(float));
  write("canon_azp.in", azp, sizeof(azp));
  qc::CanonicalQuantTensor sq;
  REQUIRE(qc::import_smoothquant_w8a8(src, &sq) == qc::Status::kOk);
  REQUIRE(sq.provenance == qc::QuantImportProvenance::kSmoothQuant);
  REQUIRE(std::string(qc::quant_import_provenance_name(sq.provenance)) == "smoothquant");
  REQUIRE(sq.row_sums.size() == static_cast<size_t>(n));
  long long sum0 = 0;
  for (long long c = 0; c < k; ++c) sum0 += wq[c];
  REQUIRE(sq.row_sums[0] == sum0);
  // bad counts and non-finite scales
  qc::CanonicalQuantTensor bad;
  qc::SmoothQuantW8A8Source s2 = src;
  s2.weight_scale_count = n - 1;
  REQUIRE(qc::import_smoothquant_w8a8(s2, &bad) == qc::Status::kInvalidShape);
  s2 = src;
  s2.weights = nullptr;
  REQUIRE(qc::import_smoothquant_w8a8(s2, &bad) == qc::Status::kInvalidArgument);
  std::vector<float> nanws = ws;
  nanws[3] = NAN;
  s2 = src;
  s2.weight_scales = nanws.data();
  REQUIRE(qc::import_smoothquant_w8a8(s2, &bad) == qc::Status::kInvalidShape);

  qc::CanonicalQuantTensor af;
  af.metadata.layout = qc::CanonicalQuantLayout::kInt8Affine;
  af.metadata.logical_rows = n;
  af.metadata.logical_columns = k;
  af.metadata.group_size = 32;
  af.metadata.scale_mode = qc::QuantScaleMode::kGroup;
  af.metadata.scale_encoding = qc::QuantScaleEncoding::kFP32;
  af.metadata.zero_point_mode = qc::QuantZeroPointMode::kInteger;
  af.metadata.scale_count = af.metadata.zero_point_count = static_cast<size_t>(n * 2);
  af.data.assign(reinterpret_cast<const uint8_t*>(wq.data()),
                 reinterpret_cast<const uint8_t*>(wq.data()) + wq.size());
  for (long long i = 0; i < n * 2; ++i) {
    af.scales.push_back(static_cast<float>(i + 1) * 0.01f);
    af.zero_points.push_back(static_cast<float>(i % 5) - 2.0f);
  }
  REQUIRE(qc::validate_canonical_quant_tensor(af) == qc::Status::kOk);
  write("canon_af_scales.in", af.scales.data(), af.scales.size() * sizeof(float));
  write("canon_af_zps.in", af.zero_points.data(), af.zero_points.size() * sizeof(float));
  qc::CanonicalQuantTensor af_bad = af;
  af_bad.scales[0] = -1.0f;
  REQUIRE(qc::validate_canonical_quant_tensor(af_bad) == qc::Status::kInvalidShape);
  af_bad = af;
  af_bad.metadata.scale_encoding = qc::QuantScaleEncoding::kFP16;
  REQUIRE(qc::validate_canonical_quant_tensor(af_bad) == qc::Status::kInvalidArgument);

  for (qc::CpuPanelLayout layout : kLayouts) {
    qc::CpuPackedWeights w;
    REQUIRE(w.prepare(sq, layout) == qc::Status::kOk);
    const qc::CpuPackedWeightsInfo i = w.info();
    REQUIRE(i.has_canonical_layout && i.prepared_version == 2);
    REQUIRE(i.canonical_layout == qc::CanonicalQuantLayout::kInt8Symmetric);
    REQUIRE(i.quant_metadata.scale_count == static_cast<size_t>(n));
    REQUIRE(w.device_scales() != nullptr && w.device_row_sums() != nullptr);
    dump(std::string("smoothquant_") + qc::cpu_panel_layout_name(layout), w, wq.data(),
         wq.size());
    qc::CpuPackedWeights g;
    REQUIRE(g.prepare(af, layout) == qc::Status::kOk);
    REQUIRE(g.info().block_size == 32 && g.info().blocks_per_row == 2);
    dump(std::string("affine_group32_") + qc::cpu_panel_layout_name(layout), g, wq.data(),
         wq.size());
  }
  qc::CpuPackedWeights w;
  REQUIRE(w.prepare(sq, static_cast<qc::CpuPanelLayout>(99)) == qc::Status::kInvalidArgument);
  qc::CanonicalQuantTensor empty;
  REQUIRE(w.prepare(empty) == qc::Status::kInvalidShape);
  return true;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: packed_weights_check <output dir>\n");
    return 2;
  }
  g_dir = argv[1];
  g_manifest = std::fopen((g_dir + "/manifest.txt").c_str(), "w");
  if (g_manifest == nullptr) return 2;
  const bool ok = run_format(qc::QuantFormat::kQ4_0, "q4_0") &&
                  run_format(qc::QuantFormat::kQ8_0, "q8_0") && run_invalid() && run_canonical();
  std::fclose(g_manifest);
  if (!ok) return 1;
  std::printf("packed_weights_check: ok\n");
  return 0;
}
