// Drop-in of CpuPackedWeights (include/quixicore_cpu/packed_weights.h:14-97
// of the reference).  prepare() keeps the canonical bytes and builds the same
// row panel ([row_panel, k_block, row_lane, block_bytes], zero-padded; for a
// canonical tensor followed by its side tables) so contract_data() /
// panel_data() / info() match the reference on the host, and also uploads
// the canonical bytes to a device mirror that the prepared GPU entry points
// read.  Move-only.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>

#include "quixicore_cpu/qgemv.h"
#include "quixicore_cpu/quant_contract.h"

namespace quixicore_cpu {

struct CanonicalQuantTensor;

enum class CpuPanelLayout {
  kAuto,
  kPortableRows1,
  kNeonRows4,
  kAvx2Rows8,
  kAvx512Rows16,
};

enum class CpuPreparedIsa {
  kPortable,
  kNeon,
  kDotProd,
  kI8MM,
  kSVE,
  kSME,
  kAvx2,
  kAvx512,
  kAvx512VNNI,
  kAMX,
};

// Field order and defaults as in the reference, plus device_bytes (the size
// of the device mirror) at the end.
struct CpuPackedWeightsInfo {
  QuantFormat format = QuantFormat::kQ8_0;
  CanonicalQuantLayout canonical_layout = CanonicalQuantLayout::kInt4Symmetric;
  QuantTensorMetadata quant_metadata{};
  bool has_canonical_layout = false;
  CpuPanelLayout layout = CpuPanelLayout::kPortableRows1;
  long long rows = 0;
  long long columns = 0;
  long long row_tile = 0;
  long long block_size = 0;
  long long blocks_per_row = 0;
  std::size_t block_bytes = 0;
  std::size_t contract_bytes = 0;
  std::size_t panel_bytes = 0;
  std::uint32_t prepared_version = 0;
  CpuPreparedIsa required_isa = CpuPreparedIsa::kPortable;
  long long column_tile = 0;
  std::size_t panel_alignment = 0;
  std::size_t scale_table_offset = static_cast<std::size_t>(-1);
  std::size_t scale_code_table_offset = static_cast<std::size_t>(-1);
  std::size_t zero_point_table_offset = static_cast<std::size_t>(-1);
  std::size_t row_sum_table_offset = static_cast<std::size_t>(-1);
  std::size_t group_index_offset = static_cast<std::size_t>(-1);
  std::size_t act_order_offset = static_cast<std::size_t>(-1);
  std::size_t activation_scale_offset = static_cast<std::size_t>(-1);
  std::size_t activation_zero_point_offset = static_cast<std::size_t>(-1);
  std::size_t lut_offset = static_cast<std::size_t>(-1);
  std::size_t logical_bytes = 0;
  std::size_t prepared_bytes = 0;
  double memory_amplification = 0.0;
  std::uint64_t preparation_ns = 0;
  std::size_t device_bytes = 0;  // device mirror: canonical bytes (+ side tables)
};

class CpuPackedWeights {
 public:
  CpuPackedWeights();
  ~CpuPackedWeights();
  CpuPackedWeights(CpuPackedWeights&& other) noexcept;
  CpuPackedWeights& operator=(CpuPackedWeights&& other) noexcept;
  CpuPackedWeights(const CpuPackedWeights&) = delete;
  CpuPackedWeights& operator=(const CpuPackedWeights&) = delete;

  // contract_packed may be host or device memory.  kAuto resolves from the
  // host CPU's features as the reference does (AVX-512 F/BW/VL/DQ: 16 rows,
  // AVX2: 8, else 1); the GPU reads the canonical bytes whatever the panel.
  Status prepare(QuantFormat format, const void* contract_packed, long long rows,
                 long long columns, CpuPanelLayout layout = CpuPanelLayout::kAuto);
  // Canonical tensor (host vectors): host panel plus side tables as in the
  // reference, and a device mirror of the data and tables.
  Status prepare(const CanonicalQuantTensor& tensor,
                 CpuPanelLayout layout = CpuPanelLayout::kAuto);
  void reset() noexcept;

  bool ready() const noexcept;
  CpuPackedWeightsInfo info() const noexcept;
  const void* contract_data() const noexcept;  // host copy of the canonical bytes
  const void* panel_data() const noexcept;     // host row panel (+ tables), 64-byte aligned
  const void* device_data() const noexcept;    // device mirror of the canonical bytes
  // Device mirror of a canonical tensor's f32 scales and int32 row sums
  // (nullptr when the tensor has none, or for GGUF formats).
  const float* device_scales() const noexcept;
  const std::int32_t* device_row_sums() const noexcept;
  const float* device_zero_points() const noexcept;   // canonical zero points (f32)

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

const char* cpu_panel_layout_name(CpuPanelLayout layout);
const char* cpu_prepared_isa_name(CpuPreparedIsa isa);

}  // namespace quixicore_cpu
