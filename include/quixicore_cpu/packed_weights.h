// Drop-in of CpuPackedWeights (include/quixicore_cpu/packed_weights.h:14-97
// of the reference).  prepare() keeps the canonical bytes and builds the same
// row panel ([row_panel, k_block, row_lane, block_bytes], zero-padded) so
// contract_data()/panel_data() stay byte-identical on the host, and also
// uploads the canonical bytes to a device mirror that qgemm_prepacked and
// qgemv_prepacked read.  Move-only.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>

#include "quixicore_cpu/qgemv.h"

namespace quixicore_cpu {

enum class CpuPanelLayout {
  kAuto,
  kPortableRows1,
  kNeonRows4,
  kAvx2Rows8,
  kAvx512Rows16,
};

struct CpuPackedWeightsInfo {
  QuantFormat format = QuantFormat::kQ8_0;
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
  long long column_tile = 0;
  std::size_t panel_alignment = 0;
  std::size_t prepared_bytes = 0;
  double memory_amplification = 0.0;
  std::uint64_t preparation_ns = 0;
  std::size_t device_bytes = 0;  // size of the device mirror (canonical bytes)
};

class CpuPackedWeights {
 public:
  CpuPackedWeights();
  ~CpuPackedWeights();
  CpuPackedWeights(CpuPackedWeights&& other) noexcept;
  CpuPackedWeights& operator=(CpuPackedWeights&& other) noexcept;
  CpuPackedWeights(const CpuPackedWeights&) = delete;
  CpuPackedWeights& operator=(const CpuPackedWeights&) = delete;

  // contract_packed may be host or device memory.
  Status prepare(QuantFormat format, const void* contract_packed, long long rows,
                 long long columns, CpuPanelLayout layout = CpuPanelLayout::kAuto);
  void reset() noexcept;

  bool ready() const noexcept;
  CpuPackedWeightsInfo info() const noexcept;
  const void* contract_data() const noexcept;  // host copy of the canonical bytes
  const void* panel_data() const noexcept;     // host row panel, 64-byte aligned
  const void* device_data() const noexcept;    // device mirror of the canonical bytes

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

const char* cpu_panel_layout_name(CpuPanelLayout layout);

}  // namespace quixicore_cpu
