// Drop-in of the canonical tensor container and the W8A8 importer of the
// reference's include/quixicore_cpu/quant_import.h.  A CanonicalQuantTensor
// owns canonical contract bytes plus logical side tables (never a device or
// panel layout), so it stays portable and serializable; the GPU copies it
// into device memory in CpuPackedWeights::prepare.
//
// Provided: the container, validate_canonical_quant_tensor,
// import_smoothquant_w8a8 and quant_import_provenance_name.  The AWQ, GPTQ,
// AutoRound and BitNet importers of the reference build layouts other than
// int8 (int4 / fp8 / fp4 / ternary), which this GPU path does not compute.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "quixicore_cpu/quant_contract.h"

namespace quixicore_cpu {

enum class QuantImportProvenance {
  kCanonical,
  kAWQ,
  kGPTQ,
  kAutoRound,
  kSmoothQuant,
  kBitNet,
};

struct CanonicalQuantTensor {
  QuantTensorMetadata metadata;
  std::vector<std::uint8_t> data;          // canonical contract bytes
  std::vector<std::uint8_t> scale_codes;
  std::vector<float> scales;
  std::vector<float> zero_points;
  std::vector<float> activation_scales;
  std::vector<int> activation_zero_points;
  std::vector<int> group_index;
  std::vector<int> act_order;
  std::vector<std::int32_t> row_sums;
  QuantImportProvenance provenance = QuantImportProvenance::kCanonical;
};

Status validate_canonical_quant_tensor(const CanonicalQuantTensor& tensor);

// SmoothQuant W8A8 export: int8 weights [rows, columns], one f32 scale per
// output row, activation scales (and optionally zero points, for the AZP
// route); the row sums are computed when not given.  Produces a
// kInt8Symmetric tensor with channel scales.
struct SmoothQuantW8A8Source {
  const std::int8_t* weights = nullptr;
  std::size_t weight_count = 0;
  const float* weight_scales = nullptr;
  std::size_t weight_scale_count = 0;
  const float* activation_scales = nullptr;
  std::size_t activation_scale_count = 0;
  const int* activation_zero_points = nullptr;
  std::size_t activation_zero_point_count = 0;
  const std::int32_t* row_sums = nullptr;
  std::size_t row_sum_count = 0;
  long long rows = 0;
  long long columns = 0;
};
Status import_smoothquant_w8a8(const SmoothQuantW8A8Source& source,
                               CanonicalQuantTensor* tensor);

const char* quant_import_provenance_name(QuantImportProvenance provenance);

}  // namespace quixicore_cpu
