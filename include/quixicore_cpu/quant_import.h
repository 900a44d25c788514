// Drop-in of the canonical tensor container and the W8A8 importer of the
// reference's include/quixicore_cpu/quant_import.h.  A CanonicalQuantTensor
// owns canonical contract bytes plus logical side tables (never a device or
// panel layout), so it stays portable and serializable; the GPU copies it
// into device memory in CpuPackedWeights::prepare.
//
// Provided: the container, validate_canonical_quant_tensor,
// quantize_canonical / dequantize_canonical for the two int8 layouts (on the
// GPU quantizers and decode kernel; the other layouts return
// kUnsupportedFormat after the reference's validation),
// import_smoothquant_w8a8 and quant_import_provenance_name.  The AWQ, GPTQ,
// AutoRound and BitNet importers of the reference build layouts other than
// int8 (int4 / fp8 / fp4 / ternary), which this GPU path does not compute.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "quixicore_cpu/float_storage.h"
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

// Canonical pack / unpack (reference :42-45,53-54;
// kernels/quantization/quant_import_ref.cpp:552-681,717-838).
// kInt8Symmetric: quantize_int8 with group_size (0 = one scale per row), codes
// and f32 scales bit-identical to the reference's.  kInt8Affine (group_size 0
// or columns): quantize_int8_asymmetric per row, integer zero points.  The
// input may be f32, f16 or bf16 storage (decoded exactly), host or device
// memory; the tensor's tables are host vectors.  Other layouts:
// kUnsupportedFormat after the reference's checks (scale_2d is NVFP4's).
Status quantize_canonical(FloatStorageInput input, long long rows, long long columns,
                          CanonicalQuantLayout layout, long long group_size,
                          CanonicalQuantTensor* tensor, bool scale_2d = false);
// output[r][c] = scale * (code - zero) in f32, bit-identical to the
// reference's decode, for the int8 layouts; output may be host or device
// memory of exactly rows * columns floats.
Status dequantize_canonical(const CanonicalQuantTensor& tensor, float* output,
                            long long output_count);

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
