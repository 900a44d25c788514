// quantize_canonical / dequantize_canonical of the reference's
// include/quixicore_cpu/quant_import.h:42-45,53-54
// (kernels/quantization/quant_import_ref.cpp:552-681,717-838) for the
// canonical int8 layouts, on the GPU quantizers and decode kernel:
//   kInt8Symmetric = quantize_int8 per row or group (:586-605);
//   kInt8Affine    = quantize_int8_asymmetric per row (:606-622).
// Every other layout returns kUnsupportedFormat after the reference's common
// validation and that layout's own shape checks (the reference computes them
// on the CPU; this GPU path computes the int8 layouts of the W8A8 route).
// The tensor is host data (std::vector tables), as in the reference; the
// input / output buffers may be host or device memory.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <limits>
#include <new>
#include <stdexcept>
#include <vector>

#include "quixicore_cpu/float_storage.h"
#include "quixicore_cpu/quant_import.h"
#include "quixicore_hip.h"
#include "qc_dropin.h"

namespace quixicore_cpu {
namespace {

using L = CanonicalQuantLayout;

// checked_product of quant_import_ref.cpp:19-26.
bool checked_product(long long a, long long b, std::size_t* out) {
  if (a <= 0 || b <= 0) return false;
  const auto ua = static_cast<unsigned long long>(a), ub = static_cast<unsigned long long>(b);
  if (ua > std::numeric_limits<std::size_t>::max() / ub) return false;
  *out = static_cast<std::size_t>(ua * ub);
  return true;
}

std::size_t storage_bytes(FloatStorageType t) { return t == FloatStorageType::kF32 ? 4 : 2; }

// Layout-specific shape checks of the layouts this path does not compute,
// in the reference's switch (:569-676), so that a caller sees the same
// kInvalidShape before kUnsupportedFormat.
Status other_layout(L layout, long long columns, long long group_size) {
  switch (layout) {
    case L::kInt4Symmetric:
    case L::kUInt4Affine:   // :571-573, quantize_u4_affine :308-311
      if (group_size <= 0 || columns % group_size != 0 || (columns & 1) != 0)
        return Status::kInvalidShape;
      break;
    case L::kFP8E4M3FN:
    case L::kFP8E5M2:
    case L::kFP4E2M1: {     // quantize_grouped_fp :192-213 with no requested mode
      const bool fp4 = layout == L::kFP4E2M1;
      const long long k_group = group_size == 0 ? columns : group_size;
      if (k_group <= 0 || columns % k_group != 0 || (fp4 && (columns & 1) != 0))
        return Status::kInvalidShape;
      break;
    }
    case L::kMXFP8E4M3E8M0:
    case L::kMXFP4E2M1E8M0:  // quantize_mx :358
      if (columns % 32 != 0) return Status::kInvalidShape;
      break;
    case L::kNVFP4E2M1E4M3:  // :641
      if (columns % 16 != 0) return Status::kInvalidShape;
      break;
    case L::kBitNetTernary: {  // :659-661
      const long long effective = group_size == 0 ? 32 : group_size;
      if (columns % effective != 0 || effective % 32 != 0) return Status::kInvalidShape;
      break;
    }
    default:
      break;
  }
  return Status::kUnsupportedFormat;
}

}  // namespace

Status quantize_canonical(FloatStorageInput input, long long rows, long long columns,
                          CanonicalQuantLayout layout, long long group_size,
                          CanonicalQuantTensor* tensor, bool scale_2d) {
  (void)scale_2d;   // NVFP4 only
  if (tensor == nullptr) return Status::kInvalidArgument;
  std::size_t elements = 0;
  if (!checked_product(rows, columns, &elements)) return Status::kInvalidShape;
  // stage_float_input (:154-172): the count, then exact f32 values, then finiteness
  if (input.data == nullptr || input.count <= 0 || static_cast<std::size_t>(input.count) != elements)
    return Status::kInvalidArgument;
  if (input.type != FloatStorageType::kF32 && input.type != FloatStorageType::kF16 &&
      input.type != FloatStorageType::kBF16)
    return Status::kInvalidArgument;
  if (elements > static_cast<std::size_t>(LLONG_MAX / 4)) return Status::kInvalidShape;
  try {
    detail::Staging st(nullptr);
    const void* xin = st.in(input.data, elements * storage_bytes(input.type));
    float* x = input.type == FloatStorageType::kF32
                   ? const_cast<float*>(static_cast<const float*>(xin))
                   : static_cast<float*>(st.scratch(elements * sizeof(float)));
    int* flag = static_cast<int*>(st.scratch(sizeof(int)));
    if (st.status() != Status::kOk) return st.status();
    const hipStream_t s = st.stream();
    if (input.type != FloatStorageType::kF32) {
      const int c = qc_hip_storage_to_f32(xin, static_cast<int>(input.type),
                                          static_cast<long long>(elements), x, s);
      if (c != QC_OK) return st.finish(c);
    }
    int nonfinite = 0;
    hipError_t e = hipMemsetAsync(flag, 0, sizeof(int), s);
    if (e == hipSuccess) {
      const int c = qc_hip_nonfinite_scan(x, static_cast<long long>(elements), flag, s);
      if (c != QC_OK) return st.finish(c);
      e = hipMemcpyAsync(&nonfinite, flag, sizeof(int), hipMemcpyDeviceToHost, s);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return detail::from_hip(e);
    if (nonfinite != 0) return Status::kInvalidArgument;

    CanonicalQuantTensor candidate;   // initialize_metadata (:174-183)
    candidate.metadata.layout = layout;
    candidate.metadata.logical_rows = rows;
    candidate.metadata.logical_columns = columns;
    candidate.metadata.group_size = group_size;
    candidate.provenance = QuantImportProvenance::kCanonical;
    int capi = QC_OK;
    if (layout == L::kInt8Symmetric) {
      const long long effective = group_size == 0 ? columns : group_size;
      if (effective <= 0 || columns % effective != 0) return Status::kInvalidShape;
      candidate.data.resize(elements);
      candidate.scales.resize(static_cast<std::size_t>(rows) *
                              static_cast<std::size_t>(columns / effective));
      auto* codes = static_cast<std::int8_t*>(st.out(candidate.data.data(), elements));
      auto* scales = static_cast<float*>(
          st.out(candidate.scales.data(), candidate.scales.size() * sizeof(float)));
      if (st.status() != Status::kOk) return st.status();
      capi = qc_hip_quantize_int8(x, codes, scales, rows, columns, effective, flag, s);
      const Status done = st.finish(capi);
      if (done != Status::kOk) return done;
      candidate.metadata.group_size = effective;
      candidate.metadata.scale_mode = effective == columns ? QuantScaleMode::kRow
                                                           : QuantScaleMode::kGroup;
      candidate.metadata.scale_encoding = QuantScaleEncoding::kFP32;
      candidate.metadata.scale_count = candidate.scales.size();
    } else if (layout == L::kInt8Affine) {
      if (group_size != 0 && group_size != columns) return Status::kInvalidShape;
      candidate.data.resize(elements);
      candidate.scales.resize(static_cast<std::size_t>(rows));
      std::vector<int> zeros(static_cast<std::size_t>(rows));
      auto* codes = static_cast<std::int8_t*>(st.out(candidate.data.data(), elements));
      auto* scales = static_cast<float*>(
          st.out(candidate.scales.data(), candidate.scales.size() * sizeof(float)));
      auto* zp = static_cast<int*>(st.out(zeros.data(), zeros.size() * sizeof(int)));
      if (st.status() != Status::kOk) return st.status();
      capi = qc_hip_quantize_int8_asymmetric(x, codes, scales, zp, rows, columns, flag, s);
      const Status done = st.finish(capi);
      if (done != Status::kOk) return done;
      candidate.zero_points.assign(zeros.begin(), zeros.end());
      candidate.metadata.group_size = columns;
      candidate.metadata.scale_mode = QuantScaleMode::kRow;
      candidate.metadata.scale_encoding = QuantScaleEncoding::kFP32;
      candidate.metadata.zero_point_mode = QuantZeroPointMode::kInteger;
      candidate.metadata.scale_count = candidate.scales.size();
      candidate.metadata.zero_point_count = candidate.zero_points.size();
    } else {
      return other_layout(layout, columns, group_size);
    }
    const Status valid = validate_canonical_quant_tensor(candidate);
    if (valid != Status::kOk) return valid;
    *tensor = std::move(candidate);
    return Status::kOk;
  } catch (const std::bad_alloc&) {
    return Status::kOutOfMemory;
  } catch (const std::length_error&) {
    return Status::kOutOfMemory;
  }
}

Status dequantize_canonical(const CanonicalQuantTensor& tensor, float* output,
                            long long output_count) {
  if (output == nullptr) return Status::kInvalidArgument;
  Status status = validate_canonical_quant_tensor(tensor);
  if (status != Status::kOk) return status;
  const QuantTensorMetadata& md = tensor.metadata;
  std::size_t elements = 0;
  if (!checked_product(md.logical_rows, md.logical_columns, &elements) || output_count <= 0 ||
      static_cast<std::size_t>(output_count) != elements)
    return Status::kInvalidShape;
  if (md.layout != L::kInt8Symmetric && md.layout != L::kInt8Affine)
    return Status::kUnsupportedFormat;
  // int8 layouts carry row / channel / group scales and no group index
  // (validate_quant_metadata); the scale of (r, c) is scales[r * groups + c / g].
  const long long groups =
      static_cast<long long>(md.scale_count / static_cast<std::size_t>(md.logical_rows));
  detail::Staging st(nullptr);
  qc_cint8_weights w{};
  w.codes = static_cast<const std::int8_t*>(st.in(tensor.data.data(), elements));
  w.scales = static_cast<const float*>(st.in(tensor.scales.data(), tensor.scales.size() * 4));
  w.zero_points = tensor.zero_points.empty()
                      ? nullptr
                      : static_cast<const float*>(
                            st.in(tensor.zero_points.data(), tensor.zero_points.size() * 4));
  w.rows = md.logical_rows;
  w.cols = md.logical_columns;
  w.groups = groups;
  float* out = static_cast<float*>(st.out(output, elements * sizeof(float)));
  if (st.status() != Status::kOk) return st.status();
  return st.finish(qc_hip_cint8_dequantize(&w, nullptr, out, st.stream()));
}

}  // namespace quixicore_cpu
