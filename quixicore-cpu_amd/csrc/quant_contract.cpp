// Canonical quantization contract on the host: the per-layout descriptor
// table, metadata and tensor validation, and the SmoothQuant W8A8 importer.
//
// The descriptor values are the reference's table
// (src/memory/quant_contract.cpp:9-62): they are contract data shared with
// every other backend.  The validation steps and their order follow
// src/memory/quant_contract.cpp:99-221 (validate_quant_metadata) and
// kernels/quantization/quant_import_ref.cpp:401-549
// (validate_canonical_quant_tensor), because callers act on the Status each
// check returns.
#include <cmath>
#include <cstring>
#include <limits>
#include <new>
#include <stdexcept>
#include <vector>

#include "quixicore_cpu/quant_contract.h"
#include "quixicore_cpu/quant_import.h"

namespace quixicore_cpu {
namespace {

using L = CanonicalQuantLayout;
using SM = QuantScaleMode;
using SE = QuantScaleEncoding;
using ZP = QuantZeroPointMode;
using PO = QuantPackingOrder;

// {version, layout, name, bits, block elements, block bytes, packing,
//  default scale mode, scale encoding, zero points, scale group,
//  global scale, act order, sparse mask, centroids, cache layout}
constexpr CanonicalQuantDescriptor kTable[] = {
    {1, L::kInt4Symmetric, "int4_symmetric", 4, 0, 0, PO::kLowKFirstNibble, SM::kGroup,
     SE::kFP32, ZP::kNone, 0, false, true, false, false, false},
    {1, L::kUInt4Affine, "uint4_affine", 4, 0, 0, PO::kLowKFirstNibble, SM::kGroup, SE::kFP32,
     ZP::kFractional, 0, false, true, false, false, false},
    {1, L::kInt8Symmetric, "int8_symmetric", 8, 0, 0, PO::kBytePerElement, SM::kRow, SE::kFP32,
     ZP::kNone, 0, false, false, false, false, false},
    {1, L::kInt8Affine, "int8_affine", 8, 0, 0, PO::kBytePerElement, SM::kRow, SE::kFP32,
     ZP::kInteger, 0, false, false, false, false, false},
    {1, L::kFP8E4M3FN, "fp8_e4m3fn", 8, 0, 0, PO::kBytePerElement, SM::kTensor, SE::kFP32,
     ZP::kNone, 0, false, false, false, false, false},
    {1, L::kFP8E5M2, "fp8_e5m2", 8, 0, 0, PO::kBytePerElement, SM::kTensor, SE::kFP32, ZP::kNone,
     0, false, false, false, false, false},
    {1, L::kFP4E2M1, "fp4_e2m1", 4, 0, 0, PO::kLowKFirstNibble, SM::kBlock, SE::kFP16, ZP::kNone,
     0, false, false, false, false, false},
    {1, L::kMXFP8E4M3E8M0, "mxfp8_e4m3_e8m0", 8, 32, 33, PO::kSplitCodesAndMetadata,
     SM::kMicroscaleK32, SE::kE8M0, ZP::kNone, 32, false, false, false, false, false},
    {1, L::kMXFP4E2M1E8M0, "mxfp4_e2m1_e8m0", 4, 32, 17, PO::kSplitCodesAndMetadata,
     SM::kMicroscaleK32, SE::kE8M0, ZP::kNone, 32, false, false, false, false, false},
    {1, L::kNVFP4E2M1E4M3, "nvfp4_e2m1_e4m3", 4, 16, 0, PO::kSplitCodesAndMetadata,
     SM::kNVFP4K16, SE::kE4M3FN, ZP::kNone, 16, true, false, false, false, false},
    {1, L::kBitNetTernary, "bitnet_ternary", 2, 32, 10, PO::kLowKFirstTwoBits, SM::kBlock,
     SE::kFP16, ZP::kNone, 32, false, false, true, false, false},
    {1, L::kTurboQuantKey, "turboquant_key", 0, 32, 0, PO::kLeastSignificantBitStream,
     SM::kTurboQuantK32, SE::kFP16, ZP::kTurboQuantOffset, 32, false, false, false, false, true},
    {1, L::kTurboQuantValue, "turboquant_value", 0, 32, 0, PO::kLeastSignificantBitStream,
     SM::kTurboQuantK32, SE::kFP16, ZP::kNone, 32, false, false, false, true, true},
};

const CanonicalQuantDescriptor* lookup(L layout) {
  for (const auto& d : kTable)
    if (d.layout == layout) return &d;
  return nullptr;
}

bool product_fits(long long a, long long b, std::size_t* out = nullptr) {
  if (a <= 0 || b <= 0) return false;
  const auto ua = static_cast<unsigned long long>(a), ub = static_cast<unsigned long long>(b);
  if (ua > std::numeric_limits<std::size_t>::max() / ub) return false;
  if (out != nullptr) *out = static_cast<std::size_t>(ua * ub);
  return true;
}

bool all_finite(const float* v, std::size_t n) {
  if (n != 0 && v == nullptr) return false;
  for (std::size_t i = 0; i < n; ++i)
    if (!std::isfinite(v[i])) return false;
  return true;
}

bool all_finite_nonnegative(const float* v, std::size_t n) {
  if (!all_finite(v, n)) return false;
  for (std::size_t i = 0; i < n; ++i)
    if (v[i] < 0.0f) return false;
  return true;
}

bool is_permutation(const std::vector<int>& order, std::size_t n) {
  if (order.empty()) return true;
  if (order.size() != n) return false;
  std::vector<bool> seen(n, false);
  for (int v : order) {
    if (v < 0 || static_cast<std::size_t>(v) >= n || seen[static_cast<std::size_t>(v)])
      return false;
    seen[static_cast<std::size_t>(v)] = true;
  }
  return true;
}

// Canonical data bytes of a layout (quant_import_ref.cpp:91-128).
Status data_bytes(const QuantTensorMetadata& md, std::size_t* bytes) {
  std::size_t elements = 0;
  if (!product_fits(md.logical_rows, md.logical_columns, &elements)) return Status::kInvalidShape;
  auto times = [&](std::size_t per_block) {
    const std::size_t blocks = elements / 32;
    if (blocks != 0 && per_block > std::numeric_limits<std::size_t>::max() / blocks)
      return Status::kInvalidShape;
    *bytes = blocks * per_block;
    return Status::kOk;
  };
  switch (md.layout) {
    case L::kInt4Symmetric:
    case L::kUInt4Affine:
    case L::kFP4E2M1:
      if (md.logical_columns % 2 != 0) return Status::kInvalidShape;
      *bytes = elements / 2;
      return Status::kOk;
    case L::kInt8Symmetric:
    case L::kInt8Affine:
    case L::kFP8E4M3FN:
    case L::kFP8E5M2:
      *bytes = elements;
      return Status::kOk;
    case L::kMXFP8E4M3E8M0: return times(33);
    case L::kMXFP4E2M1E8M0: return times(17);
    case L::kNVFP4E2M1E4M3:
      *bytes = elements / 2;
      return Status::kOk;
    case L::kBitNetTernary: return times(10);
    case L::kTurboQuantKey:
    case L::kTurboQuantValue: return Status::kUnsupportedFormat;
  }
  return Status::kUnsupportedFormat;
}

// IEEE half -> float (finite check of BitNet block scales).
float half_to_float(std::uint16_t h) {
  const int exp = (h >> 10) & 31, man = h & 1023;
  const float sign = (h & 0x8000) ? -1.0f : 1.0f;
  if (exp == 31) return man ? std::numeric_limits<float>::quiet_NaN()
                            : sign * std::numeric_limits<float>::infinity();
  if (exp == 0) return sign * std::ldexp(static_cast<float>(man), -24);
  return sign * std::ldexp(static_cast<float>(1024 + man), exp - 25);
}

// The scale modes / encodings a layout's tensor may carry
// (quant_import_ref.cpp:404-459).
bool scales_allowed(const QuantTensorMetadata& md) {
  const SM m = md.scale_mode;
  const SE e = md.scale_encoding;
  const bool row_like = m == SM::kRow || m == SM::kChannel || m == SM::kGroup;
  switch (md.layout) {
    case L::kInt4Symmetric:
    case L::kUInt4Affine:
    case L::kInt8Symmetric:
    case L::kInt8Affine: return row_like && e == SE::kFP32;
    case L::kFP8E4M3FN:
    case L::kFP8E5M2:
      return m == SM::kNone || (e == SE::kFP32 && (m == SM::kTensor || row_like ||
                                                   m == SM::kBlock));
    case L::kFP4E2M1:
      return (e == SE::kFP16 || e == SE::kFP32) && (m == SM::kTensor || row_like ||
                                                    m == SM::kBlock);
    case L::kMXFP8E4M3E8M0:
    case L::kMXFP4E2M1E8M0: return m == SM::kMicroscaleK32 && e == SE::kE8M0;
    case L::kNVFP4E2M1E4M3: return m == SM::kNVFP4K16 && e == SE::kE4M3FN;
    case L::kBitNetTernary: return m == SM::kBlock && e == SE::kFP16;
    case L::kTurboQuantKey:
    case L::kTurboQuantValue: return true;
  }
  return true;
}

}  // namespace

Status canonical_quant_descriptor(CanonicalQuantLayout layout,
                                  CanonicalQuantDescriptor* descriptor) {
  if (descriptor == nullptr) return Status::kInvalidArgument;
  const CanonicalQuantDescriptor* d = lookup(layout);
  if (d == nullptr) return Status::kUnsupportedFormat;
  *descriptor = *d;
  return Status::kOk;
}

const char* canonical_quant_layout_name(CanonicalQuantLayout layout) {
  const CanonicalQuantDescriptor* d = lookup(layout);
  return d == nullptr ? "unknown" : d->name;
}

Status validate_quant_metadata(const QuantTensorMetadata& md) {
  const CanonicalQuantDescriptor* d = lookup(md.layout);
  if (d == nullptr) return Status::kUnsupportedFormat;
  if (md.contract_version != d->contract_version ||
      !product_fits(md.logical_rows, md.logical_columns))
    return Status::kInvalidShape;
  if (!std::isfinite(md.global_scale) || md.global_scale < 0.0f || md.scale_domain_rows <= 0)
    return Status::kInvalidArgument;
  const long long cols = md.logical_columns;
  if (d->block_elements != 0 && cols % d->block_elements != 0) return Status::kInvalidShape;
  if (md.group_size < 0 || (md.group_size > 0 && cols % md.group_size != 0))
    return Status::kInvalidShape;
  if (md.act_order_count != 0 && md.act_order_count != static_cast<std::size_t>(cols))
    return Status::kInvalidShape;
  if (md.group_index_count != 0 && md.group_index_count != static_cast<std::size_t>(cols))
    return Status::kInvalidShape;
  if (md.group_index_count != 0 && md.layout != L::kInt4Symmetric &&
      md.layout != L::kUInt4Affine)
    return Status::kInvalidArgument;
  if (md.act_order_count != 0 && !d->supports_act_order) return Status::kInvalidArgument;
  if (md.sparse_mask_bytes != 0 && md.sparse_mask_bytes < static_cast<std::size_t>((cols + 7) / 8))
    return Status::kInvalidShape;
  if (md.sparse_mask_bytes != 0 && !d->supports_sparse_mask) return Status::kInvalidArgument;
  if (d->requires_centroid_table) {
    if (md.value_bits < 2 || md.value_bits > 8 ||
        md.centroid_count != (std::size_t{1} << static_cast<unsigned>(md.value_bits)))
      return Status::kInvalidShape;
  } else if (md.centroid_count != 0) {
    return Status::kInvalidArgument;
  }
  if (d->is_cache_layout) {
    const int bits = md.layout == L::kTurboQuantKey ? md.key_bits : md.value_bits;
    if (bits < 2 || bits > 8 || (cols != 64 && cols != 128 && cols != 256))
      return Status::kInvalidShape;
  }
  if (md.scale_2d && (md.layout != L::kNVFP4E2M1E4M3 || md.scale_domain_rows > 16))
    return Status::kInvalidArgument;
  if (d->has_global_scale && md.scale_mode != SM::kNVFP4K16) return Status::kInvalidArgument;
  const auto rows = static_cast<std::size_t>(md.logical_rows);
  const auto ucols = static_cast<std::size_t>(cols);
  std::size_t scales = 0;
  switch (md.scale_mode) {
    case SM::kNone: break;
    case SM::kTensor: scales = 1; break;
    case SM::kRow:
    case SM::kChannel: scales = rows; break;
    case SM::kGroup:
      if (md.group_size <= 0) return Status::kInvalidShape;
      scales = rows * (ucols / static_cast<std::size_t>(md.group_size));
      break;
    case SM::kBlock:
      if (md.scale_count == 0) return Status::kInvalidShape;
      scales = md.scale_count;
      break;
    case SM::kMicroscaleK32:
    case SM::kTurboQuantK32: scales = rows * (ucols / 32); break;
    case SM::kNVFP4K16: scales = rows * (ucols / 16); break;
  }
  if (md.scale_count != scales) return Status::kInvalidShape;
  if ((md.scale_mode == SM::kNone) != (md.scale_encoding == SE::kNone))
    return Status::kInvalidArgument;
  if (md.zero_point_count != (md.zero_point_mode == ZP::kNone ? 0 : scales))
    return Status::kInvalidShape;
  return Status::kOk;
}

Status validate_canonical_quant_tensor(const CanonicalQuantTensor& t) {
  Status st = validate_quant_metadata(t.metadata);
  if (st != Status::kOk) return st;
  const QuantTensorMetadata& md = t.metadata;
  if (!scales_allowed(md)) return Status::kInvalidArgument;
  std::size_t bytes = 0;
  st = data_bytes(md, &bytes);
  if (st != Status::kOk) return st;
  if (t.data.size() != bytes) return Status::kInvalidShape;
  const bool embedded = md.layout == L::kMXFP8E4M3E8M0 || md.layout == L::kMXFP4E2M1E8M0 ||
                        md.layout == L::kBitNetTernary;
  const bool split = md.layout == L::kNVFP4E2M1E4M3;
  if (embedded) {
    if (!t.scales.empty() || !t.scale_codes.empty()) return Status::kInvalidShape;
  } else if (split) {
    if (!t.scales.empty() || t.scale_codes.size() != md.scale_count) return Status::kInvalidShape;
  } else if (t.scales.size() != md.scale_count || !t.scale_codes.empty()) {
    return Status::kInvalidShape;
  }
  if (t.zero_points.size() != md.zero_point_count ||
      t.group_index.size() != md.group_index_count || t.act_order.size() != md.act_order_count ||
      !all_finite_nonnegative(t.scales.data(), t.scales.size()) ||
      !all_finite(t.zero_points.data(), t.zero_points.size()) ||
      !all_finite(t.activation_scales.data(), t.activation_scales.size()))
    return Status::kInvalidShape;
  if (!is_permutation(t.act_order, static_cast<std::size_t>(md.logical_columns)))
    return Status::kInvalidArgument;
  if (!t.group_index.empty()) {
    const std::size_t groups = md.scale_count / static_cast<std::size_t>(md.logical_rows);
    for (int g : t.group_index)
      if (g < 0 || static_cast<std::size_t>(g) >= groups) return Status::kInvalidArgument;
  }
  if (!t.activation_zero_points.empty() &&
      t.activation_zero_points.size() != t.activation_scales.size())
    return Status::kInvalidShape;
  if (!t.row_sums.empty() && t.row_sums.size() != static_cast<std::size_t>(md.logical_rows))
    return Status::kInvalidShape;
  // Reserved encodings: an E8M0 scale byte of 0xff (MX blocks), an E4M3
  // scale code above 0x7e (NVFP4), a non-finite or negative fp16 scale or
  // the reserved ternary code 3 (BitNet blocks).
  if (md.layout == L::kMXFP8E4M3E8M0 || md.layout == L::kMXFP4E2M1E8M0) {
    const std::size_t stride = md.layout == L::kMXFP8E4M3E8M0 ? 33 : 17;
    for (std::size_t b = 0; b < t.data.size(); b += stride)
      if (t.data[b] == 0xff) return Status::kInvalidArgument;
  }
  if (md.layout == L::kNVFP4E2M1E4M3)
    for (std::uint8_t c : t.scale_codes)
      if (c > 0x7e) return Status::kInvalidArgument;
  if (md.layout == L::kBitNetTernary) {
    for (std::size_t b = 0; b < t.data.size(); b += 10) {
      const float s = half_to_float(static_cast<std::uint16_t>(t.data[b] | (t.data[b + 1] << 8)));
      if (!std::isfinite(s) || s < 0.0f) return Status::kInvalidArgument;
      for (std::size_t i = 2; i < 10; ++i)
        for (int lane = 0; lane < 4; ++lane)
          if (((t.data[b + i] >> (2 * lane)) & 3u) == 3u) return Status::kInvalidArgument;
    }
  }
  return Status::kOk;
}

// kernels/quantization/quant_import_ref.cpp:1051-1116: argument checks
// (kInvalidArgument), counts and finiteness (kInvalidShape), then the
// kInt8Symmetric / channel-scale tensor with row sums computed in int32
// element order when not supplied.
Status import_smoothquant_w8a8(const SmoothQuantW8A8Source& s, CanonicalQuantTensor* tensor) {
  std::size_t elements = 0;
  if (tensor == nullptr || s.weights == nullptr || s.weight_scales == nullptr ||
      s.activation_scales == nullptr || !product_fits(s.rows, s.columns, &elements))
    return Status::kInvalidArgument;
  const auto rows = static_cast<std::size_t>(s.rows);
  if (s.weight_count != elements || s.weight_scale_count != rows ||
      s.activation_scale_count == 0 ||
      (s.activation_zero_point_count != 0 &&
       (s.activation_zero_points == nullptr ||
        s.activation_zero_point_count != s.activation_scale_count)) ||
      (s.row_sum_count != 0 && (s.row_sums == nullptr || s.row_sum_count != rows)) ||
      !all_finite(s.weight_scales, s.weight_scale_count) ||
      !all_finite(s.activation_scales, s.activation_scale_count))
    return Status::kInvalidShape;
  try {
    CanonicalQuantTensor t;
    t.metadata.layout = L::kInt8Symmetric;
    t.metadata.logical_rows = s.rows;
    t.metadata.logical_columns = s.columns;
    t.metadata.group_size = s.columns;
    t.provenance = QuantImportProvenance::kSmoothQuant;
    const auto* w = reinterpret_cast<const std::uint8_t*>(s.weights);
    t.data.assign(w, w + elements);
    t.scales.assign(s.weight_scales, s.weight_scales + rows);
    t.activation_scales.assign(s.activation_scales, s.activation_scales + s.activation_scale_count);
    if (s.activation_zero_point_count != 0)
      t.activation_zero_points.assign(s.activation_zero_points,
                                      s.activation_zero_points + s.activation_zero_point_count);
    t.row_sums.resize(rows);
    for (std::size_t r = 0; r < rows; ++r) {
      if (s.row_sum_count != 0) {
        t.row_sums[r] = s.row_sums[r];
        continue;
      }
      std::int32_t sum = 0;
      const std::int8_t* row = s.weights + r * static_cast<std::size_t>(s.columns);
      for (long long c = 0; c < s.columns; ++c) sum += row[c];
      t.row_sums[r] = sum;
    }
    t.metadata.scale_mode = SM::kChannel;
    t.metadata.scale_encoding = SE::kFP32;
    t.metadata.scale_count = t.scales.size();
    const Status st = validate_canonical_quant_tensor(t);
    if (st != Status::kOk) return st;
    *tensor = std::move(t);
    return Status::kOk;
  } catch (const std::bad_alloc&) {
    return Status::kOutOfMemory;
  } catch (const std::length_error&) {
    return Status::kOutOfMemory;
  }
}

const char* quant_import_provenance_name(QuantImportProvenance p) {
  switch (p) {
    case QuantImportProvenance::kCanonical: return "canonical";
    case QuantImportProvenance::kAWQ: return "awq";
    case QuantImportProvenance::kGPTQ: return "gptq";
    case QuantImportProvenance::kAutoRound: return "autoround";
    case QuantImportProvenance::kSmoothQuant: return "smoothquant";
    case QuantImportProvenance::kBitNet: return "bitnet";
  }
  return "unknown";
}

}  // namespace quixicore_cpu
