// Prepared storage projections (include/quixicore_cpu/qgemm.h:32-101 of the
// reference) over canonical int8 weights on the GPU.
//
// Validation follows kernels/quantization/qgemm_canonical.cpp in order:
// activation (for the epilogue form), each prepared weight
// (validate_prepared_projection, :4275-4291: readiness -> kInvalidArgument,
// no canonical layout -> kUnsupportedFormat, geometry -> kInvalidShape),
// compatibility and counts -> kInvalidShape, storage types ->
// kUnsupportedFormat, pointers -> kInvalidArgument.  Only then does this
// route require an int8 canonical layout without a group index or act-order
// table (others: kUnsupportedFormat).  The work is one qc_hip_cint8_project
// launch; host buffers are staged like every drop-in call.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <initializer_list>
#include <vector>

#include "qc_dropin.h"
#include "quixicore_cpu/qgemm.h"
#include "quixicore_cpu/quant_import.h"
#include "quixicore_hip.h"

namespace quixicore_cpu {
namespace {

constexpr std::size_t kMissing = static_cast<std::size_t>(-1);
constexpr long long kMaximumRowTile = 16;

bool valid_product(std::initializer_list<long long> dims) {
  long long product = 1;
  for (const long long d : dims) {
    if (d <= 0 || product > LLONG_MAX / d) return false;
    product *= d;
  }
  return true;
}

bool known(FloatStorageType t) {
  return t == FloatStorageType::kF32 || t == FloatStorageType::kF16 ||
         t == FloatStorageType::kBF16;
}

std::size_t width(FloatStorageType t) { return t == FloatStorageType::kF32 ? 4 : 2; }

bool known_activation(LinearActivation a) {
  return a == LinearActivation::kNone || a == LinearActivation::kGeluErf ||
         a == LinearActivation::kGeluTanh || a == LinearActivation::kSilu ||
         a == LinearActivation::kRelu2;
}

// kernels/quantization/qgemm_canonical.cpp:4275-4291.
Status validate_prepared(const CpuPackedWeights& w, CpuPackedWeightsInfo* info) {
  if (!w.ready()) return Status::kInvalidArgument;
  *info = w.info();
  const CanonicalQuantLayout l = info->quant_metadata.layout;
  if (!info->has_canonical_layout || l == CanonicalQuantLayout::kTurboQuantKey ||
      l == CanonicalQuantLayout::kTurboQuantValue)
    return Status::kUnsupportedFormat;
  if (!valid_product({info->rows, info->columns}) || info->row_tile <= 0 ||
      info->row_tile > kMaximumRowTile || info->block_size <= 0 || info->blocks_per_row <= 0 ||
      info->columns / info->block_size != info->blocks_per_row || w.panel_data() == nullptr)
    return Status::kInvalidShape;
  return Status::kOk;
}

// qgemm_canonical.cpp:4293-4300 (compatible_gate_up) and :4302-4309
// (compatible_qkv_plane).
bool compatible_gate_up(const CpuPackedWeightsInfo& a, const CpuPackedWeightsInfo& b) {
  return a.quant_metadata.layout == b.quant_metadata.layout && a.rows == b.rows &&
         a.columns == b.columns && a.row_tile == b.row_tile && a.block_size == b.block_size &&
         a.blocks_per_row == b.blocks_per_row && a.block_bytes == b.block_bytes;
}
bool compatible_plane(const CpuPackedWeightsInfo& q, const CpuPackedWeightsInfo& o) {
  return q.quant_metadata.layout == o.quant_metadata.layout && q.columns == o.columns &&
         q.row_tile == o.row_tile && q.block_size == o.block_size &&
         q.blocks_per_row == o.blocks_per_row && q.block_bytes == o.block_bytes;
}

// The device view of an int8 canonical tensor, or kUnsupportedFormat for a
// layout this route does not compute.
Status device_weights(const CpuPackedWeights& w, const CpuPackedWeightsInfo& info,
                      qc_cint8_weights* out) {
  const QuantTensorMetadata& md = info.quant_metadata;
  const bool int8 = md.layout == CanonicalQuantLayout::kInt8Symmetric ||
                    md.layout == CanonicalQuantLayout::kInt8Affine;
  const bool row_like = md.scale_mode == QuantScaleMode::kRow ||
                        md.scale_mode == QuantScaleMode::kChannel ||
                        md.scale_mode == QuantScaleMode::kGroup;
  if (!int8 || !row_like || info.group_index_offset != kMissing ||
      info.act_order_offset != kMissing || w.device_data() == nullptr ||
      w.device_scales() == nullptr ||
      (md.layout == CanonicalQuantLayout::kInt8Affine && w.device_zero_points() == nullptr))
    return Status::kUnsupportedFormat;
  long long groups = 1;
  if (md.scale_mode == QuantScaleMode::kGroup) {
    groups = static_cast<long long>(md.scale_count) / info.rows;
    if (groups < 1 || info.columns % groups != 0) return Status::kUnsupportedFormat;
  }
  out->codes = static_cast<const int8_t*>(w.device_data());
  out->scales = w.device_scales();
  out->zero_points =
      md.layout == CanonicalQuantLayout::kInt8Affine ? w.device_zero_points() : nullptr;
  out->rows = info.rows;
  out->cols = info.columns;
  out->groups = groups;
  return Status::kOk;
}

int type_id(FloatStorageType t) { return static_cast<int>(t); }

}  // namespace

// qgemm_canonical.cpp:4461-4629 (qgemm_prepacked_storage_impl).
static Status storage_impl(const CpuPackedWeights& weights, FloatStorageInput x,
                           FloatStorageOutput y, long long m, const float* bias,
                           LinearActivation activation, Workspace* workspace) {
  if (!known_activation(activation)) return Status::kInvalidArgument;
  CpuPackedWeightsInfo info;
  Status st = validate_prepared(weights, &info);
  if (st != Status::kOk) return st;
  if (!valid_product({m, info.columns}) || !valid_product({m, info.rows}) ||
      x.count != m * info.columns || y.count != m * info.rows)
    return Status::kInvalidShape;
  if (!known(x.type) || !known(y.type)) return Status::kUnsupportedFormat;
  if (x.data == nullptr || y.data == nullptr) return Status::kInvalidArgument;
  qc_cint8_weights w{};
  if ((st = device_weights(weights, info, &w)) != Status::kOk) return st;
  detail::WorkspaceFrame frame(workspace);
  detail::Staging g(workspace);
  const void* xd = g.in(x.data, width(x.type) * x.count);
  void* yd = g.out(y.data, width(y.type) * y.count);
  const float* bd =
      bias == nullptr ? nullptr : static_cast<const float*>(g.in(bias, sizeof(float) * info.rows));
  if (g.status() != Status::kOk) return g.status();
  void* ys[1] = {yd};
  const int yt[1] = {type_id(y.type)};
  return g.finish(qc_hip_cint8_project(0, &w, 1, xd, type_id(x.type), m, ys, yt, bd,
                                       static_cast<int>(activation), nullptr, nullptr, 0,
                                       g.stream()));
}

Status qgemm_prepacked_storage(const CpuPackedWeights& weights, FloatStorageInput x,
                               FloatStorageOutput y, long long m, Workspace* workspace) {
  return storage_impl(weights, x, y, m, nullptr, LinearActivation::kNone, workspace);
}

Status qgemm_prepacked_epilogue_storage(const CpuPackedWeights& weights, FloatStorageInput x,
                                        const float* bias, FloatStorageOutput y, long long m,
                                        LinearActivation activation, Workspace* workspace) {
  return storage_impl(weights, x, y, m, bias, activation, workspace);
}

Status qgemv_prepacked_storage(const CpuPackedWeights& weights, FloatStorageInput x,
                               FloatStorageOutput y, Workspace* workspace) {
  return qgemm_prepacked_storage(weights, x, y, 1, workspace);
}

// qgemm_canonical.cpp:4661-4768 (qgemm_prepacked_gate_up_impl).
static Status gate_up_impl(const CpuPackedWeights& gate_weights,
                           const CpuPackedWeights& up_weights, FloatStorageInput x,
                           FloatStorageOutput gate_output, FloatStorageOutput up_output,
                           FloatStorageOutput fused, long long m, bool swiglu,
                           Workspace* workspace) {
  CpuPackedWeightsInfo gi, ui;
  Status st = validate_prepared(gate_weights, &gi);
  if (st != Status::kOk) return st;
  if ((st = validate_prepared(up_weights, &ui)) != Status::kOk) return st;
  if (!compatible_gate_up(gi, ui) || !valid_product({m, gi.columns}) ||
      !valid_product({m, gi.rows}) || x.count != m * gi.columns ||
      (swiglu ? fused.count != m * gi.rows
              : (gate_output.count != m * gi.rows || up_output.count != m * gi.rows)))
    return Status::kInvalidShape;
  if (!known(x.type) ||
      (swiglu ? !known(fused.type) : (!known(gate_output.type) || !known(up_output.type))))
    return Status::kUnsupportedFormat;
  if (x.data == nullptr ||
      (swiglu ? fused.data == nullptr : (gate_output.data == nullptr || up_output.data == nullptr)))
    return Status::kInvalidArgument;
  qc_cint8_weights w[2] = {};
  if ((st = device_weights(gate_weights, gi, &w[0])) != Status::kOk) return st;
  if ((st = device_weights(up_weights, ui, &w[1])) != Status::kOk) return st;
  if (w[0].groups != w[1].groups) return Status::kUnsupportedFormat;
  detail::WorkspaceFrame frame(workspace);
  detail::Staging g(workspace);
  const void* xd = g.in(x.data, width(x.type) * x.count);
  void* ys[2] = {nullptr, nullptr};
  int yt[2] = {0, 0};
  if (swiglu) {
    ys[0] = g.out(fused.data, width(fused.type) * fused.count);
    yt[0] = type_id(fused.type);
  } else {
    ys[0] = g.out(gate_output.data, width(gate_output.type) * gate_output.count);
    ys[1] = g.out(up_output.data, width(up_output.type) * up_output.count);
    yt[0] = type_id(gate_output.type);
    yt[1] = type_id(up_output.type);
  }
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_cint8_project(swiglu ? 1 : 0, w, 2, xd, type_id(x.type), m, ys, yt,
                                       nullptr, 0, nullptr, nullptr, 0, g.stream()));
}

Status qgemm_prepacked_gate_up_storage(const CpuPackedWeights& gate_weights,
                                       const CpuPackedWeights& up_weights, FloatStorageInput x,
                                       FloatStorageOutput gate_output,
                                       FloatStorageOutput up_output, long long m,
                                       Workspace* workspace) {
  return gate_up_impl(gate_weights, up_weights, x, gate_output, up_output, {}, m, false,
                      workspace);
}

Status qgemv_prepacked_gate_up_storage(const CpuPackedWeights& gate_weights,
                                       const CpuPackedWeights& up_weights, FloatStorageInput x,
                                       FloatStorageOutput gate_output,
                                       FloatStorageOutput up_output, Workspace* workspace) {
  return qgemm_prepacked_gate_up_storage(gate_weights, up_weights, x, gate_output, up_output, 1,
                                         workspace);
}

Status qgemm_prepacked_swiglu_storage(const CpuPackedWeights& gate_weights,
                                      const CpuPackedWeights& up_weights, FloatStorageInput x,
                                      FloatStorageOutput output, long long m,
                                      Workspace* workspace) {
  return gate_up_impl(gate_weights, up_weights, x, {}, {}, output, m, true, workspace);
}

Status qgemv_prepacked_swiglu_storage(const CpuPackedWeights& gate_weights,
                                      const CpuPackedWeights& up_weights, FloatStorageInput x,
                                      FloatStorageOutput output, Workspace* workspace) {
  return qgemm_prepacked_swiglu_storage(gate_weights, up_weights, x, output, 1, workspace);
}

// qgemm_canonical.cpp:4790-4820 (qgemm_prepacked_qkv_storage validation).
Status qgemm_prepacked_qkv_storage(const CpuPackedWeights& q_weights,
                                   const CpuPackedWeights& k_weights,
                                   const CpuPackedWeights& v_weights, FloatStorageInput x,
                                   FloatStorageOutput q_output, FloatStorageOutput k_output,
                                   FloatStorageOutput v_output, long long m,
                                   Workspace* workspace) {
  CpuPackedWeightsInfo qi, ki, vi;
  Status st = validate_prepared(q_weights, &qi);
  if (st != Status::kOk) return st;
  if ((st = validate_prepared(k_weights, &ki)) != Status::kOk) return st;
  if ((st = validate_prepared(v_weights, &vi)) != Status::kOk) return st;
  if (!compatible_plane(qi, ki) || !compatible_plane(qi, vi) || !valid_product({m, qi.columns}) ||
      !valid_product({m, qi.rows}) || !valid_product({m, ki.rows}) ||
      !valid_product({m, vi.rows}) || x.count != m * qi.columns ||
      q_output.count != m * qi.rows || k_output.count != m * ki.rows ||
      v_output.count != m * vi.rows)
    return Status::kInvalidShape;
  if (!known(x.type) || !known(q_output.type) || !known(k_output.type) || !known(v_output.type))
    return Status::kUnsupportedFormat;
  if (x.data == nullptr || q_output.data == nullptr || k_output.data == nullptr ||
      v_output.data == nullptr)
    return Status::kInvalidArgument;
  qc_cint8_weights w[3] = {};
  const CpuPackedWeights* pw[3] = {&q_weights, &k_weights, &v_weights};
  const CpuPackedWeightsInfo* pi[3] = {&qi, &ki, &vi};
  for (int i = 0; i < 3; ++i)
    if ((st = device_weights(*pw[i], *pi[i], &w[i])) != Status::kOk) return st;
  if (w[1].groups != w[0].groups || w[2].groups != w[0].groups) return Status::kUnsupportedFormat;
  detail::WorkspaceFrame frame(workspace);
  detail::Staging g(workspace);
  const void* xd = g.in(x.data, width(x.type) * x.count);
  FloatStorageOutput* outs[3] = {&q_output, &k_output, &v_output};
  void* ys[3];
  int yt[3];
  for (int i = 0; i < 3; ++i) {
    ys[i] = g.out(outs[i]->data, width(outs[i]->type) * outs[i]->count);
    yt[i] = type_id(outs[i]->type);
  }
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_cint8_project(0, w, 3, xd, type_id(x.type), m, ys, yt, nullptr, 0,
                                       nullptr, nullptr, 0, g.stream()));
}

Status qgemv_prepacked_qkv_storage(const CpuPackedWeights& q_weights,
                                   const CpuPackedWeights& k_weights,
                                   const CpuPackedWeights& v_weights, FloatStorageInput x,
                                   FloatStorageOutput q_output, FloatStorageOutput k_output,
                                   FloatStorageOutput v_output, Workspace* workspace) {
  return qgemm_prepacked_qkv_storage(q_weights, k_weights, v_weights, x, q_output, k_output,
                                     v_output, 1, workspace);
}

// qgemm_canonical.cpp:5032-5225.  Only the position's cos / sin rows and the
// slot's cache rows are staged; slot -1 leaves the caches untouched.
Status qgemv_prepacked_qkv_rope_kv_storage(
    const CpuPackedWeights& q_weights, const CpuPackedWeights& k_weights,
    const CpuPackedWeights& v_weights, FloatStorageInput x, const float* cosine,
    const float* sine, FloatStorageOutput q_output, FloatStorageOutput key_cache,
    FloatStorageOutput value_cache, long long query_heads, long long kv_heads,
    long long head_dim, long long slots, long long max_position, int position, int slot,
    Workspace* workspace) {
  CpuPackedWeightsInfo qi, ki, vi;
  Status st = validate_prepared(q_weights, &qi);
  if (st != Status::kOk) return st;
  if ((st = validate_prepared(k_weights, &ki)) != Status::kOk) return st;
  if ((st = validate_prepared(v_weights, &vi)) != Status::kOk) return st;
  if (!compatible_plane(qi, ki) || !compatible_plane(qi, vi) || head_dim % 2 != 0 ||
      !valid_product({query_heads, head_dim}) || !valid_product({kv_heads, head_dim}) ||
      !valid_product({slots, kv_heads, head_dim}) || !valid_product({max_position, head_dim / 2}) ||
      position < 0 || position >= max_position || slot < -1 || slot >= slots)
    return Status::kInvalidShape;
  const long long query_dim = query_heads * head_dim;
  const long long kv_dim = kv_heads * head_dim;
  const long long half = head_dim / 2;
  const long long cache_count = slots * kv_dim;
  if (qi.rows != query_dim || ki.rows != kv_dim || vi.rows != kv_dim || x.count != qi.columns ||
      q_output.count != query_dim || key_cache.count != cache_count ||
      value_cache.count != cache_count)
    return Status::kInvalidShape;
  if (!known(x.type) || !known(q_output.type) || !known(key_cache.type) ||
      !known(value_cache.type))
    return Status::kUnsupportedFormat;
  if (x.data == nullptr || cosine == nullptr || sine == nullptr || q_output.data == nullptr ||
      key_cache.data == nullptr || value_cache.data == nullptr)
    return Status::kInvalidArgument;
  const long long query_pairs = query_heads * half;
  const long long key_pairs = slot >= 0 ? kv_heads * half : 0;
  const long long value_rows = slot >= 0 ? kv_dim : 0;
  if (query_pairs > LLONG_MAX - key_pairs || query_pairs + key_pairs > LLONG_MAX - value_rows)
    return Status::kInvalidShape;
  qc_cint8_weights w[3] = {};
  const CpuPackedWeights* pw[3] = {&q_weights, &k_weights, &v_weights};
  const CpuPackedWeightsInfo* pi[3] = {&qi, &ki, &vi};
  const int nw = slot >= 0 ? 3 : 1;
  for (int i = 0; i < nw; ++i)
    if ((st = device_weights(*pw[i], *pi[i], &w[i])) != Status::kOk) return st;
  for (int i = 1; i < nw; ++i)
    if (w[i].groups != w[0].groups) return Status::kUnsupportedFormat;
  detail::WorkspaceFrame frame(workspace);
  detail::Staging g(workspace);
  const void* xd = g.in(x.data, width(x.type) * x.count);
  const float* cd = static_cast<const float*>(g.in(cosine + position * half, sizeof(float) * half));
  const float* sd = static_cast<const float*>(g.in(sine + position * half, sizeof(float) * half));
  void* ys[3] = {g.out(q_output.data, width(q_output.type) * query_dim), nullptr, nullptr};
  int yt[3] = {type_id(q_output.type), type_id(key_cache.type), type_id(value_cache.type)};
  if (slot >= 0) {
    auto* kb = static_cast<char*>(key_cache.data) + width(key_cache.type) * slot * kv_dim;
    auto* vb = static_cast<char*>(value_cache.data) + width(value_cache.type) * slot * kv_dim;
    ys[1] = g.out(kb, width(key_cache.type) * kv_dim);
    ys[2] = g.out(vb, width(value_cache.type) * kv_dim);
  }
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_cint8_project(2, w, nw, xd, type_id(x.type), 1, ys, yt, nullptr, 0, cd,
                                       sd, head_dim, g.stream()));
}

// qgemm_canonical.cpp:5415-5433 (qgemm_prepacked_quantized): the prepared
// weights, the activation tensor, its layout, then K and the output.  This
// route then computes int8 weights against int8 activations with row,
// channel or group scales (others: kUnsupportedFormat).  Integer activation
// zero points are passed as ints too, which lets symmetric row-scaled
// weights take the int8 MFMA GEMM (qc_hip_cint8_quantized_gemm).
Status qgemm_prepacked_quantized(const CpuPackedWeights& weights,
                                 const CanonicalQuantTensor& activation, float* y,
                                 Workspace* workspace) {
  CpuPackedWeightsInfo info;
  Status st = validate_prepared(weights, &info);
  if (st != Status::kOk) return st;
  st = validate_canonical_quant_tensor(activation);
  if (st != Status::kOk) return st;
  const QuantTensorMetadata& am = activation.metadata;
  if (am.layout == CanonicalQuantLayout::kTurboQuantKey ||
      am.layout == CanonicalQuantLayout::kTurboQuantValue)
    return Status::kUnsupportedFormat;
  const long long m = am.logical_rows;
  if (am.logical_columns != info.columns) return Status::kInvalidShape;
  if (!valid_product({m, info.rows}) || y == nullptr) return Status::kInvalidArgument;
  qc_cint8_weights w{};
  if ((st = device_weights(weights, info, &w)) != Status::kOk) return st;
  const bool int8 = am.layout == CanonicalQuantLayout::kInt8Symmetric ||
                    am.layout == CanonicalQuantLayout::kInt8Affine;
  const bool row_like = am.scale_mode == QuantScaleMode::kRow ||
                        am.scale_mode == QuantScaleMode::kChannel ||
                        am.scale_mode == QuantScaleMode::kGroup;
  if (!int8 || !row_like || !activation.group_index.empty() || !activation.act_order.empty())
    return Status::kUnsupportedFormat;
  long long agroups = 1;
  if (am.scale_mode == QuantScaleMode::kGroup) {
    agroups = static_cast<long long>(am.scale_count) / m;
    if (agroups < 1 || am.logical_columns % agroups != 0) return Status::kUnsupportedFormat;
  }
  const std::size_t elements = static_cast<std::size_t>(m) * static_cast<std::size_t>(info.columns);
  // zero points that are all integers in int range also go as ints
  std::vector<int> int_zeros;
  const bool affine = am.layout == CanonicalQuantLayout::kInt8Affine;
  if (affine && agroups == 1) {
    int_zeros.reserve(activation.zero_points.size());
    for (const float z : activation.zero_points) {
      if (!(z >= -2147483648.0f && z < 2147483648.0f) || z != std::nearbyint(z)) {
        int_zeros.clear();
        break;
      }
      int_zeros.push_back(static_cast<int>(z));
    }
  }
  detail::WorkspaceFrame frame(workspace);
  detail::Staging g(workspace);
  qc_cint8_weights a{};
  a.codes = static_cast<const int8_t*>(g.in(activation.data.data(), elements));
  a.scales = static_cast<const float*>(
      g.in(activation.scales.data(), activation.scales.size() * sizeof(float)));
  a.zero_points = affine ? static_cast<const float*>(g.in(
                               activation.zero_points.data(),
                               activation.zero_points.size() * sizeof(float)))
                         : nullptr;
  a.rows = m;
  a.cols = info.columns;
  a.groups = agroups;
  const int* zi = int_zeros.empty()
                      ? nullptr
                      : static_cast<const int*>(g.in(int_zeros.data(), int_zeros.size() * sizeof(int)));
  float* yd = static_cast<float*>(
      g.out(y, sizeof(float) * static_cast<std::size_t>(m) * static_cast<std::size_t>(info.rows)));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_cint8_quantized_gemm(&w, &a, zi, yd, g.stream()));
}

// qgemm_canonical.cpp:5502-5507.
Status qgemv_prepacked_quantized(const CpuPackedWeights& weights,
                                 const CanonicalQuantTensor& activation, float* y,
                                 Workspace* workspace) {
  if (activation.metadata.logical_rows != 1) return Status::kInvalidShape;
  return qgemm_prepacked_quantized(weights, activation, y, workspace);
}

}  // namespace quixicore_cpu
