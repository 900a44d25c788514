// CpuPackedWeights (device mirror + the reference's host panel), the device
// Workspace arena, and the prepared-weight entry points qgemm_prepacked /
// qgemv_prepacked.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <new>
#include <vector>

#include "qc_dropin.h"
#include "quixicore_cpu/packed_weights.h"
#include "quixicore_cpu/qgemm.h"
#include "quixicore_cpu/quant_import.h"
#include "quixicore_hip.h"

namespace quixicore_cpu {

// ------------------------------------------------------------ Workspace ---

struct Workspace::Impl {
  struct Segment {
    void* ptr;
    std::size_t size;
  };
  std::vector<Segment> segments;
  std::size_t segment = 0;  // current segment
  std::size_t offset = 0;   // bytes used in the current segment
  std::size_t used = 0;

  ~Impl() {
    for (const Segment& s : segments) (void)hipFree(s.ptr);
  }
  bool grow(std::size_t bytes) {
    std::size_t size = segments.empty() ? std::size_t{1} << 20 : segments.back().size * 2;
    if (size < bytes) size = bytes;
    void* p = nullptr;
    if (hipMalloc(&p, size) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    segments.push_back({p, size});
    return true;
  }
};

namespace detail {

WorkspaceFrame::WorkspaceFrame(Workspace* w) : w_(w) {
  if (w_ != nullptr && w_->impl_ != nullptr) {
    segment_ = w_->impl_->segment;
    offset_ = w_->impl_->offset;
    used_ = w_->impl_->used;
  }
}

WorkspaceFrame::~WorkspaceFrame() {
  if (w_ != nullptr && w_->impl_ != nullptr) {
    w_->impl_->segment = segment_;
    w_->impl_->offset = offset_;
    w_->impl_->used = used_;
  }
}

}  // namespace detail

Workspace::Workspace() : impl_(new (std::nothrow) Impl) {}
Workspace::~Workspace() = default;
Workspace::Workspace(Workspace&& other) noexcept = default;
Workspace& Workspace::operator=(Workspace&& other) noexcept = default;

Status Workspace::reserve(std::size_t bytes) {
  if (impl_ == nullptr) return Status::kOutOfMemory;
  for (std::size_t i = impl_->segment; i < impl_->segments.size(); ++i) {
    const std::size_t used = i == impl_->segment ? impl_->offset : 0;
    if (impl_->segments[i].size - used >= bytes) return Status::kOk;
  }
  return impl_->grow(bytes) ? Status::kOk : Status::kOutOfMemory;
}

void* Workspace::allocate(std::size_t bytes, std::size_t alignment) noexcept {
  if (impl_ == nullptr || bytes == 0 || alignment == 0 || alignment > kAlignment ||
      (alignment & (alignment - 1)) != 0)
    return nullptr;
  if (bytes > std::numeric_limits<std::size_t>::max() - kAlignment) return nullptr;
  Impl& w = *impl_;
  for (;;) {
    if (w.segment < w.segments.size()) {
      const Impl::Segment& s = w.segments[w.segment];
      const std::size_t start = (w.offset + alignment - 1) & ~(alignment - 1);
      if (start <= s.size && s.size - start >= bytes) {
        w.used += start + bytes - w.offset;
        w.offset = start + bytes;
        return static_cast<char*>(s.ptr) + start;
      }
      if (w.segment + 1 < w.segments.size()) {
        w.used += s.size - w.offset;
        ++w.segment;
        w.offset = 0;
        continue;
      }
    }
    // No segment left that fits: append one and move to it.
    if (!w.grow(bytes)) return nullptr;
    if (w.segment + 1 < w.segments.size()) {
      w.used += w.segments[w.segment].size - w.offset;
      w.segment = w.segments.size() - 1;
      w.offset = 0;
    }
  }
}

void Workspace::reset() noexcept {
  if (impl_ == nullptr) return;
  impl_->segment = 0;
  impl_->offset = 0;
  impl_->used = 0;
}

std::size_t Workspace::capacity() const noexcept {
  std::size_t total = 0;
  if (impl_ != nullptr)
    for (const auto& s : impl_->segments) total += s.size;
  return total;
}

std::size_t Workspace::used() const noexcept { return impl_ == nullptr ? 0 : impl_->used; }

// ------------------------------------------------------ CpuPackedWeights ---

namespace {

// src/memory/packed_weights.cpp:141-155 (row_tile).
long long row_tile(CpuPanelLayout layout) {
  switch (layout) {
    case CpuPanelLayout::kPortableRows1: return 1;
    case CpuPanelLayout::kNeonRows4: return 4;
    case CpuPanelLayout::kAvx2Rows8: return 8;
    case CpuPanelLayout::kAvx512Rows16: return 16;
    case CpuPanelLayout::kAuto: return 0;
  }
  return 0;
}

// src/memory/packed_weights.cpp:157-166 (automatic_layout), from this
// host's CPU features: the panel stays byte-compatible with what the
// reference would build on the same machine.
CpuPanelLayout automatic_layout() {
  __builtin_cpu_init();
  if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
      __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512dq"))
    return CpuPanelLayout::kAvx512Rows16;
  if (__builtin_cpu_supports("avx2")) return CpuPanelLayout::kAvx2Rows8;
  return CpuPanelLayout::kPortableRows1;
}

// src/memory/packed_weights.cpp:168-182 (required_isa).
CpuPreparedIsa isa_for(CpuPanelLayout layout) {
  switch (layout) {
    case CpuPanelLayout::kNeonRows4: return CpuPreparedIsa::kNeon;
    case CpuPanelLayout::kAvx2Rows8: return CpuPreparedIsa::kAvx2;
    case CpuPanelLayout::kAvx512Rows16: return CpuPreparedIsa::kAvx512;
    default: return CpuPreparedIsa::kPortable;
  }
}

bool mul_fits(std::size_t a, std::size_t b, std::size_t* out) {
  if (a != 0 && b > std::numeric_limits<std::size_t>::max() / a) return false;
  *out = a * b;
  return true;
}

bool add_fits(std::size_t a, std::size_t b, std::size_t* out) {
  if (b > std::numeric_limits<std::size_t>::max() - a) return false;
  *out = a + b;
  return true;
}

// Bytes of one side table appended at `*end`, aligned to its element type
// (src/memory/packed_weights.cpp:125-134).
template <class T>
bool table_end(std::size_t count, std::size_t* end) {
  if (count == 0) return true;
  std::size_t at = (*end + alignof(T) - 1) / alignof(T) * alignof(T), bytes = 0;
  return at >= *end && mul_fits(count, sizeof(T), &bytes) && add_fits(at, bytes, end);
}

template <class T>
void put_table(const std::vector<T>& v, std::uint8_t* dst, std::size_t* cursor,
               std::size_t* offset) {
  if (v.empty()) return;
  const std::size_t at = (*cursor + alignof(T) - 1) / alignof(T) * alignof(T);
  *offset = at;
  std::memcpy(dst + at, v.data(), v.size() * sizeof(T));
  *cursor = at + v.size() * sizeof(T);
}

// Block geometry of a canonical layout's row panel
// (src/memory/packed_weights.cpp:72-122).
bool canonical_geometry(const QuantTensorMetadata& md, long long* elems, std::size_t* bytes) {
  const long long group = md.group_size > 0 ? md.group_size : md.logical_columns;
  switch (md.layout) {
    case CanonicalQuantLayout::kInt4Symmetric:
    case CanonicalQuantLayout::kUInt4Affine:
    case CanonicalQuantLayout::kFP4E2M1:
      *elems = group;
      *bytes = static_cast<std::size_t>(group / 2);
      return group > 0 && group % 2 == 0;
    case CanonicalQuantLayout::kInt8Symmetric:
    case CanonicalQuantLayout::kInt8Affine:
    case CanonicalQuantLayout::kFP8E4M3FN:
    case CanonicalQuantLayout::kFP8E5M2:
      *elems = group;
      *bytes = static_cast<std::size_t>(group);
      return group > 0;
    case CanonicalQuantLayout::kMXFP8E4M3E8M0: *elems = 32; *bytes = 33; return true;
    case CanonicalQuantLayout::kMXFP4E2M1E8M0: *elems = 32; *bytes = 17; return true;
    case CanonicalQuantLayout::kNVFP4E2M1E4M3: *elems = 16; *bytes = 8; return true;
    case CanonicalQuantLayout::kBitNetTernary: *elems = 32; *bytes = 10; return true;
    case CanonicalQuantLayout::kTurboQuantKey:
    case CanonicalQuantLayout::kTurboQuantValue: return false;
  }
  return false;
}

// Panel [row_panel, k_block, row_lane, block_bytes], rows past the end zero
// (src/memory/packed_weights.cpp:252-265).
void build_panel(const std::uint8_t* src, std::uint8_t* dst, long long rows, long long bpr,
                 long long tile, std::size_t block_bytes) {
  const long long panels = rows / tile + (rows % tile != 0 ? 1 : 0);
  for (long long panel = 0; panel < panels; ++panel)
    for (long long block = 0; block < bpr; ++block)
      for (long long lane = 0; lane < tile; ++lane) {
        const long long row = panel * tile + lane;
        if (row >= rows) continue;
        std::memcpy(dst + ((panel * bpr + block) * tile + lane) * block_bytes,
                    src + (row * bpr + block) * block_bytes, block_bytes);
      }
}

struct AlignedFree {
  void operator()(void* p) const { std::free(p); }
};

std::uint64_t ns_since(std::chrono::steady_clock::time_point t0) {
  return static_cast<std::uint64_t>(std::chrono::duration_cast<std::chrono::nanoseconds>(
                                        std::chrono::steady_clock::now() - t0)
                                        .count());
}

}  // namespace

struct CpuPackedWeights::Impl {
  CpuPackedWeightsInfo info;
  std::vector<std::uint8_t> contract;
  std::unique_ptr<std::uint8_t, AlignedFree> panel;
  void* device = nullptr;                    // [data | scales | row sums], 256-byte aligned parts
  const float* device_scales = nullptr;
  const std::int32_t* device_row_sums = nullptr;
  const float* device_zero_points = nullptr;
  ~Impl() {
    if (device != nullptr) (void)hipFree(device);
  }
  bool alloc_panel(std::size_t bytes) {
    const std::size_t aligned = (bytes + 63) / 64 * 64;
    panel.reset(static_cast<std::uint8_t*>(std::aligned_alloc(64, aligned ? aligned : 64)));
    if (panel == nullptr) return false;
    std::memset(panel.get(), 0, aligned ? aligned : 64);
    return true;
  }
};

CpuPackedWeights::CpuPackedWeights() = default;
CpuPackedWeights::~CpuPackedWeights() = default;
CpuPackedWeights::CpuPackedWeights(CpuPackedWeights&& other) noexcept = default;
CpuPackedWeights& CpuPackedWeights::operator=(CpuPackedWeights&& other) noexcept = default;

// src/memory/packed_weights.cpp:197-278 (prepare): validation order, panel
// index formula with a zero-padded last panel, and the recorded info fields.
Status CpuPackedWeights::prepare(QuantFormat format, const void* contract_packed,
                                 long long rows, long long columns, CpuPanelLayout layout) {
  const auto start = std::chrono::steady_clock::now();
  if (contract_packed == nullptr) return Status::kInvalidArgument;
  if (layout == CpuPanelLayout::kAuto) layout = automatic_layout();
  const long long tile = row_tile(layout);
  if (tile == 0) return Status::kInvalidArgument;
  std::size_t contract_bytes = 0;
  const Status st = qgemv_packed_size(format, rows, columns, &contract_bytes);
  if (st != Status::kOk) return st;
  const std::size_t block_bytes = format == QuantFormat::kQ8_0 ? 34 : 18;
  const long long bpr = columns / 32;
  const long long panels = rows / tile + (rows % tile != 0 ? 1 : 0);
  std::size_t panel_bytes = 0;
  if (!mul_fits(static_cast<std::size_t>(panels), static_cast<std::size_t>(bpr), &panel_bytes) ||
      !mul_fits(panel_bytes, static_cast<std::size_t>(tile), &panel_bytes) ||
      !mul_fits(panel_bytes, block_bytes, &panel_bytes))
    return Status::kInvalidShape;

  auto impl = std::unique_ptr<Impl>(new (std::nothrow) Impl);
  if (impl == nullptr) return Status::kOutOfMemory;
  try {
    impl->contract.resize(contract_bytes);
  } catch (const std::bad_alloc&) {
    return Status::kOutOfMemory;
  }
  if (detail::device_accessible(contract_packed)) {
    if (hipMemcpy(impl->contract.data(), contract_packed, contract_bytes,
                  hipMemcpyDeviceToHost) != hipSuccess)
      return Status::kDeviceError;
  } else {
    std::memcpy(impl->contract.data(), contract_packed, contract_bytes);
  }
  if (!impl->alloc_panel(panel_bytes)) return Status::kOutOfMemory;
  build_panel(impl->contract.data(), impl->panel.get(), rows, bpr, tile, block_bytes);
  const hipError_t e = hipMalloc(&impl->device, contract_bytes);
  if (e != hipSuccess) {
    impl->device = nullptr;
    return detail::from_hip(e);
  }
  if (hipMemcpy(impl->device, impl->contract.data(), contract_bytes, hipMemcpyHostToDevice) !=
      hipSuccess)
    return Status::kDeviceError;

  CpuPackedWeightsInfo& info = impl->info;
  info.format = format;
  info.layout = layout;
  info.rows = rows;
  info.columns = columns;
  info.row_tile = tile;
  info.block_size = 32;
  info.blocks_per_row = bpr;
  info.block_bytes = block_bytes;
  info.contract_bytes = contract_bytes;
  info.panel_bytes = panel_bytes;
  info.prepared_version = 1;
  info.required_isa = isa_for(layout);
  info.column_tile = 32;
  info.panel_alignment = 64;
  info.prepared_bytes = panel_bytes;
  info.memory_amplification =
      contract_bytes == 0 ? 0.0 : static_cast<double>(panel_bytes) / contract_bytes;
  info.device_bytes = contract_bytes;
  info.preparation_ns = ns_since(start);
  impl_ = std::move(impl);
  return Status::kOk;
}

// src/memory/packed_weights.cpp:280-412 (prepare from a canonical tensor):
// tensor validation, layout, block geometry (kUnsupportedFormat for a
// layout without one), panel and side-table sizes, then the panel followed
// by the tables in the reference's order, each at its type's alignment.
Status CpuPackedWeights::prepare(const CanonicalQuantTensor& t, CpuPanelLayout layout) {
  const auto start = std::chrono::steady_clock::now();
  Status st = validate_canonical_quant_tensor(t);
  if (st != Status::kOk) return st;
  if (layout == CpuPanelLayout::kAuto) layout = automatic_layout();
  const long long tile = row_tile(layout);
  if (tile == 0) return Status::kInvalidArgument;
  long long elems = 0;
  std::size_t block_bytes = 0;
  if (!canonical_geometry(t.metadata, &elems, &block_bytes) ||
      t.metadata.logical_columns % elems != 0)
    return Status::kUnsupportedFormat;
  const long long rows = t.metadata.logical_rows, columns = t.metadata.logical_columns;
  const long long bpr = columns / elems;
  const long long panels = rows / tile + (rows % tile != 0 ? 1 : 0);
  std::size_t panel_bytes = 0;
  if (!mul_fits(static_cast<std::size_t>(panels), static_cast<std::size_t>(bpr), &panel_bytes) ||
      !mul_fits(panel_bytes, static_cast<std::size_t>(tile), &panel_bytes) ||
      !mul_fits(panel_bytes, block_bytes, &panel_bytes))
    return Status::kInvalidShape;
  std::size_t prepared = panel_bytes;
  if (!table_end<std::uint8_t>(t.scale_codes.size(), &prepared) ||
      !table_end<float>(t.scales.size(), &prepared) ||
      !table_end<float>(t.zero_points.size(), &prepared) ||
      !table_end<float>(t.activation_scales.size(), &prepared) ||
      !table_end<int>(t.activation_zero_points.size(), &prepared) ||
      !table_end<int>(t.group_index.size(), &prepared) ||
      !table_end<int>(t.act_order.size(), &prepared) ||
      !table_end<std::int32_t>(t.row_sums.size(), &prepared))
    return Status::kInvalidShape;
  // logical bytes: the canonical data plus every table at its element size
  std::size_t logical = t.data.size();
  const std::size_t parts[][2] = {{t.scale_codes.size(), 1}, {t.scales.size(), 4},
                                  {t.zero_points.size(), 4}, {t.activation_scales.size(), 4},
                                  {t.activation_zero_points.size(), sizeof(int)},
                                  {t.group_index.size(), sizeof(int)},
                                  {t.act_order.size(), sizeof(int)}, {t.row_sums.size(), 4}};
  for (const auto& part : parts) {
    std::size_t b = 0;
    if (!mul_fits(part[0], part[1], &b) || !add_fits(logical, b, &logical))
      return Status::kInvalidShape;
  }

  auto impl = std::unique_ptr<Impl>(new (std::nothrow) Impl);
  if (impl == nullptr) return Status::kOutOfMemory;
  try {
    impl->contract = t.data;
  } catch (const std::bad_alloc&) {
    return Status::kOutOfMemory;
  }
  if (!impl->alloc_panel(prepared)) return Status::kOutOfMemory;
  CpuPackedWeightsInfo& info = impl->info;
  std::uint8_t* dst = impl->panel.get();
  build_panel(t.data.data(), dst, rows, bpr, tile, block_bytes);
  std::size_t cursor = panel_bytes;
  put_table(t.scale_codes, dst, &cursor, &info.scale_code_table_offset);
  put_table(t.scales, dst, &cursor, &info.scale_table_offset);
  put_table(t.zero_points, dst, &cursor, &info.zero_point_table_offset);
  put_table(t.activation_scales, dst, &cursor, &info.activation_scale_offset);
  put_table(t.activation_zero_points, dst, &cursor, &info.activation_zero_point_offset);
  put_table(t.group_index, dst, &cursor, &info.group_index_offset);
  put_table(t.act_order, dst, &cursor, &info.act_order_offset);
  put_table(t.row_sums, dst, &cursor, &info.row_sum_table_offset);

  // device mirror: data, f32 scales, int32 row sums and f32 zero points,
  // each 256-byte aligned
  auto up = [](std::size_t b) { return (b + 255) / 256 * 256; };
  const std::size_t d_scales = up(t.data.size());
  const std::size_t d_sums = d_scales + up(t.scales.size() * sizeof(float));
  const std::size_t d_zeros = d_sums + up(t.row_sums.size() * sizeof(std::int32_t));
  const std::size_t d_bytes = d_zeros + t.zero_points.size() * sizeof(float);
  hipError_t e = hipMalloc(&impl->device, d_bytes ? d_bytes : 256);
  if (e != hipSuccess) {
    impl->device = nullptr;
    return detail::from_hip(e);
  }
  auto* base = static_cast<std::uint8_t*>(impl->device);
  if ((e = hipMemcpy(base, t.data.data(), t.data.size(), hipMemcpyHostToDevice)) != hipSuccess ||
      (!t.scales.empty() &&
       (e = hipMemcpy(base + d_scales, t.scales.data(), t.scales.size() * sizeof(float),
                      hipMemcpyHostToDevice)) != hipSuccess) ||
      (!t.row_sums.empty() &&
       (e = hipMemcpy(base + d_sums, t.row_sums.data(), t.row_sums.size() * sizeof(std::int32_t),
                      hipMemcpyHostToDevice)) != hipSuccess) ||
      (!t.zero_points.empty() &&
       (e = hipMemcpy(base + d_zeros, t.zero_points.data(), t.zero_points.size() * sizeof(float),
                      hipMemcpyHostToDevice)) != hipSuccess))
    return Status::kDeviceError;
  impl->device_zero_points =
      t.zero_points.empty() ? nullptr : reinterpret_cast<float*>(base + d_zeros);
  impl->device_scales = t.scales.empty() ? nullptr : reinterpret_cast<float*>(base + d_scales);
  impl->device_row_sums =
      t.row_sums.empty() ? nullptr : reinterpret_cast<std::int32_t*>(base + d_sums);

  info.canonical_layout = t.metadata.layout;
  info.quant_metadata = t.metadata;
  info.has_canonical_layout = true;
  info.layout = layout;
  info.rows = rows;
  info.columns = columns;
  info.row_tile = tile;
  info.block_size = elems;
  info.blocks_per_row = bpr;
  info.block_bytes = block_bytes;
  info.contract_bytes = t.data.size();
  info.panel_bytes = panel_bytes;
  info.prepared_version = 2;
  info.required_isa = isa_for(layout);
  info.column_tile = elems;
  info.panel_alignment = 64;
  info.logical_bytes = logical;
  info.prepared_bytes = prepared;
  info.memory_amplification =
      logical == 0 ? 0.0 : static_cast<double>(prepared) / static_cast<double>(logical);
  info.device_bytes = d_bytes;
  info.preparation_ns = ns_since(start);
  impl_ = std::move(impl);
  return Status::kOk;
}

void CpuPackedWeights::reset() noexcept { impl_.reset(); }
bool CpuPackedWeights::ready() const noexcept { return impl_ != nullptr; }
CpuPackedWeightsInfo CpuPackedWeights::info() const noexcept {
  return impl_ == nullptr ? CpuPackedWeightsInfo{} : impl_->info;
}
const void* CpuPackedWeights::contract_data() const noexcept {
  return impl_ == nullptr ? nullptr : impl_->contract.data();
}
const void* CpuPackedWeights::panel_data() const noexcept {
  return impl_ == nullptr ? nullptr : impl_->panel.get();
}
const void* CpuPackedWeights::device_data() const noexcept {
  return impl_ == nullptr ? nullptr : impl_->device;
}
const float* CpuPackedWeights::device_scales() const noexcept {
  return impl_ == nullptr ? nullptr : impl_->device_scales;
}
const std::int32_t* CpuPackedWeights::device_row_sums() const noexcept {
  return impl_ == nullptr ? nullptr : impl_->device_row_sums;
}
const float* CpuPackedWeights::device_zero_points() const noexcept {
  return impl_ == nullptr ? nullptr : impl_->device_zero_points;
}

const char* cpu_prepared_isa_name(CpuPreparedIsa isa) {
  switch (isa) {
    case CpuPreparedIsa::kPortable: return "portable";
    case CpuPreparedIsa::kNeon: return "neon";
    case CpuPreparedIsa::kDotProd: return "dotprod";
    case CpuPreparedIsa::kI8MM: return "i8mm";
    case CpuPreparedIsa::kSVE: return "sve";
    case CpuPreparedIsa::kSME: return "sme";
    case CpuPreparedIsa::kAvx2: return "avx2";
    case CpuPreparedIsa::kAvx512: return "avx512";
    case CpuPreparedIsa::kAvx512VNNI: return "avx512_vnni";
    case CpuPreparedIsa::kAMX: return "amx";
  }
  return "unknown";
}

const char* cpu_panel_layout_name(CpuPanelLayout layout) {
  switch (layout) {
    case CpuPanelLayout::kAuto: return "auto";
    case CpuPanelLayout::kPortableRows1: return "portable_rows1";
    case CpuPanelLayout::kNeonRows4: return "neon_rows4";
    case CpuPanelLayout::kAvx2Rows8: return "avx2_rows8";
    case CpuPanelLayout::kAvx512Rows16: return "avx512_rows16";
  }
  return "unknown";
}

// --------------------------------------------------- prepared entry points ---

// kernels/quantization/qgemm_panel.cpp:214-240: readiness, shape product,
// canonical weights to the storage route, nulls; every M is then one launch
// over the device mirror (the reference routes M == 1 to qgemv and M < 64 to
// qgemm -- the same arithmetic contract).
Status qgemm_prepacked(const CpuPackedWeights& weights, const float* x, float* y, long long m,
                       Workspace* workspace) {
  if (!weights.ready()) return Status::kInvalidArgument;
  const CpuPackedWeightsInfo info = weights.info();
  if (m <= 0 || info.rows <= 0 || info.columns <= 0 ||
      m > std::numeric_limits<long long>::max() / info.rows ||
      m * info.rows > std::numeric_limits<long long>::max() / info.columns)
    return Status::kInvalidShape;
  if (info.has_canonical_layout)
    return qgemm_prepacked_storage(weights, {x, FloatStorageType::kF32, m * info.columns},
                                   {y, FloatStorageType::kF32, m * info.rows}, m, workspace);
  if (m > std::numeric_limits<int>::max())   // this library's dimension limit (as for n, k)
    return Status::kInvalidShape;
  if (x == nullptr || y == nullptr || weights.device_data() == nullptr)
    return Status::kInvalidArgument;
  detail::WorkspaceFrame frame(workspace);
  detail::Staging g(workspace);
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * m * info.columns));
  float* yd = static_cast<float*>(g.out(y, sizeof(float) * m * info.rows));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemm(static_cast<int>(info.format), weights.device_data(), xd, yd, m,
                               info.rows, info.columns, g.stream()));
}

// kernels/quantization/qgemm_canonical.cpp:4647-4653: the storage route with
// f32 x and y (GGUF-prepared weights: kUnsupportedFormat).
Status qgemv_prepacked(const CpuPackedWeights& weights, const float* x, float* y,
                       Workspace* workspace) {
  const CpuPackedWeightsInfo info = weights.info();
  return qgemm_prepacked_storage(weights, {x, FloatStorageType::kF32, info.columns},
                                 {y, FloatStorageType::kF32, info.rows}, 1, workspace);
}

}  // namespace quixicore_cpu
