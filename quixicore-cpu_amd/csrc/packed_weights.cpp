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

// Restores a workspace to the allocation mark taken at construction (the
// scope-exit rewind of the reference's WorkspaceFrame,
// src/memory/workspace_internal.h:15-44).
class WorkspaceFrame {
 public:
  explicit WorkspaceFrame(Workspace* w) : w_(w) {
    if (w_ != nullptr && w_->impl_ != nullptr) {
      segment_ = w_->impl_->segment;
      offset_ = w_->impl_->offset;
      used_ = w_->impl_->used;
    }
  }
  ~WorkspaceFrame() {
    if (w_ != nullptr && w_->impl_ != nullptr) {
      w_->impl_->segment = segment_;
      w_->impl_->offset = offset_;
      w_->impl_->used = used_;
    }
  }

 private:
  Workspace* w_;
  std::size_t segment_ = 0, offset_ = 0, used_ = 0;
};

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

// src/memory/packed_weights.cpp:141-155 (row_tile).  kAuto resolves to the
// one-row panel: the GPU kernels read the canonical bytes, so the panel is
// kept only for API compatibility and the smallest one is chosen.
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

struct AlignedFree {
  void operator()(void* p) const { std::free(p); }
};

}  // namespace

struct CpuPackedWeights::Impl {
  CpuPackedWeightsInfo info;
  std::vector<std::uint8_t> contract;
  std::unique_ptr<std::uint8_t, AlignedFree> panel;
  void* device = nullptr;
  ~Impl() {
    if (device != nullptr) (void)hipFree(device);
  }
};

CpuPackedWeights::CpuPackedWeights() = default;
CpuPackedWeights::~CpuPackedWeights() = default;
CpuPackedWeights::CpuPackedWeights(CpuPackedWeights&& other) noexcept = default;
CpuPackedWeights& CpuPackedWeights::operator=(CpuPackedWeights&& other) noexcept = default;

// src/memory/packed_weights.cpp:197-278 (prepare): validation order, panel
// index formula dst[(panel*bpr + block)*tile + lane] = src[row*bpr + block]
// with a zero-padded last panel, and the recorded info fields.
Status CpuPackedWeights::prepare(QuantFormat format, const void* contract_packed,
                                 long long rows, long long columns, CpuPanelLayout layout) {
  const auto start = std::chrono::steady_clock::now();
  if (contract_packed == nullptr) return Status::kInvalidArgument;
  if (layout == CpuPanelLayout::kAuto) layout = CpuPanelLayout::kPortableRows1;
  const long long tile = row_tile(layout);
  if (tile == 0) return Status::kInvalidArgument;
  std::size_t contract_bytes = 0;
  const Status st = qgemv_packed_size(format, rows, columns, &contract_bytes);
  if (st != Status::kOk) return st;
  const std::size_t block_bytes = format == QuantFormat::kQ8_0 ? 34 : 18;
  const long long bpr = columns / 32;
  const long long panels = rows / tile + (rows % tile != 0 ? 1 : 0);
  const std::size_t panel_bytes = static_cast<std::size_t>(panels) * bpr * tile * block_bytes;

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
  const std::size_t aligned = (panel_bytes + 63) / 64 * 64;
  impl->panel.reset(static_cast<std::uint8_t*>(std::aligned_alloc(64, aligned ? aligned : 64)));
  if (impl->panel == nullptr) return Status::kOutOfMemory;
  std::memset(impl->panel.get(), 0, panel_bytes);
  const std::uint8_t* src = impl->contract.data();
  std::uint8_t* dst = impl->panel.get();
  for (long long panel = 0; panel < panels; ++panel)
    for (long long block = 0; block < bpr; ++block)
      for (long long lane = 0; lane < tile; ++lane) {
        const long long row = panel * tile + lane;
        if (row >= rows) continue;
        std::memcpy(dst + ((panel * bpr + block) * tile + lane) * block_bytes,
                    src + (row * bpr + block) * block_bytes, block_bytes);
      }
  const hipError_t e = hipMalloc(&impl->device, contract_bytes);
  if (e != hipSuccess) {
    impl->device = nullptr;
    return detail::from_hip(e);
  }
  if (hipMemcpy(impl->device, src, contract_bytes, hipMemcpyHostToDevice) != hipSuccess)
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
  info.column_tile = 32;
  info.panel_alignment = 64;
  info.prepared_bytes = panel_bytes;
  info.memory_amplification =
      contract_bytes == 0 ? 0.0 : static_cast<double>(panel_bytes) / contract_bytes;
  info.device_bytes = contract_bytes;
  info.preparation_ns = static_cast<std::uint64_t>(
      std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() -
                                                           start)
          .count());
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
// nulls; every M is then one launch over the device mirror (the reference
// routes M == 1 to qgemv and M < 64 to qgemm -- the same arithmetic contract).
Status qgemm_prepacked(const CpuPackedWeights& weights, const float* x, float* y, long long m,
                       Workspace* workspace) {
  if (!weights.ready()) return Status::kInvalidArgument;
  const CpuPackedWeightsInfo info = weights.info();
  if (m <= 0 || info.rows <= 0 || info.columns <= 0 ||
      m > std::numeric_limits<long long>::max() / info.rows ||
      m * info.rows > std::numeric_limits<long long>::max() / info.columns ||
      m > std::numeric_limits<int>::max())   // this library's dimension limit (as for n, k)
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

Status qgemv_prepacked(const CpuPackedWeights& weights, const float* x, float* y,
                       Workspace* workspace) {
  return qgemm_prepacked(weights, x, y, 1, workspace);
}

}  // namespace quixicore_cpu
