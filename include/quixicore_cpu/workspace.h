// Drop-in of Workspace (include/quixicore_cpu/workspace.h:19-59 of the
// reference): a reusable, pointer-stable, segmented scratch arena.  Here the
// arena is DEVICE memory; qgemm_prepacked uses it to stage host activations
// and outputs, so warmed-up calls do not allocate.  Not thread-safe.
#pragma once

#include <cstddef>
#include <memory>

#include "quixicore_cpu/status.h"

namespace quixicore_cpu {

namespace detail {
class WorkspaceFrame;
}

class Workspace {
 public:
  static constexpr std::size_t kAlignment = 64;

  Workspace();
  ~Workspace();
  Workspace(Workspace&& other) noexcept;
  Workspace& operator=(Workspace&& other) noexcept;
  Workspace(const Workspace&) = delete;
  Workspace& operator=(const Workspace&) = delete;

  // Ensures a future contiguous allocation of at least bytes can be served.
  Status reserve(std::size_t bytes);
  // Aligned device scratch, or nullptr for zero bytes, bad alignment or
  // allocation failure.  alignment: a power of two <= kAlignment.
  void* allocate(std::size_t bytes, std::size_t alignment = kAlignment) noexcept;
  // Releases all allocations logically, keeping the backing segments.
  void reset() noexcept;
  std::size_t capacity() const noexcept;
  std::size_t used() const noexcept;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
  friend class detail::WorkspaceFrame;
};

}  // namespace quixicore_cpu
