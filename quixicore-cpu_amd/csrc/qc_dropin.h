// Internal helpers of the C++ drop-in layer: the per-device library stream and
// host<->device staging of the reference API's untyped pointers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <vector>

#include "quixicore_cpu/status.h"
#include "quixicore_cpu/workspace.h"

namespace quixicore_cpu::detail {

// One non-blocking, default-priority stream per device, created on first use.
hipStream_t library_stream();

// True for hipMalloc'd or managed memory.
bool device_accessible(const void* p);

Status from_hip(hipError_t e);

// Restores a workspace to the allocation mark taken at construction (the
// scope-exit rewind of the reference's WorkspaceFrame,
// src/memory/workspace_internal.h:15-44).
class WorkspaceFrame {
 public:
  explicit WorkspaceFrame(Workspace* w);
  ~WorkspaceFrame();
  WorkspaceFrame(const WorkspaceFrame&) = delete;
  WorkspaceFrame& operator=(const WorkspaceFrame&) = delete;

 private:
  Workspace* w_;
  std::size_t segment_ = 0, offset_ = 0, used_ = 0;
};

// Per-call staging.  in()/out() return a device view of a caller buffer:
// the buffer itself when the GPU can address it, else a device copy (taken
// from `workspace` when one is given, else hipMalloc'd and freed on scope
// exit).  finish() copies staged outputs back and waits for the stream.
// inout() is out() for a buffer the call may leave partly unwritten: the
// device copy starts as the caller's data.  finish_written() also copies
// back after a data-dependent failure reported once the work has run
// (kInvalidArgument), for ops whose reference writes what it can.
class Staging {
 public:
  explicit Staging(Workspace* workspace)
      : workspace_(workspace), stream_(library_stream()) {}
  ~Staging();
  Staging(const Staging&) = delete;
  Staging& operator=(const Staging&) = delete;

  const void* in(const void* host_or_device, std::size_t bytes);
  void* out(void* host_or_device, std::size_t bytes);
  void* inout(void* host_or_device, std::size_t bytes);
  // Device memory for the call's own use (freed with the staging).
  void* scratch(std::size_t bytes) { return device(bytes); }
  Status finish(int capi_status);
  Status finish_written(int capi_status);
  Status status() const { return status_; }
  hipStream_t stream() const { return stream_; }

 private:
  struct Back {
    void* host;
    void* dev;
    std::size_t bytes;
  };
  void* device(std::size_t bytes);

  Workspace* workspace_;
  hipStream_t stream_;
  Status status_ = Status::kOk;
  std::vector<void*> owned_;
  std::vector<Back> back_;
};

}  // namespace quixicore_cpu::detail
