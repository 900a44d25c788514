// Per-(device, stream) scratch cache of the allocating entry points.  A
// stream-ordered allocation per call (hipMallocAsync / hipFreeAsync) costs
// about 10 us on this stack, more than a small projection's kernels; a
// cached buffer costs a table lookup.
#include <memory>
#include <mutex>
#include <vector>

#include "qc_internal.h"

namespace qc {
namespace {

std::mutex g_ws_mu;                                        // guards the two lists below
std::vector<std::unique_ptr<StreamWorkspace>> g_ws_table;  // entries live until exit
std::vector<void*> g_ws_retired;                           // buffers a captured graph may use

}  // namespace

hipError_t stream_workspace(hipStream_t s, StreamWorkspace** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  for (auto& w : g_ws_table)
    if (w->device == dev && w->stream == s) {
      *out = w.get();
      return hipSuccess;
    }
  g_ws_table.push_back(std::make_unique<StreamWorkspace>());
  g_ws_table.back()->device = dev;
  g_ws_table.back()->stream = s;
  *out = g_ws_table.back().get();
  return hipSuccess;
}

hipError_t stream_buffer(StreamWorkspace* w, hipStream_t s, size_t bytes, int tag, void** out) {
  if (tag < 0 || tag >= kStreamBuffers) return hipErrorInvalidValue;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) return e;
  const bool capturing = cap != hipStreamCaptureStatusNone;
  if (w->bytes[tag] >= bytes) {
    w->captured[tag] = w->captured[tag] || capturing;
    *out = w->ptr[tag];
    return hipSuccess;
  }
  if (w->ptr[tag] != nullptr) {
    if (capturing || w->captured[tag]) {
      std::lock_guard<std::mutex> lock(g_ws_mu);
      g_ws_retired.push_back(w->ptr[tag]);
    } else {
      if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
      if ((e = hipFree(w->ptr[tag])) != hipSuccess) return e;
    }
    w->ptr[tag] = nullptr;
    w->bytes[tag] = 0;
  }
  void* p = nullptr;
  if ((e = hipMalloc(&p, bytes ? bytes : 256)) != hipSuccess) return e;
  w->ptr[tag] = p;
  w->bytes[tag] = bytes ? bytes : 256;
  w->captured[tag] = capturing;
  *out = w->ptr[tag];
  return hipSuccess;
}

}  // namespace qc
