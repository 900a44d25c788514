// The prepared storage projection scenarios (tests/cpp/storage_scenarios.h)
// through this library's C++ drop-in API with host buffers.  Writes every
// status and output under argv[1]; tests/test_gpu_canonical.py compares them
// with the reference's run of the same scenarios (oracle/_ref) and with the
// f64 restatement.
#include <cstdio>

#include "storage_scenarios.h"

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: storage_check <output dir>\n");
    return 2;
  }
  storage_scenarios::Sink sink(argv[1]);
  if (sink.manifest == nullptr) return 2;
  storage_scenarios::run(sink);
  std::printf("storage_check: ok\n");
  return 0;
}
