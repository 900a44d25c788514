// The quantize_canonical / dequantize_canonical scenarios
// (tests/cpp/canonical_quant_scenarios.h) through this library's C++ drop-in
// API with host buffers.  Writes every status and output under argv[1];
// tests/test_gpu_canonical_quant.py compares them with the reference's run of
// the same scenarios (oracle/_ref).
#include <cstdio>

#include "canonical_quant_scenarios.h"

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: canonical_quant_check <output dir>\n");
    return 2;
  }
  storage_scenarios::Sink sink(argv[1]);
  if (sink.manifest == nullptr) return 2;
  canonical_quant_scenarios::run(sink);
  std::printf("canonical_quant_check: ok\n");
  return 0;
}
