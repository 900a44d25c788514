// Drop-in of the storage descriptors of include/quixicore_cpu/float_storage.h
// of the reference (:18-30): raw IEEE binary32 / binary16 / bfloat16 buffers
// with an element count.  The prepared storage projections
// (include/quixicore_cpu/qgemm.h) take and return these; 16-bit values are
// decoded exactly, accumulated in f32 and rounded once at the store.
// Pointers may be host or device memory (host buffers are staged).
#pragma once

#include "quixicore_cpu/status.h"

namespace quixicore_cpu {

enum class FloatStorageType { kF32, kF16, kBF16 };

struct FloatStorageInput {
  const void* data = nullptr;
  FloatStorageType type = FloatStorageType::kF32;
  long long count = 0;
};

struct FloatStorageOutput {
  void* data = nullptr;
  FloatStorageType type = FloatStorageType::kF32;
  long long count = 0;
};

}  // namespace quixicore_cpu
