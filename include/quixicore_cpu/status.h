// Drop-in of include/quixicore_cpu/status.h:5-11 of the reference: the same
// enumerators in the same order.  kDeviceError is appended for HIP runtime
// failures, which the CPU reference cannot have.
#pragma once

namespace quixicore_cpu {

enum class Status {
  kOk,
  kInvalidShape,       // non-positive dims, block-size violations
  kUnsupportedFormat,  // a QuantFormat this build has no kernel for
  kInvalidArgument,    // null pointer, non-finite input or scale
  kOutOfMemory,        // device staging / mirror allocation failed
  kDeviceError,        // the HIP runtime rejected a launch or copy
};

}  // namespace quixicore_cpu
