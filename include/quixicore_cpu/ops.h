// The part of include/quixicore_cpu/ops.h of the reference that the prepared
// projection epilogue takes (:56): the activation applied after the bias.
#pragma once

namespace quixicore_cpu {

enum class LinearActivation { kNone, kGeluErf, kGeluTanh, kSilu, kRelu2 };

}  // namespace quixicore_cpu
