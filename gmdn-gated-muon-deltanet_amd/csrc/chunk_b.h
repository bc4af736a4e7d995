// Internal launch interface of the fused chunk (Level B) kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gmdn {}  // namespace gmdn
