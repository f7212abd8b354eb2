#pragma once

// porch's runtime namespace under the name the reference's programs use
// (porch::cuda_jit, reference include/porch/cuda_jit.hpp).  On MI355X the
// runtime is porch::hip_jit; this is a namespace alias, not a CUDA header.

#include "porch/hip_jit.hpp"

namespace porch {
    namespace cuda_jit = hip_jit;
} // namespace porch
