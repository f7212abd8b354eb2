#pragma once

// Scalar and index types of porch's public API (reference:
// include/porch/types.hpp:8-19).  Tensors hold float32_t values; shapes,
// strides and offsets are index_t.

#include <stddef.h>
#include <stdint.h>

namespace porch {

    using index_t = int64_t;
    using float32_t = float;
    using float64_t = double;

#if defined(__FLT16_MANT_DIG__)
    using float16_t = _Float16;
#endif
#if defined(__SIZEOF_FLOAT128__)
    using float128_t = __float128;
#endif

} // namespace porch
