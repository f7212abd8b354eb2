// Compound ops as graphs of primitives (reference src/ops.cpp:5-18).  The
// expression order is part of the result: the planner recognises these
// graphs (softmax's max/exp/sum/divide becomes one row program) but
// evaluates exactly these operations.

#include "porch/ops.hpp"

namespace porch {

    tensor_expr relu(tensor_expr value) { return maximum(value, 0.0F); }

    tensor_expr softmax(tensor_expr value, size_t axis) {
        const std::vector<index_t> shape = value.shape();
        const tensor_expr shifted = value - broadcast_to(max(value, axis, true), shape);
        const tensor_expr numerator = exp(shifted);
        return numerator / broadcast_to(sum(numerator, axis, true), shape);
    }

    tensor_expr logistic(tensor_expr value) {
        return reciprocal(1.0F + exp(0.0F - value));
    }

} // namespace porch
