#pragma once

// Value ranges of kernel-expression nodes, used to pick cheaper exact
// instruction sequences where the operands are provably tame:
//
//   reciprocal / division by x with |x| in [2^-125, 2^125]: the hardware
//   reciprocal plus one Newton step is the correctly rounded 1/x (checked
//   exhaustively on gfx950 over whole binades at both ends of that range);
//   exp of x <= 88: no overflow handling is needed.
//
// Ranges are closed float intervals plus a may-be-NaN flag.  Every rule is
// conservative under IEEE round-to-nearest: rounding is monotone, so the
// rounded operation applied to interval endpoints bounds every rounded
// result inside.

#include "lower.hpp"

#include <functional>
#include <vector>

namespace porch::cg {

    struct vrange {
        float lo;
        float hi;
        bool nan;
        static vrange any();
        static vrange exactly(float v);
        [[nodiscard]] bool within(float a, float b) const { return !nan && lo >= a && hi <= b; }
    };

    // Range of every node of `k` (indexed like k.nodes).  `row_value_range`
    // gives the range of row reduction `row` (any() when unknown); `refine`
    // may narrow a node's computed range from facts the generic rules do not
    // see (e.g. x - max(x) <= 0 in a row program).
    std::vector<vrange> value_ranges(
        const kexpr& k, const std::function<vrange(int row)>& row_value_range = nullptr,
        const std::function<vrange(int id, const vrange& computed)>& refine = nullptr
    );

    // |x| in [2^-125, 2^125] or NaN: the fast reciprocal is exact here.
    bool reciprocal_is_tame(const vrange& r);

} // namespace porch::cg
