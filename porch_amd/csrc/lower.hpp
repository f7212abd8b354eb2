#pragma once

// Lowering of a fused region of the IR to a kernel expression (kexpr).
//
// The reference evaluates a fused graph at a linear output index and pastes
// div/mod index chains textually for every view (reference
// src/tensor.cpp:511-614, 722-818).  Here every view is composed into the
// memory index of each leaf as a function of the kernel's coordinates:
//
//   * affine:  index = c0 + sum_d w[d] * q_d   (slices, transposes,
//     broadcasts, unsqueeze and reshapes that split or merge dimensions
//     without carries all stay affine);
//   * generic: an integer C expression over q_0..q_{r-1} with div/mod,
//     used when a reshape of a strided view needs carries.
//
// Concat becomes a select whose condition is affine in the coordinates;
// loads under a branch are only evaluated when the branch is taken.  The
// emitters use the strides w[d] to choose vector loads, LDS-staged
// transposes and hoisting of row-invariant loads.

#include "graph.hpp"

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace porch::cg {

    struct ival {
        bool is_affine = true;
        int64_t c0 = 0;
        std::vector<int64_t> w; // one weight per kernel coordinate
        std::string code;       // generic form (when !is_affine)

        static ival constant(int64_t value, size_t rank);
        static ival coordinate(size_t d, size_t rank);
        [[nodiscard]] bool is_constant() const;
        [[nodiscard]] std::string str() const; // C expression
        [[nodiscard]] std::string key() const;
    };

    enum class kop {
        load,     // slot + index
        constant, // value
        add,
        subtract,
        multiply,
        divide,
        maximum,
        minimum,
        exp,
        reciprocal,
        select,   // cond ? a : b, cond = (lhs < bound)
        row_value // the row-uniform result of reduction `row`
    };

    struct kcond {
        ival lhs;
        int64_t bound = 0; // condition: lhs < bound
    };

    struct knode {
        kop op = kop::constant;
        int a = -1;
        int b = -1;
        int slot = -1; // load: kernel argument slot
        ival index;    // load
        // load: ranges [lo, hi) of the kernel coordinates under which the
        // load executes (the union over the branches that reach it)
        std::vector<std::pair<int64_t, int64_t>> box;
        float value = 0.0F;
        kcond cond;    // select
        int row = -1;  // row_value
    };

    // Arena of kernel expression nodes with structural sharing.
    struct kexpr {
        std::vector<knode> nodes;
        std::map<std::string, int> interned;

        int add(knode n);
        [[nodiscard]] const knode& at(int i) const {
            return nodes[static_cast<size_t>(i)];
        }
        // Loads reachable from `root` (each once).
        [[nodiscard]] std::vector<int> loads(int root) const;
        // Nodes reachable from `root` in evaluation order.
        [[nodiscard]] std::vector<int> postorder(int root) const;
    };

    // What a graph node becomes when the lowering reaches it.
    struct binding {
        enum class kind { slot, row_value };
        kind what = kind::slot;
        int slot = -1; // kernel argument holding the node's contiguous values
        int64_t offset = 0; // ... from this element of the slot on
        int row = -1;  // row reduction index
    };

    struct lowering {
        const ir::graph& g;
        kexpr& out;
        std::vector<int64_t> extent; // kernel coordinate extents
        std::map<int, binding> bound; // graph node -> replacement
        std::vector<int> input_slot;  // graph input index -> kernel slot

        // Ranges [lo, hi) of the kernel coordinates in the current branch.
        std::vector<std::pair<int64_t, int64_t>> box;

        lowering(const ir::graph& graph, kexpr& arena,
                 std::vector<int64_t> extents);

        // Value of graph node `id` at coordinates `coords` (one ival per
        // dimension of the node's shape).
        int at(int id, const std::vector<ival>& coords);
        // Value of graph node `id` at linear index `lin` of its shape.
        int at_linear(int id, const ival& lin);

        [[nodiscard]] std::vector<ival> identity() const;
        [[nodiscard]] ival linearize(
            const std::vector<ival>& coords, const std::vector<int64_t>& shape
        ) const;
        [[nodiscard]] std::vector<ival> delinearize(
            const ival& lin, const std::vector<int64_t>& shape
        ) const;
        // Smallest and largest value of an affine ival over the box.
        [[nodiscard]] std::pair<int64_t, int64_t> range(const ival& v) const;
    };

    std::string float_literal(float value);

} // namespace porch::cg
