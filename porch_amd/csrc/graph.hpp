#pragma once

// porch's IR as a flat, topologically ordered node table: the form in which
// graphs cross the C ABI and the unit the planner caches by.  The node
// vocabulary, shape rules and error messages are the reference's
// (reference src/tensor.cpp:26-60 for the nodes, 190-339 and 341-496 for
// validation and shape inference).

#include "porch_amd.h"

#include <cstdint>
#include <string>
#include <vector>

namespace porch::ir {

    enum class op : int32_t {
        input = PORCH_OP_INPUT,
        scalar = PORCH_OP_SCALAR,
        add = PORCH_OP_ADD,
        subtract = PORCH_OP_SUBTRACT,
        multiply = PORCH_OP_MULTIPLY,
        divide = PORCH_OP_DIVIDE,
        matmul = PORCH_OP_MATMUL,
        slice = PORCH_OP_SLICE,
        reshape = PORCH_OP_RESHAPE,
        unsqueeze = PORCH_OP_UNSQUEEZE,
        transpose = PORCH_OP_TRANSPOSE,
        broadcast = PORCH_OP_BROADCAST,
        concat = PORCH_OP_CONCAT,
        sum = PORCH_OP_SUM,
        max = PORCH_OP_MAX,
        maximum = PORCH_OP_MAXIMUM,
        minimum = PORCH_OP_MINIMUM,
        exp = PORCH_OP_EXP,
        reciprocal = PORCH_OP_RECIPROCAL,
        permute = PORCH_OP_PERMUTE,
        batched_matmul = PORCH_OP_BATCHED_MATMUL,
    };

    constexpr int op_count = 21;

    struct node {
        op kind = op::input;
        int lhs = -1;
        int rhs = -1;
        int input = -1;
        float scalar = 0.0F;
        int64_t axis = 0;
        bool keepdim = false;
        std::vector<int64_t> shape;   // input / slice / reshape / broadcast;
                                      // permute: the permutation
        std::vector<int64_t> strides; // slice
        int64_t offset = 0;           // slice

        // Filled by infer():
        bool is_scalar = false;
        std::vector<int64_t> out; // inferred shape (empty for scalars)
    };

    struct graph {
        std::vector<node> nodes; // operands precede users; root is last
        int n_inputs = 0;        // 1 + largest input slot referenced

        [[nodiscard]] int root() const {
            return static_cast<int>(nodes.size()) - 1;
        }
        [[nodiscard]] const node& at(int index) const {
            return nodes[static_cast<size_t>(index)];
        }
    };

    bool is_elementwise_binary(op kind);
    bool is_reduction(op kind);
    bool is_view(op kind);

    // Copies a C-ABI node table, checking indices and kinds
    // (std::invalid_argument on malformed tables).
    graph from_c(const porch_graph* table);

    // Keeps only nodes reachable from the root, merges structurally equal
    // nodes (same kind, operands and parameters) and re-infers shapes.
    graph compact(const graph& g);

    // Shape inference and validation of every node, in order; throws the
    // reference's exceptions and messages.
    void infer(graph& g);

    // Canonical byte string of a compacted graph: kinds, operands, input
    // slots, parameters and scalar bit patterns.  Equal keys mean the same
    // generated kernels.
    std::string canonical_key(const graph& g);

    size_t checked_numel(const std::vector<int64_t>& shape);
    int64_t numel(const std::vector<int64_t>& shape);
    std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& shape);
    std::vector<int64_t> reduced_shape(
        const std::vector<int64_t>& shape, size_t axis, bool keepdim
    );

} // namespace porch::ir
