#pragma once

// Partitioning, code generation, compilation and execution of a graph.
// The MI355X replacement for the reference's lower_nested_reductions +
// materialize_expression (reference src/tensor.cpp:964-1066) and its
// per-launch module loading (src/cuda_jit.cpp:789-948).
//
// A graph is split into the fewest kernels the kernel classes allow:
//   1. an elementwise region over exactly one matmul (or batched matmul)
//      -> gemm with epilogue;
//   2. a region whose reductions all run along the last axis of one row
//      space and are consumed through broadcasts -> one row program
//      (softmax, normalisations, a root reduction over the last axis);
//   3. a root reduction over another axis -> reduce.column;
//   4. anything else -> one pointwise kernel.
// Sub-results a region cannot absorb (other reductions, other matmuls,
// non-trivial matmul operands) are materialised once each into temporaries
// and read by the consuming kernel; the reference re-materialises a shared
// reduction at every use.
//
// Plans are cached by the graph's canonical key; a cache hit does no string
// work beyond building the key, and launches kernels whose modules were
// loaded once.

#include "codegen.hpp"
#include "graph.hpp"
#include "runtime.hpp"

#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace porch::plan {

    struct arg_ref {
        enum class kind { input, temp, output };
        kind what = kind::input;
        int index = 0;
    };

    struct step {
        cg::kernel_code code;
        arg_ref dest;
        std::shared_ptr<const rt::code_object> object;
        rt::kernel_handle kernel;
    };

    struct graph_plan {
        std::vector<int64_t> out_shape;
        int n_inputs = 0;
        std::vector<int64_t> input_elems; // floats each input slot must hold
        std::vector<int64_t> temp_elems;
        std::vector<step> steps;
        double codegen_ms = 0.0;
        double compile_ms = 0.0;

        std::mutex load_mutex;
        bool loaded = false;

        [[nodiscard]] std::string describe() const;
    };

    // Plans (code generation only).
    std::shared_ptr<graph_plan> build(const ir::graph& g, int compute_units);
    // hiprtc for every step (no device needed).
    void compile(graph_plan& plan);

    // Cached plan for a compacted graph (plans and compiles on a miss).
    std::shared_ptr<graph_plan> lookup(const ir::graph& g, bool* hit);
    void clear_cache();

    // Launches the plan on the calling thread's stream.  `inputs[i]` backs
    // input slot i.  Returns the output buffer (no allocation when the
    // output is empty).
    // `start` / `stop` (optional) are attached to the first and the last
    // kernel launch.
    std::shared_ptr<rt::buffer_state> run(
        graph_plan& plan, const std::vector<rt::buffer_state*>& inputs,
        const std::function<std::shared_ptr<rt::buffer_state>(size_t)>& allocate,
        hip::event_t start = nullptr, hip::event_t stop = nullptr
    );

    // Byte offset of each temporary in one device region (256-byte
    // aligned, in plan order); *total receives the region's size.
    std::vector<size_t> workspace_layout(const graph_plan& plan, size_t* total);

    // run() into the existing buffer `out`, with the temporaries at
    // `workspace` (laid out by workspace_layout; at most `workspace_bytes`):
    // allocates no device memory.  Throws invalid_argument when `out` or the
    // workspace is too small.
    void run_in_workspace(graph_plan& plan, const std::vector<rt::buffer_state*>& inputs,
                          rt::buffer_state& out, char* workspace, size_t workspace_bytes);

} // namespace porch::plan
