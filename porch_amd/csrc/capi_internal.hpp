#pragma once

// Shared by the translation units of the C ABI (capi.cpp, noalloc.hip).

#include "porch_amd.h"

#include "internal.hpp"
#include "planner.hpp"

#include <functional>
#include <memory>
#include <vector>

struct porch_buffer {
    porch::hip_jit::device_buffer handle;
};

namespace porch::capi {

    // Runs `body`, mapping an exception onto its status code and the calling
    // thread's last error message (porch_last_error).
    porch_status guarded_call(const std::function<void()>& body);

    // The validated and planned graph behind a node table, cached by the
    // table's bytes.
    struct prepared_graph {
        std::shared_ptr<plan::graph_plan> plan; // null: the result is empty
        std::vector<int64_t> out_shape;
        int n_inputs = 0;
        bool hit = false; // served from a cache
    };
    prepared_graph prepare(const porch_graph* graph);

    // The runtime buffers behind the handles (null handles stay null).
    std::vector<rt::buffer_state*> input_states(const porch_buffer* const* inputs, int32_t n_inputs);

    // Writes a result shape as porch_materialize does.
    void write_result_shape(const std::vector<int64_t>& shape, int64_t* out, int32_t capacity,
                            int32_t* rank);

} // namespace porch::capi
