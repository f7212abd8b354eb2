#pragma once

// Internal access between the public C++ API, the runtime and the C ABI.

#include "porch/hip_jit.hpp"
#include "porch/tensor.hpp"
#include "runtime.hpp"

#include <memory>

namespace porch::hip_jit {

    // The state behind a device_buffer handle.
    struct device_buffer_state : rt::buffer_state {
        using rt::buffer_state::buffer_state;
    };

    struct buffer_access {
        static const std::shared_ptr<device_buffer_state>& state(
            const device_buffer& buffer
        ) {
            return buffer.state_;
        }
        static device_buffer wrap(std::shared_ptr<device_buffer_state> state) {
            device_buffer buffer;
            buffer.state_ = std::move(state);
            return buffer;
        }
    };

} // namespace porch::hip_jit
