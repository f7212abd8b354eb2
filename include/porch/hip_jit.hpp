#pragma once

// Runtime of the MI355X backend: stream-ordered device buffers, hiprtc
// compilation to gfx950 code objects and raw kernel launches.  Same surface
// as the reference's porch::cuda_jit (include/porch/cuda_jit.hpp:16-97);
// porch/cuda_jit.hpp aliases that name to this namespace so programs
// written against the reference compile unchanged.

#include "porch/types.hpp"

#include <memory>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace porch::hip_jit {

    struct device_buffer_state;

    // Shared handle to a device allocation.  A default or 0-byte buffer owns
    // no memory.  The last handle frees the memory on the stream that
    // produced it, after every other stream that read it.
    class device_buffer {
      public:
        device_buffer() = default;
        explicit device_buffer(size_t bytes);

        [[nodiscard]] bool empty() const noexcept;
        [[nodiscard]] size_t size_bytes() const noexcept;
        // Device address (nullptr when empty); for interop and tests.
        [[nodiscard]] void* device_pointer() const noexcept;

      private:
        friend struct buffer_access;
        std::shared_ptr<device_buffer_state> state_;
    };

    // hiprtc rejected a source; log() is the compiler output.
    class compilation_error : public std::runtime_error {
      public:
        explicit compilation_error(std::string log);

        [[nodiscard]] const std::string& log() const noexcept;

      private:
        std::string log_;
    };

    // True when libamdhip64 and libhiprtc load and device 0 initialises.
    [[nodiscard]] bool is_available() noexcept;

    // AMD GPUs run code objects, not PTX: always throws std::runtime_error
    // (a compile failure of `source` is reported as compilation_error).
    [[nodiscard]] std::string compile_to_ptx(
        std::string_view source, const std::vector<std::string>& options = {}
    );

    // hiprtc -> gfx950 code object (ELF bytes), cached by (source, options).
    [[nodiscard]] std::string compile_to_code_object(
        std::string_view source, const std::vector<std::string>& options = {}
    );

    [[nodiscard]] device_buffer make_device_buffer(
        std::span<const float32_t> source
    );
    void copy_to_device(
        device_buffer& buffer, std::span<const float32_t> source
    );
    void copy_to_host(const device_buffer& buffer, std::span<float32_t> target);
    void synchronize();

    // Launchers with the reference's parameter convention
    // (in0..in{n-1}, out, uint64 count); `code_object` is the output of
    // compile_to_code_object.
    void launch_elementwise_binary(
        std::string_view code_object, std::string_view function,
        std::span<const float32_t> lhs, std::span<const float32_t> rhs,
        std::span<float32_t> out
    );
    void launch_elementwise_binary(
        std::string_view code_object, std::string_view function,
        const device_buffer& lhs, const device_buffer& rhs, device_buffer& out,
        size_t count
    );
    void launch_fused_elementwise(
        std::string_view code_object, std::string_view function,
        const std::vector<const device_buffer*>& inputs, device_buffer& out,
        size_t count
    );
    void launch_fused_reduction(
        std::string_view code_object, std::string_view function,
        const std::vector<const device_buffer*>& inputs, device_buffer& out,
        size_t count
    );

} // namespace porch::hip_jit
