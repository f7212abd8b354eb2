// porch::hip_jit — the public runtime API (reference
// include/porch/cuda_jit.hpp:16-97, src/cuda_jit.cpp:617-948) over the HIP
// runtime in runtime.cpp.

#include "internal.hpp"

#include <cstring>
#include <stdexcept>

namespace porch::hip_jit {
    namespace {

        void require_bytes(const device_buffer& buffer, size_t bytes, const char* name) {
            if (buffer.size_bytes() < bytes) {
                throw std::invalid_argument(
                    std::string{name} + " device buffer is too small"
                );
            }
        }

        void launch_reference_geometry(
            std::string_view code_object, std::string_view function,
            const std::vector<const device_buffer*>& inputs, device_buffer& out,
            size_t count, bool one_block_per_output, const char* what
        ) {
            if (count == 0) return;
            for (const device_buffer* input : inputs) {
                if (input == nullptr)
                    throw std::invalid_argument(std::string{what} + " input is null");
                if (input->empty())
                    throw std::invalid_argument(std::string{what} + " input is empty");
            }
            require_bytes(out, count * sizeof(float32_t), "out");
            std::shared_ptr<rt::stream> s = rt::current_stream();
            for (const device_buffer* input : inputs)
                buffer_access::state(*input)->before_read(s);
            buffer_access::state(out)->before_write(s);

            auto object = std::make_shared<rt::code_object>();
            object->bytes.assign(code_object.data(), code_object.size());
            const rt::kernel_handle kernel = rt::load_kernel(object, function);

            std::vector<void*> pointers;
            for (const device_buffer* input : inputs)
                pointers.push_back(buffer_access::state(*input)->ptr);
            pointers.push_back(buffer_access::state(out)->ptr);
            uint64_t element_count = count;
            std::vector<void*> params;
            for (void*& p : pointers) params.push_back(&p);
            params.push_back(&element_count);
            const uint64_t blocks = one_block_per_output ? count : (count + 255) / 256;
            if (blocks > 0x7fffffffULL)
                throw std::invalid_argument("launch grid is too large");
            rt::launch(kernel, static_cast<unsigned>(blocks), 1, 1, 256, 0,
                       params.data(), *s);
            buffer_access::state(out)->after_write(s);
        }

    } // namespace

    device_buffer::device_buffer(size_t bytes) {
        if (bytes != 0) state_ = std::make_shared<device_buffer_state>(bytes);
    }

    bool device_buffer::empty() const noexcept {
        return state_ == nullptr || state_->bytes == 0;
    }

    size_t device_buffer::size_bytes() const noexcept {
        return state_ == nullptr ? 0 : state_->bytes;
    }

    void* device_buffer::device_pointer() const noexcept {
        return state_ == nullptr ? nullptr : state_->ptr;
    }

    compilation_error::compilation_error(std::string log)
        : std::runtime_error(log), log_(std::move(log)) {}

    const std::string& compilation_error::log() const noexcept { return log_; }

    bool is_available() noexcept {
        if (!hip::libraries_present()) return false;
        try {
            (void)rt::device();
            return true;
        }
        catch (...) {
            return false;
        }
    }

    std::string compile_to_ptx(
        std::string_view source, const std::vector<std::string>& options
    ) {
        (void)source;
        (void)options;
        throw std::runtime_error(
            "the HIP JIT backend produces gfx950 code objects, not PTX; use "
            "compile_to_code_object"
        );
    }

    std::string compile_to_code_object(
        std::string_view source, const std::vector<std::string>& options
    ) {
        return rt::compile(source, options)->bytes;
    }

    device_buffer make_device_buffer(std::span<const float32_t> source) {
        device_buffer buffer{source.size_bytes()};
        copy_to_device(buffer, source);
        return buffer;
    }

    void copy_to_device(device_buffer& buffer, std::span<const float32_t> source) {
        if (source.empty()) return;
        require_bytes(buffer, source.size_bytes(), "target");
        std::shared_ptr<rt::stream> s = rt::current_stream();
        device_buffer_state& state = *buffer_access::state(buffer);
        state.before_write(s);
        // Staged through pinned memory, the DMA runs behind the caller;
        // without a staging chunk the copy is direct and waited for.  Either
        // way the source span may be released as soon as this returns.
        if (!rt::upload_staged(state.ptr, source.data(), source.size_bytes(), *s)) {
            const hip::api& h = hip::runtime();
            hip::check(
                h.memcpy_htod_async(state.ptr, source.data(), source.size_bytes(), s->handle()),
                "hipMemcpyHtoDAsync"
            );
            s->synchronize();
        }
        state.after_write(s);
    }

    void copy_to_host(const device_buffer& buffer, std::span<float32_t> target) {
        if (target.empty()) return;
        require_bytes(buffer, target.size_bytes(), "source");
        std::shared_ptr<rt::stream> s = rt::current_stream();
        device_buffer_state& state = *buffer_access::state(buffer);
        state.before_read(s);
        // Large results come back through pinned chunks, pipelined with the
        // copy out of them; small ones (or without a chunk) directly.
        if (target.size_bytes() < (size_t{1} << 20) ||
            !rt::download_staged(target.data(), state.ptr, target.size_bytes(), *s)) {
            const hip::api& h = hip::runtime();
            hip::check(
                h.memcpy_dtoh_async(target.data(), state.ptr, target.size_bytes(), s->handle()),
                "hipMemcpyDtoHAsync"
            );
            s->synchronize();
        }
    }

    void synchronize() { rt::current_stream()->synchronize(); }

    void launch_elementwise_binary(
        std::string_view code_object, std::string_view function,
        std::span<const float32_t> lhs, std::span<const float32_t> rhs,
        std::span<float32_t> out
    ) {
        if (lhs.size() != rhs.size() || lhs.size() != out.size())
            throw std::invalid_argument("GPU elementwise operands must match");
        device_buffer device_lhs = make_device_buffer(lhs);
        device_buffer device_rhs = make_device_buffer(rhs);
        device_buffer device_out{out.size_bytes()};
        launch_elementwise_binary(code_object, function, device_lhs, device_rhs,
                                  device_out, out.size());
        copy_to_host(device_out, out);
    }

    void launch_elementwise_binary(
        std::string_view code_object, std::string_view function,
        const device_buffer& lhs, const device_buffer& rhs, device_buffer& out,
        size_t count
    ) {
        launch_fused_elementwise(code_object, function, {&lhs, &rhs}, out, count);
    }

    void launch_fused_elementwise(
        std::string_view code_object, std::string_view function,
        const std::vector<const device_buffer*>& inputs, device_buffer& out,
        size_t count
    ) {
        launch_reference_geometry(code_object, function, inputs, out, count, false,
                                  "GPU elementwise");
    }

    void launch_fused_reduction(
        std::string_view code_object, std::string_view function,
        const std::vector<const device_buffer*>& inputs, device_buffer& out,
        size_t count
    ) {
        launch_reference_geometry(code_object, function, inputs, out, count, true,
                                  "GPU reduction");
    }

} // namespace porch::hip_jit
