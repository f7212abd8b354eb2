#pragma once

// Backend selection (reference include/porch/backend.hpp:9-37).  porch has a
// single GPU JIT backend; its enumerator keeps the reference spelling
// `cuda_jit` (with `hip_jit` as a synonym) so existing programs compile, and
// it reports the name "cuda-jit" that those programs check.

#include "porch/tensor.hpp"

#include <string_view>

namespace porch {

    enum class backend_kind {
        cuda_jit,
        hip_jit = cuda_jit,
    };

    class backend {
      public:
        constexpr explicit backend(
            backend_kind kind = backend_kind::cuda_jit
        ) noexcept
            : kind_(kind) {}

        [[nodiscard]] constexpr backend_kind kind() const noexcept {
            return kind_;
        }
        [[nodiscard]] constexpr bool is_cuda_jit() const noexcept {
            return kind_ == backend_kind::cuda_jit;
        }
        [[nodiscard]] constexpr bool is_hip_jit() const noexcept {
            return is_cuda_jit();
        }

        friend constexpr bool operator==(
            const backend&, const backend&
        ) noexcept = default;

      private:
        backend_kind kind_;
    };

    [[nodiscard]] backend backend_for(device placement) noexcept;
    [[nodiscard]] bool is_backend_available(backend target) noexcept;
    [[nodiscard]] std::string_view backend_name(backend target) noexcept;

} // namespace porch
