#pragma once

// porch's tensor API (reference include/porch/tensor.hpp:11-225), re-authored
// for the MI355X backend with the same declarations so programs written
// against the reference compile and link unchanged.
//
// A `tensor` is a 16-byte shared handle.  Its state is either realized
// storage (a device buffer plus an on-demand host mirror) or a pending
// expression that materializes exactly once.  A `tensor_expr` is an
// immutable DAG of IR nodes; arithmetic, views, reductions and matmul only
// record nodes.  Materialization plans the DAG into fused gfx950 kernels,
// compiles them with hiprtc (cached by graph hash) and launches them on the
// calling thread's stream.

#include "porch/cuda_jit.hpp"
#include "porch/types.hpp"

#include <initializer_list>
#include <memory>
#include <span>
#include <vector>

namespace porch {

    class tensor_expr;

    namespace detail {
        struct tensor_access;
        struct expr_access;
    } // namespace detail

    // A GPU ordinal.  porch places every tensor on a GPU; the ordinal is
    // placement metadata and expressions require equal placements.
    class device {
      public:
        constexpr explicit device(int ordinal = 0) noexcept
            : ordinal_(ordinal) {}

        [[nodiscard]] constexpr int ordinal() const noexcept {
            return ordinal_;
        }
        // Reference spelling of "this is a GPU device"; always true.
        [[nodiscard]] constexpr bool is_cuda() const noexcept { return true; }
        [[nodiscard]] constexpr bool is_gpu() const noexcept { return true; }

        friend constexpr bool operator==(
            const device&, const device&
        ) noexcept = default;

      private:
        int ordinal_;
    };

    struct all_t {};

    inline constexpr all_t all{};

    // Half-open range [start, stop) with a positive step; negative
    // endpoints count from the end and are clamped to the extent.
    struct slice {
        index_t start;
        index_t stop;
        index_t step = 1;
    };

    // One subscript of operator[]: an integer (drops the dimension), a
    // slice, or `all`.
    class tensor_index {
      public:
        tensor_index(index_t index);
        tensor_index(slice range);
        tensor_index(all_t marker);

      private:
        friend class tensor;

        enum class kind {
            index,
            slice,
            all,
        };

        kind kind_;
        index_t index_ = 0;
        slice slice_{0, 0, 1};
    };

    class tensor_layout {
      public:
        explicit tensor_layout(std::vector<index_t> shape);
        tensor_layout(
            std::vector<index_t> shape, std::vector<index_t> strides,
            index_t storage_offset = 0
        );

        [[nodiscard]] std::span<const index_t> shape() const noexcept;
        [[nodiscard]] std::span<const index_t> strides() const noexcept;
        [[nodiscard]] index_t storage_offset() const noexcept;
        [[nodiscard]] size_t rank() const noexcept;
        [[nodiscard]] size_t numel() const noexcept;
        [[nodiscard]] bool is_contiguous() const noexcept;

      private:
        std::vector<index_t> shape_;
        std::vector<index_t> strides_;
        index_t storage_offset_ = 0;
    };

    class tensor {
      public:
        tensor(
            std::vector<index_t> shape, std::vector<float32_t> values,
            device placement = device{}
        );
        tensor(
            std::vector<index_t> shape, std::vector<float32_t> values,
            cuda_jit::device_buffer device_values, device placement = device{}
        );
        // A realised tensor over existing device storage, read through
        // `layout` (element strides, possibly zero, and an offset).  An
        // extension: the reference rejects non-contiguous storage
        // (src/tensor.cpp:1193-1197).  The storage is shared, not copied;
        // expressions read it in place, and data() gathers the values in
        // row-major order on the device.
        tensor(
            tensor_layout layout, cuda_jit::device_buffer storage,
            device placement = device{}
        );

        [[nodiscard]] std::span<const index_t> shape() const noexcept;
        [[nodiscard]] std::span<const index_t> strides() const noexcept;
        [[nodiscard]] const tensor_layout& layout() const noexcept;
        [[nodiscard]] index_t storage_offset() const noexcept;
        [[nodiscard]] bool is_contiguous() const noexcept;
        [[nodiscard]] size_t rank() const noexcept;
        [[nodiscard]] size_t numel() const noexcept;
        [[nodiscard]] device placement() const noexcept;
        [[nodiscard]] std::span<const float32_t> data() const;
        [[nodiscard]] std::vector<float32_t> cpu() const;
        [[nodiscard]] const cuda_jit::device_buffer& device_data() const;
        const tensor& realize() const;
        void synchronize() const;
        [[nodiscard]] tensor_expr operator[](
            std::initializer_list<tensor_index> indices
        ) const;
        [[nodiscard]] tensor_expr operator[](tensor_index index) const;

      private:
        friend struct detail::tensor_access;
        friend class tensor_expr;

        struct state;

        explicit tensor(std::shared_ptr<state> initial_state) noexcept;

        std::shared_ptr<state> state_;
    };

    class tensor_expr {
      public:
        struct node;

        tensor_expr(const tensor& value);
        tensor_expr(float32_t value);

        [[nodiscard]] tensor eval() const;
        [[nodiscard]] std::vector<index_t> shape() const;
        [[nodiscard]] size_t rank() const;
        [[nodiscard]] size_t numel() const;

        operator tensor() const;

      private:
        friend struct detail::expr_access;

        explicit tensor_expr(std::shared_ptr<const node> root);

        std::shared_ptr<const node> root_;
    };

    [[nodiscard]] tensor full(
        std::vector<index_t> shape, float32_t value, device placement = device{}
    );
    [[nodiscard]] tensor zeros(
        std::vector<index_t> shape, device placement = device{}
    );
    [[nodiscard]] tensor add(const tensor& lhs, const tensor& rhs);
    [[nodiscard]] tensor subtract(const tensor& lhs, const tensor& rhs);
    [[nodiscard]] tensor multiply(const tensor& lhs, const tensor& rhs);
    [[nodiscard]] tensor divide(const tensor& lhs, const tensor& rhs);
    [[nodiscard]] tensor_expr matmul(tensor_expr lhs, tensor_expr rhs);
    // [B, M, K] @ [B, K, N] -> [B, M, N]: matmul per batch entry.  An
    // extension with no counterpart in the reference (whose matmul is
    // rank-2 only); broadcast_to a rank-2 operand to share it across the
    // batch without copying it.
    [[nodiscard]] tensor_expr batched_matmul(tensor_expr lhs, tensor_expr rhs);
    [[nodiscard]] tensor_expr reshape(
        tensor_expr value, std::vector<index_t> shape
    );
    [[nodiscard]] tensor_expr unsqueeze(tensor_expr value, size_t axis);
    [[nodiscard]] tensor_expr transpose(tensor_expr value);
    // Rank-N axis permutation: output dimension i is dimension dims[i] of
    // value.  An extension with no counterpart in the reference (whose
    // transpose is rank-2 only); a pure index map, so it fuses like
    // transpose.
    [[nodiscard]] tensor_expr permute(tensor_expr value, std::vector<size_t> dims);
    [[nodiscard]] tensor_expr broadcast_to(
        tensor_expr value, std::vector<index_t> shape
    );
    [[nodiscard]] tensor_expr concat(
        tensor_expr lhs, tensor_expr rhs, size_t axis
    );
    [[nodiscard]] tensor_expr sum(
        tensor_expr value, size_t axis, bool keepdim = false
    );
    [[nodiscard]] tensor_expr max(
        tensor_expr value, size_t axis, bool keepdim = false
    );
    [[nodiscard]] tensor_expr maximum(tensor_expr lhs, tensor_expr rhs);
    [[nodiscard]] tensor_expr minimum(tensor_expr lhs, tensor_expr rhs);
    [[nodiscard]] tensor_expr exp(tensor_expr value);
    [[nodiscard]] tensor_expr reciprocal(tensor_expr value);

    [[nodiscard]] tensor materialize(const tensor_expr& expression);

    [[nodiscard]] tensor_expr operator+(tensor_expr lhs, tensor_expr rhs);
    [[nodiscard]] tensor_expr operator-(tensor_expr lhs, tensor_expr rhs);
    [[nodiscard]] tensor_expr operator*(tensor_expr lhs, tensor_expr rhs);
    [[nodiscard]] tensor_expr operator/(tensor_expr lhs, tensor_expr rhs);

} // namespace porch
