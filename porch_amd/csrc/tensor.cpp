// porch::tensor / porch::tensor_expr — lazy IR recording and
// materialisation (reference src/tensor.cpp:62-122, 1070-1511).
//
// Differences from the reference, all source-compatible:
//   * input nodes own a handle to the tensor they read, so an expression
//     stays valid after the tensors it was built from go out of scope (the
//     reference stores a raw `const tensor*`, src/tensor.cpp:50);
//   * a lazy tensor that has already materialised is referenced by its
//     storage instead of re-inlining (and recomputing) its expression;
//   * the host mirror is allocated on the first data()/cpu() call, not
//     zero-filled at every materialisation (src/tensor.cpp:1019,1073-1075).

#include "internal.hpp"
#include "planner.hpp"

#include "porch/tensor.hpp"

#include <atomic>
#include <chrono>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <unordered_map>

namespace porch {

    struct realized_storage {
        realized_storage(hip_jit::device_buffer buffer, std::vector<float32_t> values,
                         bool current)
            : device_values(std::move(buffer)), host(std::move(values)),
              host_current(current) {}

        hip_jit::device_buffer device_values;
        std::vector<float32_t> host;
        bool host_current = false;
        std::mutex host_mutex;
    };

    struct lazy_materialization {
        explicit lazy_materialization(std::shared_ptr<const tensor_expr::node> e)
            : expression(std::move(e)) {}

        std::shared_ptr<realized_storage> storage();

        std::shared_ptr<const tensor_expr::node> expression;
        std::once_flag once;
        std::shared_ptr<realized_storage> realized;
        std::atomic<bool> done{false};
    };

    struct tensor::state {
        tensor_layout layout;
        device placement;
        std::shared_ptr<realized_storage> realized;
        std::shared_ptr<lazy_materialization> lazy;
        // Strided storage: the values gathered in row-major order, made once
        // on first data().
        std::once_flag dense_once;
        std::shared_ptr<realized_storage> dense;

        state(tensor_layout l, device p) : layout(std::move(l)), placement(p) {}

        [[nodiscard]] std::shared_ptr<realized_storage> storage() const {
            if (realized != nullptr) return realized;
            return lazy->storage();
        }
    };

    namespace detail {
        struct tensor_access {
            using state_t = tensor::state;
            static const std::shared_ptr<tensor::state>& state(const tensor& t) {
                return t.state_;
            }
            static tensor make(std::shared_ptr<tensor::state> s) {
                return tensor(std::move(s));
            }
        };
        struct expr_access {
            static const std::shared_ptr<const tensor_expr::node>& root(
                const tensor_expr& e
            ) {
                return e.root_;
            }
            static tensor_expr make(std::shared_ptr<const tensor_expr::node> n) {
                return tensor_expr(std::move(n));
            }
        };
    } // namespace detail

    using state_t = detail::tensor_access::state_t;

    struct tensor_expr::node {
        ir::op kind = ir::op::input;
        std::optional<tensor> input;
        float32_t scalar = 0.0F;
        std::shared_ptr<const node> lhs;
        std::shared_ptr<const node> rhs;
        std::vector<index_t> shape;
        std::vector<index_t> strides;
        index_t offset = 0;
        size_t axis = 0;
        bool keepdim = false;
    };

    namespace {

        using node_ptr = std::shared_ptr<const tensor_expr::node>;

        node_ptr make_node(ir::op kind, node_ptr lhs = nullptr, node_ptr rhs = nullptr) {
            auto n = std::make_shared<tensor_expr::node>();
            n->kind = kind;
            n->lhs = std::move(lhs);
            n->rhs = std::move(rhs);
            return n;
        }

        index_t normalize_index(index_t index, index_t extent) {
            if (index < 0) index += extent;
            if (index < 0 || index >= extent)
                throw std::out_of_range("tensor index is out of bounds");
            return index;
        }

        index_t normalize_slice_endpoint(index_t index, index_t extent) {
            if (index < 0) index += extent;
            if (index < 0) return 0;
            if (index > extent) return extent;
            return index;
        }

        size_t slice_length(index_t start, index_t stop, index_t step) {
            if (step <= 0) throw std::invalid_argument("tensor slice step must be positive");
            if (stop <= start) return 0;
            return static_cast<size_t>((stop - start + step - 1) / step);
        }

        bool is_contiguous_layout(std::span<const index_t> shape,
                                  std::span<const index_t> strides) {
            if (shape.size() != strides.size()) return false;
            index_t expected = 1;
            for (size_t d = shape.size(); d > 0; --d) {
                if (strides[d - 1] != expected) return false;
                expected *= shape[d - 1];
            }
            return true;
        }

        // Floats of storage a layout reaches: offset + sum (extent-1)*stride + 1.
        size_t storage_span(const tensor_layout& layout) {
            if (layout.numel() == 0) return 0;
            index_t last = layout.storage_offset();
            for (size_t d = 0; d < layout.rank(); ++d)
                last += (layout.shape()[d] - 1) * layout.strides()[d];
            return static_cast<size_t>(last) + 1;
        }

        // The input node of a tensor's storage (for strided storage, the
        // flat span its layout reaches).
        node_ptr storage_node(const tensor& value) {
            auto n = std::make_shared<tensor_expr::node>();
            n->kind = ir::op::input;
            n->input = value;
            return n;
        }

        // The DAG of an expression as a node table, inputs in first-visit
        // order (lhs before rhs), as the reference numbers them
        // (src/tensor.cpp:261-277).
        struct graph_builder {
            ir::graph g;
            std::unordered_map<const tensor_expr::node*, int> index;
            std::unordered_map<const state_t*, int> slot_of;
            std::vector<tensor> inputs;
            std::optional<device> placement;

            int visit(const node_ptr& root) {
                struct frame {
                    const tensor_expr::node* n;
                    bool expanded;
                };
                std::vector<frame> stack{{root.get(), false}};
                while (!stack.empty()) {
                    frame f = stack.back();
                    stack.pop_back();
                    if (index.count(f.n)) continue;
                    if (!f.expanded) {
                        stack.push_back({f.n, true});
                        // rhs pushed first so lhs is visited (and numbered)
                        // first.
                        if (f.n->rhs && !index.count(f.n->rhs.get()))
                            stack.push_back({f.n->rhs.get(), false});
                        if (f.n->lhs && !index.count(f.n->lhs.get()))
                            stack.push_back({f.n->lhs.get(), false});
                        continue;
                    }
                    ir::node out;
                    out.kind = f.n->kind;
                    out.lhs = f.n->lhs ? index.at(f.n->lhs.get()) : -1;
                    out.rhs = f.n->rhs ? index.at(f.n->rhs.get()) : -1;
                    out.scalar = f.n->scalar;
                    out.axis = static_cast<int64_t>(f.n->axis);
                    out.keepdim = f.n->keepdim;
                    out.offset = f.n->offset;
                    out.strides = f.n->strides;
                    if (f.n->kind == ir::op::input) {
                        const tensor& t = *f.n->input;
                        const state_t* st = detail::tensor_access::state(t).get();
                        if (!placement) placement = t.placement();
                        else if (*placement != t.placement())
                            throw std::invalid_argument("tensor expression devices must match");
                        auto found = slot_of.find(st);
                        if (found == slot_of.end()) {
                            found = slot_of.emplace(st, static_cast<int>(inputs.size())).first;
                            inputs.push_back(t);
                        }
                        out.input = found->second;
                        if (t.is_contiguous())
                            out.shape.assign(t.shape().begin(), t.shape().end());
                        else // strided storage, read through a slice above
                            out.shape = {static_cast<index_t>(storage_span(t.layout()))};
                        g.n_inputs = static_cast<int>(inputs.size());
                    }
                    else {
                        out.shape = f.n->shape;
                    }
                    index.emplace(f.n, static_cast<int>(g.nodes.size()));
                    g.nodes.push_back(std::move(out));
                }
                return index.at(root.get());
            }
        };

        tensor make_realized(std::vector<index_t> shape, hip_jit::device_buffer buffer,
                             std::vector<float32_t> host, bool host_current, device placement) {
            auto st = std::make_shared<state_t>(tensor_layout{std::move(shape)}, placement);
            st->realized = std::make_shared<realized_storage>(
                std::move(buffer), std::move(host), host_current
            );
            return detail::tensor_access::make(std::move(st));
        }

        tensor materialize_node(const node_ptr& root) {
            const auto start = std::chrono::steady_clock::now();
            graph_builder b;
            (void)b.visit(root);
            ir::infer(b.g);
            if (b.inputs.empty())
                throw std::invalid_argument("tensor expression must reference at least one tensor");
            const ir::node& r = b.g.at(b.g.root());
            if (r.is_scalar)
                throw std::invalid_argument("scalar expression cannot materialize to a tensor");
            const size_t count = ir::checked_numel(r.out);
            const device placement = *b.placement;
            if (count == 0) {
                return make_realized(r.out, hip_jit::device_buffer{}, {}, true, placement);
            }
            const ir::graph compacted = ir::compact(b.g);
            bool hit = false;
            std::shared_ptr<plan::graph_plan> p = plan::lookup(compacted, &hit);

            std::vector<std::shared_ptr<realized_storage>> storages;
            std::vector<rt::buffer_state*> buffers;
            storages.reserve(b.inputs.size());
            for (const tensor& t : b.inputs) {
                storages.push_back(detail::tensor_access::state(t)->storage());
                buffers.push_back(
                    hip_jit::buffer_access::state(storages.back()->device_values).get()
                );
            }
            std::shared_ptr<rt::buffer_state> out = plan::run(
                *p, buffers,
                [](size_t bytes) -> std::shared_ptr<rt::buffer_state> {
                    return std::make_shared<hip_jit::device_buffer_state>(bytes);
                }
            );
            hip_jit::device_buffer result = hip_jit::buffer_access::wrap(
                std::static_pointer_cast<hip_jit::device_buffer_state>(out)
            );
            const double ms = rt::elapsed_ms(start);
            {
                std::scoped_lock lock{rt::counters_mutex()};
                if (hit) {
                    rt::counters().plan_hits += 1;
                    rt::counters().last_hit_us = ms * 1000.0;
                }
                else {
                    rt::counters().plan_misses += 1;
                    rt::counters().last_miss_ms = ms;
                }
            }
            return make_realized(r.out, std::move(result), {}, false, placement);
        }

        std::vector<index_t> infer_shape(const node_ptr& root, bool* is_scalar,
                                         bool* has_input, device* placement) {
            graph_builder b;
            (void)b.visit(root);
            ir::infer(b.g);
            const ir::node& r = b.g.at(b.g.root());
            if (is_scalar) *is_scalar = r.is_scalar;
            if (has_input) *has_input = !b.inputs.empty();
            if (placement && b.placement) *placement = *b.placement;
            return r.out;
        }

    } // namespace

    std::shared_ptr<realized_storage> lazy_materialization::storage() {
        std::call_once(once, [this] {
            tensor materialized = materialize_node(expression);
            realized = detail::tensor_access::state(materialized)->realized;
            done.store(true, std::memory_order_release);
        });
        return realized;
    }

    // ------------------------------------------------------------------
    // tensor_index, tensor_layout
    // ------------------------------------------------------------------

    tensor_index::tensor_index(index_t index) : kind_(kind::index), index_(index) {}
    tensor_index::tensor_index(slice range) : kind_(kind::slice), slice_(range) {}
    tensor_index::tensor_index(all_t) : kind_(kind::all) {}

    tensor_layout::tensor_layout(std::vector<index_t> shape)
        : shape_(std::move(shape)), strides_(ir::contiguous_strides(shape_)) {
        (void)ir::checked_numel(shape_);
    }

    tensor_layout::tensor_layout(std::vector<index_t> shape, std::vector<index_t> strides,
                                 index_t storage_offset)
        : shape_(std::move(shape)), strides_(std::move(strides)),
          storage_offset_(storage_offset) {
        if (shape_.size() != strides_.size())
            throw std::invalid_argument("tensor layout rank mismatch");
        if (storage_offset_ < 0)
            throw std::invalid_argument("tensor layout offset must be non-negative");
        for (const index_t stride : strides_) {
            if (stride < 0)
                throw std::invalid_argument("tensor layout strides must be non-negative");
        }
        (void)ir::checked_numel(shape_);
    }

    std::span<const index_t> tensor_layout::shape() const noexcept { return shape_; }
    std::span<const index_t> tensor_layout::strides() const noexcept { return strides_; }
    index_t tensor_layout::storage_offset() const noexcept { return storage_offset_; }
    size_t tensor_layout::rank() const noexcept { return shape_.size(); }
    size_t tensor_layout::numel() const noexcept {
        size_t count = 1;
        for (const index_t e : shape_) count *= static_cast<size_t>(e);
        return count;
    }
    bool tensor_layout::is_contiguous() const noexcept {
        return storage_offset_ == 0 && is_contiguous_layout(shape_, strides_);
    }

    // ------------------------------------------------------------------
    // tensor
    // ------------------------------------------------------------------

    tensor::tensor(std::shared_ptr<state> initial_state) noexcept
        : state_(std::move(initial_state)) {}

    tensor::tensor(std::vector<index_t> shape, std::vector<float32_t> values, device placement)
        : state_(std::make_shared<state>(tensor_layout{std::move(shape)}, placement)) {
        if (values.size() != state_->layout.numel())
            throw std::invalid_argument("tensor data size does not match shape");
        hip_jit::device_buffer buffer = hip_jit::make_device_buffer(values);
        state_->realized =
            std::make_shared<realized_storage>(std::move(buffer), std::move(values), true);
    }

    tensor::tensor(std::vector<index_t> shape, std::vector<float32_t> values,
                   cuda_jit::device_buffer device_values, device placement)
        : state_(std::make_shared<state>(tensor_layout{std::move(shape)}, placement)) {
        if (values.size() != state_->layout.numel())
            throw std::invalid_argument("tensor data size does not match shape");
        if (device_values.size_bytes() < values.size() * sizeof(float32_t))
            throw std::invalid_argument("tensor device storage is too small");
        state_->realized = std::make_shared<realized_storage>(
            std::move(device_values), std::move(values), true
        );
    }

    std::span<const index_t> tensor::shape() const noexcept { return state_->layout.shape(); }
    std::span<const index_t> tensor::strides() const noexcept {
        return state_->layout.strides();
    }
    const tensor_layout& tensor::layout() const noexcept { return state_->layout; }
    index_t tensor::storage_offset() const noexcept { return state_->layout.storage_offset(); }
    bool tensor::is_contiguous() const noexcept { return state_->layout.is_contiguous(); }
    size_t tensor::rank() const noexcept { return state_->layout.rank(); }
    size_t tensor::numel() const noexcept { return state_->layout.numel(); }
    device tensor::placement() const noexcept { return state_->placement; }

    tensor::tensor(tensor_layout layout, cuda_jit::device_buffer storage, device placement)
        : state_(std::make_shared<state>(std::move(layout), placement)) {
        if (storage.size_bytes() < storage_span(state_->layout) * sizeof(float32_t))
            throw std::invalid_argument("tensor device storage is too small");
        state_->realized = std::make_shared<realized_storage>(
            std::move(storage), std::vector<float32_t>{}, false
        );
    }

    std::span<const float32_t> tensor::data() const {
        std::shared_ptr<realized_storage> storage;
        if (state_->layout.is_contiguous()) {
            storage = state_->storage();
        }
        else {
            std::call_once(state_->dense_once, [this] {
                const tensor dense = materialize(tensor_expr{*this});
                state_->dense = detail::tensor_access::state(dense)->storage();
            });
            storage = state_->dense;
        }
        std::scoped_lock lock{storage->host_mutex};
        if (!storage->host_current) {
            storage->host.resize(numel());
            hip_jit::copy_to_host(storage->device_values, storage->host);
            storage->host_current = true;
        }
        return storage->host;
    }

    std::vector<float32_t> tensor::cpu() const {
        const std::span<const float32_t> host = data();
        return {host.begin(), host.end()};
    }

    const cuda_jit::device_buffer& tensor::device_data() const {
        return state_->storage()->device_values;
    }

    const tensor& tensor::realize() const {
        (void)state_->storage();
        return *this;
    }

    void tensor::synchronize() const {
        std::shared_ptr<realized_storage> storage = state_->storage();
        std::shared_ptr<rt::stream> s = rt::current_stream();
        if (!storage->device_values.empty()) {
            hip_jit::buffer_access::state(storage->device_values)->before_read(s);
        }
        s->synchronize();
    }

    tensor_expr tensor::operator[](std::initializer_list<tensor_index> indices) const {
        if (indices.size() > rank()) throw std::invalid_argument("too many tensor indices");
        std::vector<index_t> out_shape;
        std::vector<index_t> out_strides;
        index_t offset = storage_offset();
        size_t dim = 0;
        for (const tensor_index& index : indices) {
            const index_t extent = shape()[dim];
            const index_t stride = strides()[dim];
            switch (index.kind_) {
                case tensor_index::kind::index:
                    offset += normalize_index(index.index_, extent) * stride;
                    break;
                case tensor_index::kind::slice: {
                    const index_t start = normalize_slice_endpoint(index.slice_.start, extent);
                    const index_t stop = normalize_slice_endpoint(index.slice_.stop, extent);
                    const size_t length = slice_length(start, stop, index.slice_.step);
                    offset += start * stride;
                    out_shape.push_back(static_cast<index_t>(length));
                    out_strides.push_back(stride * index.slice_.step);
                    break;
                }
                case tensor_index::kind::all:
                    out_shape.push_back(extent);
                    out_strides.push_back(stride);
                    break;
            }
            ++dim;
        }
        for (; dim < rank(); ++dim) {
            out_shape.push_back(shape()[dim]);
            out_strides.push_back(strides()[dim]);
        }
        (void)ir::checked_numel(out_shape);
        auto n = std::make_shared<tensor_expr::node>();
        n->kind = ir::op::slice;
        // Offsets and strides above are in storage elements: over strided
        // storage the slice applies to the raw storage, not to the view.
        n->lhs = is_contiguous() ? detail::expr_access::root(tensor_expr{*this})
                                 : storage_node(*this);
        n->shape = std::move(out_shape);
        n->strides = std::move(out_strides);
        n->offset = offset;
        return detail::expr_access::make(std::move(n));
    }

    tensor_expr tensor::operator[](tensor_index index) const { return (*this)[{index}]; }

    // ------------------------------------------------------------------
    // tensor_expr
    // ------------------------------------------------------------------

    tensor_expr::tensor_expr(const tensor& value) {
        const std::shared_ptr<state_t>& st = detail::tensor_access::state(value);
        if (st->lazy != nullptr && !st->lazy->done.load(std::memory_order_acquire)) {
            root_ = st->lazy->expression;
            return;
        }
        if (!value.is_contiguous()) {
            // Strided storage: the view is a slice of the raw storage.
            const tensor_layout& layout = value.layout();
            auto view = std::make_shared<tensor_expr::node>();
            view->kind = ir::op::slice;
            view->lhs = storage_node(value);
            view->shape.assign(layout.shape().begin(), layout.shape().end());
            view->strides.assign(layout.strides().begin(), layout.strides().end());
            view->offset = layout.storage_offset();
            root_ = std::move(view);
            return;
        }
        root_ = storage_node(value);
    }

    tensor_expr::tensor_expr(float32_t value) {
        auto n = std::make_shared<tensor_expr::node>();
        n->kind = ir::op::scalar;
        n->scalar = value;
        root_ = std::move(n);
    }

    tensor_expr::tensor_expr(std::shared_ptr<const node> root) : root_(std::move(root)) {}

    tensor tensor_expr::eval() const { return materialize(*this); }

    std::vector<index_t> tensor_expr::shape() const {
        bool scalar = false;
        std::vector<index_t> s = infer_shape(root_, &scalar, nullptr, nullptr);
        if (scalar) return {};
        return s;
    }

    size_t tensor_expr::rank() const { return shape().size(); }

    size_t tensor_expr::numel() const { return ir::checked_numel(shape()); }

    tensor_expr::operator tensor() const {
        bool scalar = false;
        bool has_input = false;
        device placement{};
        std::vector<index_t> s = infer_shape(root_, &scalar, &has_input, &placement);
        if (!has_input)
            throw std::invalid_argument("tensor expression must reference at least one tensor");
        if (scalar)
            throw std::invalid_argument("scalar expression cannot convert to a tensor");
        (void)ir::checked_numel(s);
        auto st = std::make_shared<state_t>(tensor_layout{std::move(s)}, placement);
        st->lazy = std::make_shared<lazy_materialization>(root_);
        return detail::tensor_access::make(std::move(st));
    }

    // ------------------------------------------------------------------
    // free functions
    // ------------------------------------------------------------------

    tensor full(std::vector<index_t> shape, float32_t value, device placement) {
        const size_t count = ir::checked_numel(shape);
        return tensor{std::move(shape), std::vector<float32_t>(count, value), placement};
    }

    tensor zeros(std::vector<index_t> shape, device placement) {
        return full(std::move(shape), 0.0F, placement);
    }

    tensor add(const tensor& lhs, const tensor& rhs) {
        return materialize(tensor_expr{lhs} + tensor_expr{rhs});
    }
    tensor subtract(const tensor& lhs, const tensor& rhs) {
        return materialize(tensor_expr{lhs} - tensor_expr{rhs});
    }
    tensor multiply(const tensor& lhs, const tensor& rhs) {
        return materialize(tensor_expr{lhs} * tensor_expr{rhs});
    }
    tensor divide(const tensor& lhs, const tensor& rhs) {
        return materialize(tensor_expr{lhs} / tensor_expr{rhs});
    }

    namespace {
        tensor_expr binary(ir::op kind, const tensor_expr& lhs, const tensor_expr& rhs) {
            return detail::expr_access::make(make_node(
                kind, detail::expr_access::root(lhs), detail::expr_access::root(rhs)
            ));
        }
        tensor_expr unary(ir::op kind, const tensor_expr& value) {
            return detail::expr_access::make(make_node(kind, detail::expr_access::root(value)));
        }
        tensor_expr with_shape(ir::op kind, const tensor_expr& value,
                               std::vector<index_t> shape) {
            auto n = std::make_shared<tensor_expr::node>();
            n->kind = kind;
            n->lhs = detail::expr_access::root(value);
            n->shape = std::move(shape);
            return detail::expr_access::make(std::move(n));
        }
        tensor_expr with_axis(ir::op kind, const tensor_expr& value, size_t axis,
                              bool keepdim) {
            auto n = std::make_shared<tensor_expr::node>();
            n->kind = kind;
            n->lhs = detail::expr_access::root(value);
            n->axis = axis;
            n->keepdim = keepdim;
            return detail::expr_access::make(std::move(n));
        }
    } // namespace

    tensor_expr matmul(tensor_expr lhs, tensor_expr rhs) {
        return binary(ir::op::matmul, lhs, rhs);
    }
    tensor_expr batched_matmul(tensor_expr lhs, tensor_expr rhs) {
        return binary(ir::op::batched_matmul, lhs, rhs);
    }
    tensor_expr reshape(tensor_expr value, std::vector<index_t> shape) {
        return with_shape(ir::op::reshape, value, std::move(shape));
    }
    tensor_expr unsqueeze(tensor_expr value, size_t axis) {
        return with_axis(ir::op::unsqueeze, value, axis, false);
    }
    tensor_expr transpose(tensor_expr value) { return unary(ir::op::transpose, value); }
    tensor_expr permute(tensor_expr value, std::vector<size_t> dims) {
        return with_shape(ir::op::permute, value, std::vector<index_t>(dims.begin(), dims.end()));
    }
    tensor_expr broadcast_to(tensor_expr value, std::vector<index_t> shape) {
        return with_shape(ir::op::broadcast, value, std::move(shape));
    }
    tensor_expr concat(tensor_expr lhs, tensor_expr rhs, size_t axis) {
        auto n = std::make_shared<tensor_expr::node>();
        n->kind = ir::op::concat;
        n->lhs = detail::expr_access::root(lhs);
        n->rhs = detail::expr_access::root(rhs);
        n->axis = axis;
        return detail::expr_access::make(std::move(n));
    }
    tensor_expr sum(tensor_expr value, size_t axis, bool keepdim) {
        return with_axis(ir::op::sum, value, axis, keepdim);
    }
    tensor_expr max(tensor_expr value, size_t axis, bool keepdim) {
        return with_axis(ir::op::max, value, axis, keepdim);
    }
    tensor_expr maximum(tensor_expr lhs, tensor_expr rhs) {
        return binary(ir::op::maximum, lhs, rhs);
    }
    tensor_expr minimum(tensor_expr lhs, tensor_expr rhs) {
        return binary(ir::op::minimum, lhs, rhs);
    }
    tensor_expr exp(tensor_expr value) { return unary(ir::op::exp, value); }
    tensor_expr reciprocal(tensor_expr value) { return unary(ir::op::reciprocal, value); }

    tensor materialize(const tensor_expr& expression) {
        return materialize_node(detail::expr_access::root(expression));
    }

    tensor_expr operator+(tensor_expr lhs, tensor_expr rhs) {
        return binary(ir::op::add, lhs, rhs);
    }
    tensor_expr operator-(tensor_expr lhs, tensor_expr rhs) {
        return binary(ir::op::subtract, lhs, rhs);
    }
    tensor_expr operator*(tensor_expr lhs, tensor_expr rhs) {
        return binary(ir::op::multiply, lhs, rhs);
    }
    tensor_expr operator/(tensor_expr lhs, tensor_expr rhs) {
        return binary(ir::op::divide, lhs, rhs);
    }

} // namespace porch
