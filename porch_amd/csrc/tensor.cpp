// porch::tensor / porch::tensor_expr: lazy IR recording and
// materialisation, behind the reference's public declarations
// (include/porch/tensor.hpp; behaviour of src/tensor.cpp:1070-1511).
//
// A tensor's state is a layout, a placement and a value cell: device values
// (with a host copy made on demand), or a recorded graph that produces them
// on first use.  Differences from the reference, all source-compatible:
//   * input nodes own a handle to the tensor they read, so an expression
//     stays valid after the tensors it was built from go out of scope (the
//     reference stores a raw `const tensor*`, src/tensor.cpp:50);
//   * once a recorded graph has run, it is dropped (releasing the tensors
//     it read), and expressions over the tensor read its values instead of
//     re-inlining and recomputing the graph;
//   * no host mirror is allocated at materialisation (the reference
//     zero-fills one each time, src/tensor.cpp:1019,1073-1075): data()
//     fetches one on first use, and cpu() copies straight from the device
//     into the vector it returns when no mirror exists;
//   * indexing restricts the tensor's strided view of its storage one
//     subscript at a time (integers fix an axis, ranges narrow it).

#include "internal.hpp"
#include "planner.hpp"

#include "porch/tensor.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <memory>
#include <mutex>
#include <optional>
#include <span>
#include <stdexcept>
#include <unordered_map>

namespace porch {

    using node_ptr = std::shared_ptr<const tensor_expr::node>;

    namespace {

        // Values resident in device memory.  The host copy is either given
        // at construction (the values a tensor was built from) or fetched
        // from the device on first request and kept; a fetched copy is
        // left uninitialised until the transfer fills it.
        class resident_values {
          public:
            explicit resident_values(hip_jit::device_buffer memory) : memory_(std::move(memory)) {}
            resident_values(hip_jit::device_buffer memory, std::vector<float32_t> host)
                : memory_(std::move(memory)), given_(std::move(host)), host_(given_), host_ready_(true) {}

            [[nodiscard]] const hip_jit::device_buffer& memory() const noexcept { return memory_; }

            // The first `count` values in host memory.
            std::span<const float32_t> host(size_t count) {
                std::scoped_lock hold{fetch_};
                if (!host_ready_) {
                    fetched_.reset(new float32_t[count]);
                    const std::span<float32_t> target{fetched_.get(), count};
                    hip_jit::copy_to_host(memory_, target);
                    host_ = target;
                    host_ready_ = true;
                }
                return host_;
            }

            // The first `count` values as a new vector: from the host copy
            // if there is one, else transferred straight into the vector
            // (no host copy is kept).
            std::vector<float32_t> copy(size_t count) {
                {
                    std::scoped_lock hold{fetch_};
                    if (host_ready_) return {host_.begin(), host_.end()};
                }
                std::vector<float32_t> out(count);
                hip_jit::copy_to_host(memory_, out);
                return out;
            }

          private:
            hip_jit::device_buffer memory_;
            std::mutex fetch_;
            std::vector<float32_t> given_;
            std::unique_ptr<float32_t[]> fetched_;
            std::span<const float32_t> host_;
            bool host_ready_ = false;
        };

        using values_ptr = std::shared_ptr<resident_values>;

        values_ptr run_graph(const node_ptr& root);

        // What a tensor handle stands for: device values, or a recorded
        // graph that produces them on first use.  The graph runs once,
        // on whichever thread asks first; a run that throws leaves it
        // recorded, so the next use runs it again.  Once the values exist
        // the graph is dropped, releasing the tensors it read.
        class value_cell {
          public:
            explicit value_cell(values_ptr values) : values_(std::move(values)), ready_(true) {}
            explicit value_cell(node_ptr graph) : graph_(std::move(graph)) {}

            values_ptr get() {
                if (ready_.load(std::memory_order_acquire)) return values_;
                std::scoped_lock hold{run_};
                if (!ready_.load(std::memory_order_relaxed)) {
                    values_ = run_graph(pending());
                    ready_.store(true, std::memory_order_release);
                    std::scoped_lock hold_graph{graph_lock_};
                    graph_.reset();
                }
                return values_;
            }

            // The recorded graph while its values do not exist yet, else
            // null.  Never waits for a run in progress.
            [[nodiscard]] node_ptr pending() const {
                if (ready_.load(std::memory_order_acquire)) return nullptr;
                std::scoped_lock hold{graph_lock_};
                return graph_;
            }

          private:
            std::mutex run_;
            mutable std::mutex graph_lock_;
            node_ptr graph_;
            values_ptr values_;
            std::atomic<bool> ready_{false};
        };

    } // namespace

    struct tensor::state {
        tensor_layout layout;
        device placement;
        value_cell cell;
        // Over strided storage: the viewed values gathered into row-major
        // order on the device, on the first data() call.
        std::mutex gather_lock;
        values_ptr gathered;

        state(tensor_layout l, device p, values_ptr v)
            : layout(std::move(l)), placement(p), cell(std::move(v)) {}
        state(tensor_layout l, device p, node_ptr graph)
            : layout(std::move(l)), placement(p), cell(std::move(graph)) {}
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

        node_ptr make_node(ir::op kind, node_ptr lhs = nullptr, node_ptr rhs = nullptr) {
            auto n = std::make_shared<tensor_expr::node>();
            n->kind = kind;
            n->lhs = std::move(lhs);
            n->rhs = std::move(rhs);
            return n;
        }

        // A strided view of flat storage: the element at coordinates
        // (c_0, ..., c_{r-1}) sits at `base + sum c_d * step[d]`.
        struct strided_view {
            index_t base = 0;
            std::vector<index_t> extent;
            std::vector<index_t> step;
        };

        // Subscripting axis `axis` of `v` with an integer: the coordinate
        // is fixed (counted from the end when negative) and the axis goes.
        void fix_axis(strided_view& v, size_t axis, index_t at) {
            const index_t n = v.extent[axis];
            const index_t c = at < 0 ? at + n : at;
            if (c < 0 || c >= n) throw std::out_of_range("tensor index is out of bounds");
            v.base += c * v.step[axis];
            v.extent.erase(v.extent.begin() + static_cast<std::ptrdiff_t>(axis));
            v.step.erase(v.step.begin() + static_cast<std::ptrdiff_t>(axis));
        }

        // Subscripting axis `axis` of `v` with a range: each endpoint is
        // counted from the end when negative and clamped to [0, extent];
        // the axis keeps every `r.step`-th coordinate from the first.
        void narrow_axis(strided_view& v, size_t axis, const slice& r) {
            if (r.step <= 0) throw std::invalid_argument("tensor slice step must be positive");
            const index_t n = v.extent[axis];
            const auto endpoint = [n](index_t e) { return std::clamp<index_t>(e < 0 ? e + n : e, 0, n); };
            const index_t first = endpoint(r.start);
            const index_t end = endpoint(r.stop);
            v.base += first * v.step[axis];
            v.extent[axis] = end > first ? (end - first - 1) / r.step + 1 : 0;
            v.step[axis] *= r.step;
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

        tensor make_tensor(std::vector<index_t> shape, device placement, values_ptr values) {
            return detail::tensor_access::make(
                std::make_shared<state_t>(tensor_layout{std::move(shape)}, placement, std::move(values))
            );
        }

        struct graph_result {
            values_ptr values;
            std::vector<index_t> shape;
            device placement;
        };

        // Plans the graph under `root` (cached by its structure), runs its
        // kernels on the calling thread's stream over the device values of
        // the tensors it reads, and returns the result's values.
        graph_result run_graph_with_shape(const node_ptr& root) {
            const auto start = std::chrono::steady_clock::now();
            graph_builder b;
            (void)b.visit(root);
            ir::infer(b.g);
            if (b.inputs.empty())
                throw std::invalid_argument("tensor expression must reference at least one tensor");
            const ir::node& r = b.g.at(b.g.root());
            if (r.is_scalar)
                throw std::invalid_argument("scalar expression cannot materialize to a tensor");
            graph_result result{nullptr, r.out, *b.placement};
            if (ir::checked_numel(r.out) == 0) {
                result.values = std::make_shared<resident_values>(hip_jit::device_buffer{}, std::vector<float32_t>{});
                return result;
            }
            const ir::graph compacted = ir::compact(b.g);
            bool hit = false;
            std::shared_ptr<plan::graph_plan> p = plan::lookup(compacted, &hit);

            // the inputs' values stay referenced until the launches are queued
            std::vector<values_ptr> held;
            std::vector<rt::buffer_state*> buffers;
            held.reserve(b.inputs.size());
            for (const tensor& t : b.inputs) {
                held.push_back(detail::tensor_access::state(t)->cell.get());
                buffers.push_back(hip_jit::buffer_access::state(held.back()->memory()).get());
            }
            std::shared_ptr<rt::buffer_state> out = plan::run(
                *p, buffers,
                [](size_t bytes) -> std::shared_ptr<rt::buffer_state> {
                    return std::make_shared<hip_jit::device_buffer_state>(bytes);
                }
            );
            result.values = std::make_shared<resident_values>(hip_jit::buffer_access::wrap(
                std::static_pointer_cast<hip_jit::device_buffer_state>(out)
            ));
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
            return result;
        }

        values_ptr run_graph(const node_ptr& root) { return run_graph_with_shape(root).values; }

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

    namespace {
        std::vector<index_t> checked_shape(std::vector<index_t> shape, size_t values) {
            if (values != ir::checked_numel(shape))
                throw std::invalid_argument("tensor data size does not match shape");
            return shape;
        }
    } // namespace

    tensor::tensor(std::vector<index_t> shape, std::vector<float32_t> values, device placement) {
        shape = checked_shape(std::move(shape), values.size());
        hip_jit::device_buffer memory = hip_jit::make_device_buffer(values);
        state_ = std::make_shared<state>(
            tensor_layout{std::move(shape)}, placement,
            std::make_shared<resident_values>(std::move(memory), std::move(values))
        );
    }

    tensor::tensor(std::vector<index_t> shape, std::vector<float32_t> values,
                   cuda_jit::device_buffer device_values, device placement) {
        shape = checked_shape(std::move(shape), values.size());
        if (device_values.size_bytes() < values.size() * sizeof(float32_t))
            throw std::invalid_argument("tensor device storage is too small");
        state_ = std::make_shared<state>(
            tensor_layout{std::move(shape)}, placement,
            std::make_shared<resident_values>(std::move(device_values), std::move(values))
        );
    }

    tensor::tensor(tensor_layout layout, cuda_jit::device_buffer storage, device placement) {
        if (storage.size_bytes() < storage_span(layout) * sizeof(float32_t))
            throw std::invalid_argument("tensor device storage is too small");
        state_ = std::make_shared<state>(
            std::move(layout), placement, std::make_shared<resident_values>(std::move(storage))
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

    namespace {
        // The device values holding a tensor's elements in row-major order:
        // its own, or for a view over strided storage, a gathered copy made
        // once.
        values_ptr row_major_values(const tensor& t, state_t& st) {
            if (st.layout.is_contiguous()) return st.cell.get();
            std::scoped_lock hold{st.gather_lock};
            if (st.gathered == nullptr) st.gathered = run_graph(detail::expr_access::root(tensor_expr{t}));
            return st.gathered;
        }
    } // namespace

    std::span<const float32_t> tensor::data() const {
        return row_major_values(*this, *state_)->host(numel());
    }

    std::vector<float32_t> tensor::cpu() const {
        return row_major_values(*this, *state_)->copy(numel());
    }

    const cuda_jit::device_buffer& tensor::device_data() const {
        return state_->cell.get()->memory();
    }

    const tensor& tensor::realize() const {
        (void)state_->cell.get();
        return *this;
    }

    void tensor::synchronize() const {
        const values_ptr values = state_->cell.get();
        std::shared_ptr<rt::stream> s = rt::current_stream();
        if (!values->memory().empty()) hip_jit::buffer_access::state(values->memory())->before_read(s);
        s->synchronize();
    }

    tensor_expr tensor::operator[](std::initializer_list<tensor_index> indices) const {
        if (indices.size() > rank()) throw std::invalid_argument("too many tensor indices");
        // Start from the tensor's own view of its storage and restrict it
        // one subscript at a time; axes past the last subscript stay whole.
        strided_view view{storage_offset(), {shape().begin(), shape().end()},
                          {strides().begin(), strides().end()}};
        size_t axis = 0; // the axis of `view` the next subscript applies to
        for (const tensor_index& ix : indices) {
            if (ix.kind_ == tensor_index::kind::index) {
                fix_axis(view, axis, ix.index_);
                continue;
            }
            if (ix.kind_ == tensor_index::kind::slice) narrow_axis(view, axis, ix.slice_);
            ++axis;
        }
        (void)ir::checked_numel(view.extent);
        auto n = std::make_shared<tensor_expr::node>();
        n->kind = ir::op::slice;
        // The view's base and steps count storage elements, so over strided
        // storage the slice reads the raw storage, not the tensor's view.
        n->lhs = is_contiguous() ? detail::expr_access::root(tensor_expr{*this}) : storage_node(*this);
        n->shape = std::move(view.extent);
        n->strides = std::move(view.step);
        n->offset = view.base;
        return detail::expr_access::make(std::move(n));
    }

    tensor_expr tensor::operator[](tensor_index index) const { return (*this)[{index}]; }

    // ------------------------------------------------------------------
    // tensor_expr
    // ------------------------------------------------------------------

    tensor_expr::tensor_expr(const tensor& value) {
        const std::shared_ptr<state_t>& st = detail::tensor_access::state(value);
        // a tensor whose graph has not run yet is inlined into this one
        if (node_ptr graph = st->cell.pending()) {
            root_ = std::move(graph);
            return;
        }
        root_ = storage_node(value);
        if (value.is_contiguous()) return;
        // over strided storage the tensor is a slice of the raw storage
        const tensor_layout& layout = value.layout();
        auto view = std::make_shared<tensor_expr::node>();
        view->kind = ir::op::slice;
        view->lhs = std::move(root_);
        view->shape.assign(layout.shape().begin(), layout.shape().end());
        view->strides.assign(layout.strides().begin(), layout.strides().end());
        view->offset = layout.storage_offset();
        root_ = std::move(view);
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
        return detail::tensor_access::make(std::make_shared<state_t>(tensor_layout{std::move(s)}, placement, root_));
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
        graph_result r = run_graph_with_shape(detail::expr_access::root(expression));
        return make_tensor(std::move(r.shape), r.placement, std::move(r.values));
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
