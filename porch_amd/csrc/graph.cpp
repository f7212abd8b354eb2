#include "graph.hpp"

#include <algorithm>
#include <cstring>
#include <map>
#include <stdexcept>
#include <tuple>

namespace porch::ir {

    bool is_elementwise_binary(op kind) {
        switch (kind) {
            case op::add:
            case op::subtract:
            case op::multiply:
            case op::divide:
            case op::maximum:
            case op::minimum:
                return true;
            default:
                return false;
        }
    }

    bool is_reduction(op kind) { return kind == op::sum || kind == op::max; }

    bool is_view(op kind) {
        switch (kind) {
            case op::slice:
            case op::reshape:
            case op::unsqueeze:
            case op::transpose:
            case op::permute:
            case op::broadcast:
            case op::concat:
                return true;
            default:
                return false;
        }
    }

    size_t checked_numel(const std::vector<int64_t>& shape) {
        size_t count = 1;
        for (const int64_t extent : shape) {
            if (extent < 0) {
                throw std::invalid_argument(
                    "tensor shape extents must be non-negative"
                );
            }
            count *= static_cast<size_t>(extent);
        }
        return count;
    }

    int64_t numel(const std::vector<int64_t>& shape) {
        int64_t count = 1;
        for (const int64_t extent : shape) count *= extent;
        return count;
    }

    std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& shape) {
        std::vector<int64_t> strides(shape.size(), 1);
        int64_t stride = 1;
        for (size_t d = shape.size(); d > 0; --d) {
            strides[d - 1] = stride;
            stride *= shape[d - 1];
        }
        return strides;
    }

    std::vector<int64_t> reduced_shape(
        const std::vector<int64_t>& shape, size_t axis, bool keepdim
    ) {
        if (keepdim) {
            std::vector<int64_t> result = shape;
            result[axis] = 1;
            return result;
        }
        std::vector<int64_t> result;
        for (size_t d = 0; d < shape.size(); ++d) {
            if (d != axis) result.push_back(shape[d]);
        }
        // A rank-1 reduction keeps one element (reference
        // src/tensor.cpp:316).
        if (result.empty()) result.push_back(1);
        return result;
    }

    graph from_c(const porch_graph* table) {
        if (table == nullptr) throw std::invalid_argument("graph is null");
        if (table->n_nodes <= 0 || table->nodes == nullptr) {
            throw std::invalid_argument("graph has no nodes");
        }
        if (table->n_dims < 0 || (table->n_dims > 0 && table->dims == nullptr)) {
            throw std::invalid_argument("graph dims are malformed");
        }
        graph g;
        g.nodes.resize(static_cast<size_t>(table->n_nodes));
        auto dims = [&](int64_t start, int64_t count) {
            if (start < 0 || count < 0 || start + count > table->n_dims) {
                throw std::invalid_argument("graph node dims are out of range");
            }
            return std::vector<int64_t>(
                table->dims + start, table->dims + start + count
            );
        };
        for (int32_t i = 0; i < table->n_nodes; ++i) {
            const porch_node& c = table->nodes[i];
            node& n = g.nodes[static_cast<size_t>(i)];
            if (c.op < 0 || c.op >= op_count) {
                throw std::invalid_argument("unknown tensor expression node");
            }
            n.kind = static_cast<op>(c.op);
            // Operand fields a kind does not use are ignored.
            auto operand = [&](int32_t index) {
                if (index < 0 || index >= i) {
                    throw std::invalid_argument(
                        "graph operands must refer to earlier nodes"
                    );
                }
                return static_cast<int>(index);
            };
            const bool binary = is_elementwise_binary(n.kind) ||
                                n.kind == op::matmul || n.kind == op::batched_matmul ||
                                n.kind == op::concat;
            const bool unary = !binary && n.kind != op::input &&
                               n.kind != op::scalar;
            n.lhs = (binary || unary) ? operand(c.lhs) : -1;
            n.rhs = binary ? operand(c.rhs) : -1;
            n.scalar = c.scalar;
            if (c.axis < 0) throw std::invalid_argument("axis must be non-negative");
            n.axis = c.axis;
            n.keepdim = c.keepdim != 0;
            n.offset = c.offset;
            if (c.rank < 0) throw std::invalid_argument("rank must be non-negative");
            switch (n.kind) {
                case op::input:
                    if (c.input < 0) {
                        throw std::invalid_argument("input slot must be non-negative");
                    }
                    n.input = c.input;
                    g.n_inputs = std::max(g.n_inputs, c.input + 1);
                    n.shape = dims(c.dims, c.rank);
                    break;
                case op::slice:
                    n.shape = dims(c.dims, c.rank);
                    n.strides = dims(c.dims + c.rank, c.rank);
                    break;
                case op::reshape:
                case op::broadcast:
                case op::permute:
                    n.shape = dims(c.dims, c.rank);
                    break;
                default:
                    break;
            }
        }
        return g;
    }

    namespace {

        void require_same_shape(const node& lhs, const node& rhs) {
            if (lhs.is_scalar || rhs.is_scalar) return;
            if (lhs.out == rhs.out) return;
            throw std::invalid_argument("tensor expression shapes must match");
        }

        void require_axis(int64_t axis, size_t rank, const char* operation) {
            if (axis < 0 || static_cast<size_t>(axis) >= rank) {
                throw std::invalid_argument(
                    std::string{operation} + " axis is out of bounds"
                );
            }
        }

        void require_broadcastable(
            const std::vector<int64_t>& source,
            const std::vector<int64_t>& target
        ) {
            if (source.size() > target.size()) {
                throw std::invalid_argument(
                    "broadcast target rank must be at least source rank"
                );
            }
            const size_t offset = target.size() - source.size();
            for (size_t d = 0; d < source.size(); ++d) {
                if (source[d] != 1 && source[d] != target[offset + d]) {
                    throw std::invalid_argument(
                        "broadcast shapes are not compatible"
                    );
                }
            }
        }

        void infer_node(graph& g, size_t index) {
            node& n = g.nodes[index];
            const node* lhs = n.lhs >= 0 ? &g.nodes[n.lhs] : nullptr;
            const node* rhs = n.rhs >= 0 ? &g.nodes[n.rhs] : nullptr;
            n.is_scalar = false;
            n.out.clear();
            switch (n.kind) {
                case op::input:
                    (void)checked_numel(n.shape);
                    n.out = n.shape;
                    return;
                case op::scalar:
                    n.is_scalar = true;
                    return;
                case op::add:
                case op::subtract:
                case op::multiply:
                case op::divide:
                case op::maximum:
                case op::minimum:
                    require_same_shape(*lhs, *rhs);
                    if (lhs->is_scalar) {
                        n.is_scalar = rhs->is_scalar;
                        n.out = rhs->out;
                    }
                    else {
                        n.out = lhs->out;
                    }
                    return;
                case op::matmul:
                    if (lhs->is_scalar || rhs->is_scalar) {
                        throw std::invalid_argument(
                            "matmul operands must be tensors"
                        );
                    }
                    if (lhs->out.size() != 2 || rhs->out.size() != 2) {
                        throw std::invalid_argument(
                            "matmul requires rank-2 tensors"
                        );
                    }
                    if (lhs->out[1] != rhs->out[0]) {
                        throw std::invalid_argument(
                            "matmul inner dimensions must match"
                        );
                    }
                    n.out = {lhs->out[0], rhs->out[1]};
                    return;
                case op::batched_matmul:
                    if (lhs->is_scalar || rhs->is_scalar) {
                        throw std::invalid_argument(
                            "batched_matmul operands must be tensors"
                        );
                    }
                    if (lhs->out.size() != 3 || rhs->out.size() != 3) {
                        throw std::invalid_argument(
                            "batched_matmul requires rank-3 tensors"
                        );
                    }
                    if (lhs->out[0] != rhs->out[0]) {
                        throw std::invalid_argument(
                            "batched_matmul batch dimensions must match"
                        );
                    }
                    if (lhs->out[2] != rhs->out[1]) {
                        throw std::invalid_argument(
                            "batched_matmul inner dimensions must match"
                        );
                    }
                    n.out = {lhs->out[0], lhs->out[1], rhs->out[2]};
                    return;
                case op::slice: {
                    if (n.strides.size() != n.shape.size()) {
                        throw std::invalid_argument("tensor layout rank mismatch");
                    }
                    (void)checked_numel(n.shape);
                    // The view must stay inside its source (the reference
                    // guarantees this by construction in operator[]).
                    if (lhs->is_scalar) {
                        throw std::invalid_argument(
                            "slice operand must be a tensor"
                        );
                    }
                    const int64_t source_count = numel(lhs->out);
                    if (numel(n.shape) > 0) {
                        int64_t last = n.offset;
                        for (size_t d = 0; d < n.shape.size(); ++d) {
                            if (n.strides[d] < 0) {
                                throw std::invalid_argument(
                                    "tensor layout strides must be non-negative"
                                );
                            }
                            last += (n.shape[d] - 1) * n.strides[d];
                        }
                        if (n.offset < 0 || last >= source_count) {
                            throw std::out_of_range(
                                "tensor slice is out of bounds"
                            );
                        }
                    }
                    n.out = n.shape;
                    return;
                }
                case op::reshape:
                    if (lhs->is_scalar) {
                        throw std::invalid_argument(
                            "reshape operand must be a tensor"
                        );
                    }
                    if (checked_numel(lhs->out) != checked_numel(n.shape)) {
                        throw std::invalid_argument(
                            "reshape must preserve tensor element count"
                        );
                    }
                    n.out = n.shape;
                    return;
                case op::unsqueeze:
                    if (lhs->is_scalar) {
                        throw std::invalid_argument(
                            "unsqueeze operand must be a tensor"
                        );
                    }
                    if (static_cast<size_t>(n.axis) > lhs->out.size()) {
                        throw std::invalid_argument(
                            "unsqueeze axis is out of bounds"
                        );
                    }
                    n.out = lhs->out;
                    n.out.insert(n.out.begin() + n.axis, 1);
                    return;
                case op::transpose:
                    if (lhs->is_scalar) {
                        throw std::invalid_argument(
                            "transpose operand must be a tensor"
                        );
                    }
                    if (lhs->out.size() != 2) {
                        throw std::invalid_argument(
                            "transpose currently requires a rank-2 tensor"
                        );
                    }
                    n.out = {lhs->out[1], lhs->out[0]};
                    return;
                case op::permute: {
                    if (lhs->is_scalar) {
                        throw std::invalid_argument(
                            "permute operand must be a tensor"
                        );
                    }
                    const size_t rank = lhs->out.size();
                    std::vector<bool> seen(rank, false);
                    bool valid = n.shape.size() == rank;
                    for (size_t i = 0; valid && i < rank; ++i) {
                        const int64_t axis = n.shape[i];
                        valid = axis >= 0 && static_cast<size_t>(axis) < rank &&
                                !seen[static_cast<size_t>(axis)];
                        if (valid) seen[static_cast<size_t>(axis)] = true;
                    }
                    if (!valid) {
                        throw std::invalid_argument(
                            "permute axes must be a permutation of the operand's dimensions"
                        );
                    }
                    n.out.resize(rank);
                    for (size_t i = 0; i < rank; ++i) {
                        n.out[i] = lhs->out[static_cast<size_t>(n.shape[i])];
                    }
                    return;
                }
                case op::broadcast:
                    if (!lhs->is_scalar) require_broadcastable(lhs->out, n.shape);
                    n.out = n.shape;
                    return;
                case op::concat: {
                    if (lhs->is_scalar || rhs->is_scalar) {
                        throw std::invalid_argument(
                            "concat operands must be tensors"
                        );
                    }
                    if (lhs->out.size() != rhs->out.size()) {
                        throw std::invalid_argument(
                            "concat operands must have the same rank"
                        );
                    }
                    require_axis(n.axis, lhs->out.size(), "concat");
                    for (size_t d = 0; d < lhs->out.size(); ++d) {
                        if (d == static_cast<size_t>(n.axis)) continue;
                        if (lhs->out[d] != rhs->out[d]) {
                            throw std::invalid_argument(
                                "concat non-axis dimensions must match"
                            );
                        }
                    }
                    n.out = lhs->out;
                    n.out[n.axis] += rhs->out[n.axis];
                    return;
                }
                case op::sum:
                case op::max:
                    if (lhs->is_scalar) {
                        throw std::invalid_argument(
                            "reduction operand must be a tensor"
                        );
                    }
                    require_axis(n.axis, lhs->out.size(), "reduction");
                    n.out = reduced_shape(lhs->out, n.axis, n.keepdim);
                    return;
                case op::exp:
                case op::reciprocal:
                    n.is_scalar = lhs->is_scalar;
                    n.out = lhs->out;
                    return;
            }
            throw std::invalid_argument("unknown tensor expression node");
        }

        std::vector<bool> reachable(const graph& g) {
            std::vector<bool> live(g.nodes.size(), false);
            if (g.nodes.empty()) return live;
            live.back() = true;
            for (size_t i = g.nodes.size(); i > 0; --i) {
                const node& n = g.nodes[i - 1];
                if (!live[i - 1]) continue;
                if (n.lhs >= 0) live[n.lhs] = true;
                if (n.rhs >= 0) live[n.rhs] = true;
            }
            return live;
        }

    } // namespace

    void infer(graph& g) {
        const std::vector<bool> live = reachable(g);
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            if (live[i]) infer_node(g, i);
        }
    }

    graph compact(const graph& source) {
        const std::vector<bool> live = reachable(source);
        graph out;
        out.n_inputs = source.n_inputs;
        std::vector<int> remap(source.nodes.size(), -1);
        std::map<std::string, int> seen;
        for (size_t i = 0; i < source.nodes.size(); ++i) {
            if (!live[i]) continue;
            node n = source.nodes[i];
            if (n.lhs >= 0) n.lhs = remap[n.lhs];
            if (n.rhs >= 0) n.rhs = remap[n.rhs];
            // Structural identity of the node (operands already merged).
            std::string key;
            auto put = [&key](const void* data, size_t size) {
                key.append(static_cast<const char*>(data), size);
            };
            const int32_t kind = static_cast<int32_t>(n.kind);
            put(&kind, sizeof kind);
            put(&n.lhs, sizeof n.lhs);
            put(&n.rhs, sizeof n.rhs);
            put(&n.input, sizeof n.input);
            uint32_t bits = 0;
            std::memcpy(&bits, &n.scalar, sizeof bits);
            if (n.kind == op::scalar) put(&bits, sizeof bits);
            put(&n.axis, sizeof n.axis);
            const char keep = n.keepdim ? 1 : 0;
            put(&keep, 1);
            const uint64_t rank = n.shape.size();
            put(&rank, sizeof rank);
            if (!n.shape.empty()) put(n.shape.data(), n.shape.size() * 8);
            if (!n.strides.empty()) put(n.strides.data(), n.strides.size() * 8);
            put(&n.offset, sizeof n.offset);
            auto found = seen.find(key);
            const bool is_root = i + 1 == source.nodes.size();
            if (found != seen.end() && !is_root) {
                remap[i] = found->second;
                continue;
            }
            remap[i] = static_cast<int>(out.nodes.size());
            seen.emplace(std::move(key), remap[i]);
            out.nodes.push_back(std::move(n));
        }
        infer(out);
        return out;
    }

    std::string canonical_key(const graph& g) {
        std::string key;
        key.reserve(g.nodes.size() * 48);
        auto put = [&key](const void* data, size_t size) {
            key.append(static_cast<const char*>(data), size);
        };
        for (const node& n : g.nodes) {
            const int32_t fields[5] = {
                static_cast<int32_t>(n.kind), n.lhs, n.rhs, n.input,
                n.keepdim ? 1 : 0
            };
            put(fields, sizeof fields);
            uint32_t bits = 0;
            std::memcpy(&bits, &n.scalar, sizeof bits);
            put(&bits, sizeof bits);
            put(&n.axis, sizeof n.axis);
            put(&n.offset, sizeof n.offset);
            const uint32_t sizes[2] = {
                static_cast<uint32_t>(n.shape.size()),
                static_cast<uint32_t>(n.strides.size())
            };
            put(sizes, sizeof sizes);
            if (!n.shape.empty()) put(n.shape.data(), n.shape.size() * 8);
            if (!n.strides.empty()) put(n.strides.data(), n.strides.size() * 8);
        }
        return key;
    }

} // namespace porch::ir
