// porch host evaluator — TEST INFRASTRUCTURE ONLY.
//
// A CPU restatement of the reference's evaluation of a porch IR graph, used
// as the correctness oracle by tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py.  Nothing in the product (porch_amd/,
// include/) includes, links or calls this file.
//
// It follows the reference's algorithm, not the MI355X kernels:
//   * every node is evaluated at a linear output index, with the
//     reference's index formulas for views:
//       slice      src = offset + sum_d ((i / prod_{e>d} S_e) % S_d) * stride_d
//                  (reference src/tensor.cpp:511-530)
//       broadcast  src = sum over non-1 source dims of coord * contiguous
//                  source stride, right-aligned (532-560)
//       transpose  src = (i % S0) * S1 + i / S0 (562-571)
//       concat     axis coordinate < lhs extent ? lhs : rhs, with the
//                  coordinates re-linearised per operand (766-818)
//       reshape / unsqueeze  identity (731-741)
//       permute    (no reference counterpart; the rank-N generalisation of
//                  transpose) output coordinate i is source coordinate
//                  perm[i]: src = sum_i c_i * contiguous source stride_{perm[i]}
//   * + - * / in binary32 without contraction, maximum/minimum as the
//     ternaries l > r ? l : r and l < r ? l : r (616-683), reciprocal as
//     1.0f / x (863-868), exp as std::exp on float (the reference calls
//     NVRTC's __expf, 856-862; its bits are not reproducible off NVIDIA
//     hardware, so exp is compared within a tolerance);
//   * matmul as s = 0.0f; for k: s += L(row*K + k) * R(k*N + col)
//     (684-721), without FMA contraction;
//   * batched_matmul (no reference counterpart) as that matmul for each
//     batch entry b over L(b*M*K + ...) and R(b*K*N + ...);
//   * every sum/max — nested ones first, as lower_nested_reductions does
//     (964-989) — with the block-reduction order of
//     fused_reduction_kernel_source (896-962): 256 lanes each fold the
//     axis positions t, t+256, ... in order (sum from 0.0f, max from
//     -FLT_MAX with t = t > v ? t : v), then a shared-memory tree with
//     strides 128, 64, ..., 1.
//
// Evaluation is vectorised over blocks of indices and parallelised with
// OpenMP; nested reductions and matmul products are computed once and
// indexed (the reference recomputes them; the values are the same).

#include "porch_amd.h"

#include <omp.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

    constexpr int64_t block = 4096;

    struct onode {
        int32_t op = 0;
        int lhs = -1;
        int rhs = -1;
        int input = -1;
        float scalar = 0.0F;
        int64_t axis = 0;
        bool keepdim = false;
        std::vector<int64_t> param_shape;
        std::vector<int64_t> strides;
        int64_t offset = 0;
        // inferred
        bool is_scalar = false;
        std::vector<int64_t> shape;
    };

    std::vector<int64_t> contiguous(const std::vector<int64_t>& shape) {
        std::vector<int64_t> s(shape.size(), 1);
        int64_t stride = 1;
        for (size_t d = shape.size(); d > 0; --d) {
            s[d - 1] = stride;
            stride *= shape[d - 1];
        }
        return s;
    }

    int64_t count_of(const std::vector<int64_t>& shape) {
        int64_t n = 1;
        for (const int64_t e : shape) n *= e;
        return n;
    }

    std::vector<int64_t> reduced(const std::vector<int64_t>& shape, size_t axis, bool keep) {
        if (keep) {
            std::vector<int64_t> r = shape;
            r[axis] = 1;
            return r;
        }
        std::vector<int64_t> r;
        for (size_t d = 0; d < shape.size(); ++d)
            if (d != axis) r.push_back(shape[d]);
        if (r.empty()) r.push_back(1);
        return r;
    }

    struct evaluator {
        std::vector<onode> nodes;
        std::vector<const float*> inputs;
        std::vector<int64_t> input_counts;
        // Node -> fully evaluated values (nested reductions, matmuls).
        std::map<int, std::vector<float>> done;

        void infer() {
            for (onode& n : nodes) {
                const onode* l = n.lhs >= 0 ? &nodes[n.lhs] : nullptr;
                const onode* r = n.rhs >= 0 ? &nodes[n.rhs] : nullptr;
                switch (n.op) {
                    case PORCH_OP_INPUT:
                        n.shape = n.param_shape;
                        break;
                    case PORCH_OP_SCALAR:
                        n.is_scalar = true;
                        break;
                    case PORCH_OP_ADD:
                    case PORCH_OP_SUBTRACT:
                    case PORCH_OP_MULTIPLY:
                    case PORCH_OP_DIVIDE:
                    case PORCH_OP_MAXIMUM:
                    case PORCH_OP_MINIMUM:
                        if (l->is_scalar && r->is_scalar) n.is_scalar = true;
                        n.shape = l->is_scalar ? r->shape : l->shape;
                        if (!l->is_scalar && !r->is_scalar && l->shape != r->shape)
                            throw std::invalid_argument("tensor expression shapes must match");
                        break;
                    case PORCH_OP_MATMUL:
                        if (l->shape.size() != 2 || r->shape.size() != 2 ||
                            l->shape[1] != r->shape[0])
                            throw std::invalid_argument("matmul shapes");
                        n.shape = {l->shape[0], r->shape[1]};
                        break;
                    case PORCH_OP_BATCHED_MATMUL:
                        if (l->shape.size() != 3 || r->shape.size() != 3 ||
                            l->shape[0] != r->shape[0] || l->shape[2] != r->shape[1])
                            throw std::invalid_argument("batched_matmul shapes");
                        n.shape = {l->shape[0], l->shape[1], r->shape[2]};
                        break;
                    case PORCH_OP_SLICE:
                    case PORCH_OP_RESHAPE:
                    case PORCH_OP_BROADCAST:
                        n.shape = n.param_shape;
                        break;
                    case PORCH_OP_UNSQUEEZE:
                        n.shape = l->shape;
                        n.shape.insert(n.shape.begin() + n.axis, 1);
                        break;
                    case PORCH_OP_TRANSPOSE:
                        n.shape = {l->shape[1], l->shape[0]};
                        break;
                    case PORCH_OP_PERMUTE: {
                        if (n.param_shape.size() != l->shape.size())
                            throw std::invalid_argument("permute rank");
                        std::vector<bool> seen(l->shape.size(), false);
                        for (const int64_t a : n.param_shape) {
                            if (a < 0 || a >= static_cast<int64_t>(l->shape.size()) || seen[a])
                                throw std::invalid_argument("permute axes");
                            seen[a] = true;
                            n.shape.push_back(l->shape[a]);
                        }
                        break;
                    }
                    case PORCH_OP_CONCAT:
                        n.shape = l->shape;
                        n.shape[n.axis] += r->shape[n.axis];
                        break;
                    case PORCH_OP_SUM:
                    case PORCH_OP_MAX:
                        n.shape = reduced(l->shape, static_cast<size_t>(n.axis), n.keepdim);
                        break;
                    case PORCH_OP_EXP:
                    case PORCH_OP_RECIPROCAL:
                        n.is_scalar = l->is_scalar;
                        n.shape = l->shape;
                        break;
                    default:
                        throw std::invalid_argument("unknown node");
                }
            }
        }

        // value(node, idx[j]) for j < n into out[j].
        void eval(int id, const int64_t* idx, int64_t n, float* out) {
            const onode& nd = nodes[id];
            auto found = done.find(id);
            if (found != done.end()) {
                const float* v = found->second.data();
                for (int64_t j = 0; j < n; ++j) out[j] = v[idx[j]];
                return;
            }
            switch (nd.op) {
                case PORCH_OP_INPUT: {
                    const float* v = inputs[nd.input];
                    const int64_t limit = input_counts[nd.input];
                    for (int64_t j = 0; j < n; ++j) {
                        if (idx[j] < 0 || idx[j] >= limit)
                            throw std::out_of_range("oracle: input index out of range");
                        out[j] = v[idx[j]];
                    }
                    return;
                }
                case PORCH_OP_SCALAR:
                    for (int64_t j = 0; j < n; ++j) out[j] = nd.scalar;
                    return;
                case PORCH_OP_ADD:
                case PORCH_OP_SUBTRACT:
                case PORCH_OP_MULTIPLY:
                case PORCH_OP_DIVIDE:
                case PORCH_OP_MAXIMUM:
                case PORCH_OP_MINIMUM: {
                    std::vector<float> a(static_cast<size_t>(n));
                    std::vector<float> b(static_cast<size_t>(n));
                    eval(nd.lhs, idx, n, a.data());
                    eval(nd.rhs, idx, n, b.data());
                    for (int64_t j = 0; j < n; ++j) {
                        const float l = a[j];
                        const float r = b[j];
                        float v = 0.0F;
                        switch (nd.op) {
                            case PORCH_OP_ADD: v = l + r; break;
                            case PORCH_OP_SUBTRACT: v = l - r; break;
                            case PORCH_OP_MULTIPLY: v = l * r; break;
                            case PORCH_OP_DIVIDE: v = l / r; break;
                            case PORCH_OP_MAXIMUM: v = (l > r) ? l : r; break;
                            default: v = (l < r) ? l : r; break;
                        }
                        out[j] = v;
                    }
                    return;
                }
                case PORCH_OP_EXP: {
                    eval(nd.lhs, idx, n, out);
                    for (int64_t j = 0; j < n; ++j) out[j] = std::exp(out[j]);
                    return;
                }
                case PORCH_OP_RECIPROCAL: {
                    eval(nd.lhs, idx, n, out);
                    for (int64_t j = 0; j < n; ++j) out[j] = 1.0F / out[j];
                    return;
                }
                case PORCH_OP_SLICE: {
                    std::vector<int64_t> src(static_cast<size_t>(n));
                    for (int64_t j = 0; j < n; ++j) {
                        int64_t s = nd.offset;
                        int64_t size = 1;
                        for (size_t d = nd.shape.size(); d > 0; --d) {
                            const size_t k = d - 1;
                            if (nd.strides[k] != 0)
                                s += ((idx[j] / size) % nd.shape[k]) * nd.strides[k];
                            size *= nd.shape[k];
                        }
                        src[j] = s;
                    }
                    eval(nd.lhs, src.data(), n, out);
                    return;
                }
                case PORCH_OP_RESHAPE:
                case PORCH_OP_UNSQUEEZE:
                    eval(nd.lhs, idx, n, out);
                    return;
                case PORCH_OP_TRANSPOSE: {
                    const std::vector<int64_t>& s = nodes[nd.lhs].shape;
                    std::vector<int64_t> src(static_cast<size_t>(n));
                    for (int64_t j = 0; j < n; ++j)
                        src[j] = (idx[j] % s[0]) * s[1] + idx[j] / s[0];
                    eval(nd.lhs, src.data(), n, out);
                    return;
                }
                case PORCH_OP_PERMUTE: {
                    const std::vector<int64_t> sstr = contiguous(nodes[nd.lhs].shape);
                    std::vector<int64_t> src(static_cast<size_t>(n));
                    for (int64_t j = 0; j < n; ++j) {
                        int64_t rest = idx[j];
                        int64_t s = 0;
                        for (size_t d = nd.shape.size(); d > 0; --d) {
                            const size_t k = d - 1;
                            s += (rest % nd.shape[k]) * sstr[nd.param_shape[k]];
                            rest /= nd.shape[k];
                        }
                        src[j] = s;
                    }
                    eval(nd.lhs, src.data(), n, out);
                    return;
                }
                case PORCH_OP_BROADCAST: {
                    const onode& source = nodes[nd.lhs];
                    if (source.is_scalar) {
                        eval(nd.lhs, idx, n, out);
                        return;
                    }
                    const std::vector<int64_t> sstr = contiguous(source.shape);
                    const std::vector<int64_t> tsize = contiguous(nd.shape);
                    const size_t off = nd.shape.size() - source.shape.size();
                    std::vector<int64_t> src(static_cast<size_t>(n));
                    for (int64_t j = 0; j < n; ++j) {
                        int64_t s = 0;
                        for (size_t d = 0; d < source.shape.size(); ++d) {
                            if (source.shape[d] == 1) continue;
                            const size_t t = off + d;
                            s += ((idx[j] / tsize[t]) % nd.shape[t]) * sstr[d];
                        }
                        src[j] = s;
                    }
                    eval(nd.lhs, src.data(), n, out);
                    return;
                }
                case PORCH_OP_CONCAT: {
                    const onode& l = nodes[nd.lhs];
                    const onode& r = nodes[nd.rhs];
                    const std::vector<int64_t> ostr = contiguous(nd.shape);
                    const std::vector<int64_t> lstr = contiguous(l.shape);
                    const std::vector<int64_t> rstr = contiguous(r.shape);
                    const size_t axis = static_cast<size_t>(nd.axis);
                    std::vector<int64_t> li, ri, lpos, rpos;
                    for (int64_t j = 0; j < n; ++j) {
                        const int64_t a = (idx[j] / ostr[axis]) % nd.shape[axis];
                        int64_t ls = 0;
                        int64_t rs = 0;
                        for (size_t d = 0; d < nd.shape.size(); ++d) {
                            const int64_t c = (idx[j] / ostr[d]) % nd.shape[d];
                            ls += c * lstr[d];
                            rs += (d == axis ? c - l.shape[axis] : c) * rstr[d];
                        }
                        if (a < l.shape[axis]) {
                            li.push_back(ls);
                            lpos.push_back(j);
                        }
                        else {
                            ri.push_back(rs);
                            rpos.push_back(j);
                        }
                    }
                    std::vector<float> lv(li.size());
                    std::vector<float> rv(ri.size());
                    if (!li.empty()) eval(nd.lhs, li.data(), static_cast<int64_t>(li.size()), lv.data());
                    if (!ri.empty()) eval(nd.rhs, ri.data(), static_cast<int64_t>(ri.size()), rv.data());
                    for (size_t k = 0; k < lpos.size(); ++k) out[lpos[k]] = lv[k];
                    for (size_t k = 0; k < rpos.size(); ++k) out[rpos[k]] = rv[k];
                    return;
                }
                default:
                    throw std::logic_error("oracle: unmaterialised reduction or matmul");
            }
        }

        // All values of node `id` (linear indices 0..count-1).
        std::vector<float> evaluate_all(int id) {
            const int64_t count = count_of(nodes[id].shape);
            std::vector<float> result(static_cast<size_t>(count));
            std::string error;
#pragma omp parallel for schedule(dynamic, 4)
            for (int64_t start = 0; start < count; start += block) {
                try {
                    const int64_t n = std::min(block, count - start);
                    std::vector<int64_t> idx(static_cast<size_t>(n));
                    for (int64_t j = 0; j < n; ++j) idx[j] = start + j;
                    eval(id, idx.data(), n, result.data() + start);
                }
                catch (const std::exception& e) {
#pragma omp critical
                    error = e.what();
                }
            }
            if (!error.empty()) throw std::runtime_error(error);
            return result;
        }

        // Materialise every reduction and matmul below `id` (post-order),
        // then `id` itself if it is one.
        void prepare(int id) {
            if (id < 0 || done.count(id)) return;
            const onode& n = nodes[id];
            prepare(n.lhs);
            prepare(n.rhs);
            if (n.op == PORCH_OP_SUM || n.op == PORCH_OP_MAX) done[id] = reduce(id);
            if (n.op == PORCH_OP_MATMUL || n.op == PORCH_OP_BATCHED_MATMUL) done[id] = matmul(id);
        }

        std::vector<float> reduce(int id) {
            const onode& n = nodes[id];
            const onode& src = nodes[n.lhs];
            const bool is_max = n.op == PORCH_OP_MAX;
            const size_t axis = static_cast<size_t>(n.axis);
            const std::vector<int64_t> sstr = contiguous(src.shape);
            const std::vector<int64_t>& oshape = n.shape;
            const std::vector<int64_t> osize = contiguous(oshape);
            const int64_t outputs = count_of(oshape);
            const int64_t extent = src.shape[axis];
            std::vector<float> result(static_cast<size_t>(outputs));
            std::string error;
#pragma omp parallel for schedule(dynamic, 1)
            for (int64_t o = 0; o < outputs; ++o) {
                try {
                    // reference emit_reduction_source_index (573-614)
                    int64_t base = 0;
                    size_t out_dim = 0;
                    for (size_t d = 0; d < src.shape.size(); ++d) {
                        if (d == axis) continue;
                        if (n.keepdim) {
                            base += ((o / osize[d]) % oshape[d]) * sstr[d];
                            continue;
                        }
                        base += ((o / osize[out_dim]) % oshape[out_dim]) * sstr[d];
                        ++out_dim;
                    }
                    std::vector<int64_t> idx(static_cast<size_t>(extent));
                    for (int64_t a = 0; a < extent; ++a) idx[a] = base + a * sstr[axis];
                    std::vector<float> v(static_cast<size_t>(extent));
                    for (int64_t s = 0; s < extent; s += block) {
                        const int64_t m = std::min(block, extent - s);
                        eval(n.lhs, idx.data() + s, m, v.data() + s);
                    }
                    float lanes[256];
                    for (int t = 0; t < 256; ++t) {
                        float total = is_max ? -FLT_MAX : 0.0F;
                        for (int64_t a = t; a < extent; a += 256) {
                            if (is_max) total = total > v[a] ? total : v[a];
                            else total += v[a];
                        }
                        lanes[t] = total;
                    }
                    for (int stride = 128; stride > 0; stride /= 2) {
                        for (int t = 0; t < stride; ++t) {
                            if (is_max)
                                lanes[t] = lanes[t] > lanes[t + stride] ? lanes[t] : lanes[t + stride];
                            else
                                lanes[t] += lanes[t + stride];
                        }
                    }
                    result[o] = lanes[0];
                }
                catch (const std::exception& e) {
#pragma omp critical
                    error = e.what();
                }
            }
            if (!error.empty()) throw std::runtime_error(error);
            return result;
        }

        // matmul, and batched_matmul as one matmul per batch entry.
        std::vector<float> matmul(int id) {
            const onode& n = nodes[id];
            const std::vector<float> a = evaluate_all(n.lhs);
            const std::vector<float> b = evaluate_all(n.rhs);
            const bool batched = n.op == PORCH_OP_BATCHED_MATMUL;
            const int64_t batch = batched ? n.shape[0] : 1;
            const int64_t M = n.shape[batched ? 1 : 0];
            const int64_t N = n.shape[batched ? 2 : 1];
            const int64_t K = nodes[n.lhs].shape[batched ? 2 : 1];
            std::vector<float> c(static_cast<size_t>(batch * M * N), 0.0F);
            // Row i accumulates over k in order: per element exactly
            // s = 0; s += a[i,0]*b[0,j]; s += a[i,1]*b[1,j]; ...
#pragma omp parallel for schedule(static)
            for (int64_t bi = 0; bi < batch * M; ++bi) {
                const int64_t e = bi / (M > 0 ? M : 1);
                const int64_t i = bi % (M > 0 ? M : 1);
                float* row = c.data() + (e * M + i) * N;
                for (int64_t k = 0; k < K; ++k) {
                    const float x = a[static_cast<size_t>((e * M + i) * K + k)];
                    const float* brow = b.data() + (e * K + k) * N;
                    for (int64_t j = 0; j < N; ++j) {
                        const float p = x * brow[j];
                        row[j] = row[j] + p;
                    }
                }
            }
            return c;
        }
    };

} // namespace

extern "C" {

// Evaluates the graph's root into out[out_count].  Returns 0 on success,
// otherwise writes a message into error[error_capacity] and returns 1.
int32_t porch_oracle_eval(const porch_node* table, int32_t n_nodes, const int64_t* dims,
                          int64_t n_dims, const float* const* inputs,
                          const int64_t* input_counts, int32_t n_inputs, float* out,
                          int64_t out_count, char* error, size_t error_capacity) {
    try {
        evaluator ev;
        ev.nodes.resize(static_cast<size_t>(n_nodes));
        for (int32_t i = 0; i < n_nodes; ++i) {
            const porch_node& c = table[i];
            onode& n = ev.nodes[static_cast<size_t>(i)];
            n.op = c.op;
            n.lhs = c.lhs;
            n.rhs = c.rhs;
            n.input = c.input;
            n.scalar = c.scalar;
            n.axis = c.axis;
            n.keepdim = c.keepdim != 0;
            n.offset = c.offset;
            const bool has_shape = c.op == PORCH_OP_INPUT || c.op == PORCH_OP_SLICE ||
                                   c.op == PORCH_OP_RESHAPE || c.op == PORCH_OP_BROADCAST ||
                                   c.op == PORCH_OP_PERMUTE;
            const int64_t needed = c.op == PORCH_OP_SLICE ? 2 * int64_t{c.rank}
                                   : has_shape          ? int64_t{c.rank}
                                                        : 0;
            if (needed > 0 && (c.dims < 0 || c.rank < 0 || c.dims + needed > n_dims))
                throw std::invalid_argument("oracle: dims out of range");
            if (has_shape)
                n.param_shape.assign(dims + c.dims, dims + c.dims + c.rank);
            if (c.op == PORCH_OP_SLICE)
                n.strides.assign(dims + c.dims + c.rank, dims + c.dims + 2 * c.rank);
            if (c.op == PORCH_OP_INPUT && (c.input < 0 || c.input >= n_inputs))
                throw std::invalid_argument("oracle: input slot out of range");
        }
        ev.inputs.assign(inputs, inputs + n_inputs);
        ev.input_counts.assign(input_counts, input_counts + n_inputs);
        ev.infer();
        const int root = n_nodes - 1;
        if (count_of(ev.nodes[root].shape) != out_count)
            throw std::invalid_argument("oracle: output size mismatch");
        ev.prepare(root);
        std::vector<float> values = ev.done.count(root) ? ev.done[root] : ev.evaluate_all(root);
        std::memcpy(out, values.data(), values.size() * sizeof(float));
        return 0;
    }
    catch (const std::exception& e) {
        if (error != nullptr && error_capacity > 0) {
            std::strncpy(error, e.what(), error_capacity - 1);
            error[error_capacity - 1] = '\0';
        }
        return 1;
    }
}

// Threads OpenMP will use (the CPU baseline states its core count).
int32_t porch_oracle_threads(void) { return omp_get_max_threads(); }

} // extern "C"
