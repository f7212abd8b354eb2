#include "planner.hpp"

#include <algorithm>
#include <chrono>
#include <functional>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>
#include <unordered_map>

namespace porch::plan {
    namespace {

        bool is_elementwise(ir::op kind) {
            return ir::is_elementwise_binary(kind) || kind == ir::op::exp ||
                   kind == ir::op::reciprocal;
        }

        bool is_product(ir::op kind) {
            return kind == ir::op::matmul || kind == ir::op::batched_matmul;
        }

        bool is_boundary(ir::op kind) {
            return ir::is_reduction(kind) || is_product(kind);
        }

        struct builder {
            const ir::graph& g;
            graph_plan& plan;
            int compute_units;
            std::map<int, int> temp_of;
            // Element offset of a node's values within its temporary (0
            // unless several nodes share one: the column softmax's max
            // and sum).
            std::map<int, int64_t> offset_of;
            cg::index_width width;

            // The nodes that read each node.
            std::vector<std::vector<int>> users;

            builder(const ir::graph& graph, graph_plan& target, int cus)
                : g(graph), plan(target), compute_units(cus) {
                users.resize(g.nodes.size());
                for (size_t i = 0; i < g.nodes.size(); ++i) {
                    const ir::node& n = g.nodes[i];
                    if (n.lhs >= 0) users[static_cast<size_t>(n.lhs)].push_back(static_cast<int>(i));
                    if (n.rhs >= 0 && n.rhs != n.lhs) users[static_cast<size_t>(n.rhs)].push_back(static_cast<int>(i));
                }
                int64_t largest = 0;
                for (const ir::node& n : g.nodes) {
                    largest = std::max(largest, ir::numel(n.out));
                    if (n.kind == ir::op::input)
                        largest = std::max(largest, ir::numel(n.shape));
                    if (n.kind == ir::op::slice) {
                        int64_t last = n.offset;
                        for (size_t d = 0; d < n.shape.size(); ++d)
                            last += std::max<int64_t>(n.shape[d] - 1, 0) * n.strides[d];
                        largest = std::max(largest, last + 1);
                    }
                }
                width.wide = largest >= (int64_t{1} << 30);
            }

            [[nodiscard]] int n_slots() const {
                return g.n_inputs + static_cast<int>(plan.temp_elems.size());
            }

            // Floats each kernel slot's buffer is guaranteed to hold.
            [[nodiscard]] std::vector<int64_t> slot_elems() const {
                std::vector<int64_t> elems(plan.input_elems.begin(), plan.input_elems.end());
                elems.insert(elems.end(), plan.temp_elems.begin(), plan.temp_elems.end());
                return elems;
            }

            void bind_inputs(cg::lowering& low) const {
                for (int i = 0; i < g.n_inputs; ++i) low.input_slot[static_cast<size_t>(i)] = i;
                for (const auto& [node, temp] : temp_of) {
                    cg::binding b;
                    b.what = cg::binding::kind::slot;
                    b.slot = g.n_inputs + temp;
                    const auto off = offset_of.find(node);
                    if (off != offset_of.end()) b.offset = off->second;
                    low.bound[node] = b;
                }
            }

            // Matmul / reduction nodes reachable from `id` through pointwise
            // and view nodes, excluding `skip` and materialised nodes.
            void boundaries(int id, std::set<int>& found, const std::set<int>& skip,
                            bool is_root) {
                std::set<int> seen;
                std::function<void(int, bool)> walk = [&](int x, bool root) {
                    if (x < 0 || seen.count(x)) return;
                    seen.insert(x);
                    if (temp_of.count(x)) return;
                    if (skip.count(x)) return;
                    const ir::node& n = g.at(x);
                    if (!root && is_boundary(n.kind)) {
                        found.insert(x);
                        return;
                    }
                    walk(n.lhs, false);
                    walk(n.rhs, false);
                };
                walk(id, is_root);
            }

            arg_ref ensure_temp(int id) {
                auto found = temp_of.find(id);
                if (found != temp_of.end()) return {arg_ref::kind::temp, found->second};
                // The max of a softmax along a non-last axis comes with its
                // sum, from one read of the values.
                const int paired_sum = column_softmax_sum(id);
                if (paired_sum >= 0) {
                    ensure_temp(paired_sum);
                    found = temp_of.find(id);
                    if (found != temp_of.end()) return {arg_ref::kind::temp, found->second};
                }
                const int t = static_cast<int>(plan.temp_elems.size());
                plan.temp_elems.push_back(ir::numel(g.at(id).out));
                arg_ref dest{arg_ref::kind::temp, t};
                emit(id, dest);
                temp_of[id] = t;
                return dest;
            }

            void add_step(cg::kernel_code code, arg_ref dest) {
                step s;
                s.code = std::move(code);
                s.dest = dest;
                plan.steps.push_back(std::move(s));
            }

            // ---------------------------------------------------------
            // gemm
            // ---------------------------------------------------------
            int epilogue_matmul(int id) {
                // The single matmul (or batched matmul) reached from `id`
                // through elementwise nodes only (so the epilogue runs at
                // the product's own coordinates).
                std::set<int> found;
                std::set<int> seen;
                std::function<void(int)> walk = [&](int x) {
                    if (x < 0 || seen.count(x) || temp_of.count(x)) return;
                    seen.insert(x);
                    const ir::node& n = g.at(x);
                    if (is_product(n.kind)) {
                        found.insert(x);
                        return;
                    }
                    if (!is_elementwise(n.kind)) return;
                    walk(n.lhs);
                    walk(n.rhs);
                };
                walk(id);
                if (found.size() != 1) return -1;
                const int mm = *found.begin();
                if (g.at(mm).out != g.at(id).out) return -1;
                // Every path to the matmul must be elementwise: a view in
                // between would read the accumulator at other coordinates.
                std::set<std::pair<int, bool>> visited;
                bool via_view = false;
                std::function<void(int, bool)> check = [&](int x, bool view) {
                    if (x < 0 || temp_of.count(x) || via_view) return;
                    if (x == mm) {
                        if (view) via_view = true;
                        return;
                    }
                    const ir::node& n = g.at(x);
                    if (is_boundary(n.kind)) return;
                    const bool next = view || !is_elementwise(n.kind);
                    if (!visited.insert({x, view}).second) return;
                    check(n.lhs, next);
                    check(n.rhs, next);
                };
                check(id, false);
                if (via_view) return -1;
                return mm;
            }

            bool pure_view_of_input(int id) {
                const ir::node& n = g.at(id);
                if (temp_of.count(id)) return true;
                if (n.kind == ir::op::input) return true;
                if (n.kind == ir::op::slice || n.kind == ir::op::reshape ||
                    n.kind == ir::op::unsqueeze || n.kind == ir::op::transpose ||
                    n.kind == ir::op::permute || n.kind == ir::op::broadcast)
                    return pure_view_of_input(n.lhs);
                return false;
            }

            // Operand `id` of shape [rows, cols] or [batch, rows, cols]: a
            // strided view read in place, or a materialised temporary.
            // Whether node `id` reads node `target` (directly or not).
            bool depends_on(int id, int target) const {
                std::set<int> seen;
                std::function<bool(int)> walk = [&](int x) {
                    if (x < 0 || !seen.insert(x).second) return false;
                    if (x == target) return true;
                    const ir::node& n = g.at(x);
                    return walk(n.lhs) || walk(n.rhs);
                };
                return walk(id);
            }

            cg::gemm_operand operand(int id, const std::vector<int64_t>& shape) {
                const size_t rank = shape.size();
                if (pure_view_of_input(id)) {
                    cg::kexpr k;
                    cg::lowering low(g, k, shape);
                    bind_inputs(low);
                    const int root = low.at(id, low.identity());
                    const cg::knode& n = k.at(root);
                    if (n.op == cg::kop::load && n.index.is_affine) {
                        cg::gemm_operand op;
                        op.slot = n.slot;
                        op.offset = n.index.c0;
                        op.stride_batch = rank == 3 ? n.index.w[0] : 0;
                        op.stride_row = n.index.w[rank - 2];
                        op.stride_col = n.index.w[rank - 1];
                        return op;
                    }
                }
                const arg_ref t = ensure_temp(id);
                cg::gemm_operand op;
                op.slot = g.n_inputs + t.index;
                // the column softmax's sum sits after its max in their
                // shared temporary
                const auto off = offset_of.find(id);
                op.offset = off != offset_of.end() ? off->second : 0;
                op.stride_batch = rank == 3 ? shape[1] * shape[2] : 0;
                op.stride_row = shape[rank - 1];
                op.stride_col = 1;
                return op;
            }

            bool try_gemm(int id, arg_ref dest) {
                const int mm = epilogue_matmul(id);
                if (mm < 0) return false;
                const ir::node& m = g.at(mm);
                const std::vector<int64_t>& ls = g.at(m.lhs).out;
                const std::vector<int64_t>& rs = g.at(m.rhs).out;
                const bool batched = m.kind == ir::op::batched_matmul;
                const size_t o = batched ? 1 : 0; // leading batch axis
                const int64_t M = ls[o];
                const int64_t K = ls[o + 1];
                const int64_t N = rs[o + 1];
                cg::gemm_request r;
                r.batched = batched;
                r.batch = batched ? ls[0] : 1;
                r.m = M;
                r.n = N;
                r.k = K;
                r.a = operand(m.lhs, ls);
                r.b = operand(m.rhs, rs);
                // Other boundaries in the epilogue region.
                std::set<int> others;
                boundaries(id, others, {mm}, true);
                // A boundary that reads the product itself (softmax over a
                // product: its row max and sum) needs the product
                // materialised anyway; an epilogue would compute it a second
                // time.  Leave the region to the row or pointwise paths,
                // which read that one temporary.
                for (const int b : others)
                    if (depends_on(b, mm)) return false;
                for (const int b : others) ensure_temp(b);
                cg::kexpr k;
                cg::lowering low(g, k, m.out);
                bind_inputs(low);
                cg::binding acc;
                acc.what = cg::binding::kind::row_value;
                acc.row = 0;
                low.bound[mm] = acc;
                r.epilogue = low.at(id, low.identity());
                r.expr = &k;
                r.n_slots = n_slots();
                r.width = width;
                r.compute_units = compute_units;
                if (cg::gemm_wide(r)) {
                    const int64_t chunks = cg::gemm_wide_chunks(r);
                    if (chunks == 1) {
                        add_step(cg::emit_gemm_wide(r), dest);
                        return true;
                    }
                    const int t = static_cast<int>(plan.temp_elems.size());
                    plan.temp_elems.push_back(chunks * r.batch * r.m * r.n);
                    add_step(cg::emit_gemm_wide(r), {arg_ref::kind::temp, t});
                    cg::gemm_request c = r;
                    c.n_slots = n_slots();
                    add_step(cg::emit_gemm_combine(c, chunks, g.n_inputs + t), dest);
                    return true;
                }
                if (cg::gemm_few_rows(r)) {
                    // A few rows: chunks of K in parallel, their partial
                    // products summed by a second kernel (none with one chunk).
                    const int64_t partials = cg::gemm_few_rows_partials(r);
                    if (partials == 0) {
                        add_step(cg::emit_gemm_few_rows(r), dest);
                        return true;
                    }
                    const int t = static_cast<int>(plan.temp_elems.size());
                    plan.temp_elems.push_back(partials);
                    add_step(cg::emit_gemm_few_rows(r), {arg_ref::kind::temp, t});
                    cg::gemm_request c = r;
                    c.n_slots = n_slots();
                    add_step(cg::emit_gemm_combine(c, cg::gemm_few_rows_chunks(r), g.n_inputs + t), dest);
                    return true;
                }
                if (cg::gemm_narrow(r)) {
                    const int64_t chunks = cg::gemm_narrow_chunks(r);
                    if (chunks == 1) {
                        add_step(cg::emit_gemm_narrow(r), dest);
                        return true;
                    }
                    const int t = static_cast<int>(plan.temp_elems.size());
                    plan.temp_elems.push_back(chunks * r.batch * r.m * r.n);
                    add_step(cg::emit_gemm_narrow(r), {arg_ref::kind::temp, t});
                    cg::gemm_request c = r;
                    c.n_slots = n_slots();
                    add_step(cg::emit_gemm_combine(c, chunks, g.n_inputs + t), dest);
                    return true;
                }
                if (cg::gemm_few_cols(r)) {
                    add_step(cg::emit_gemm_few_cols(r), dest);
                    return true;
                }
                if (cg::gemm_band(r)) {
                    add_step(cg::emit_gemm_band(r), dest);
                    return true;
                }
                r.k_chunks = cg::gemm_k_chunks(r);
                if (r.k_chunks > 1) {
                    // Too few tiles for the machine: chunks of K in
                    // parallel, their partial products summed after.
                    const int t = static_cast<int>(plan.temp_elems.size());
                    plan.temp_elems.push_back(r.k_chunks * r.batch * r.m * r.n);
                    add_step(cg::emit_gemm(r), {arg_ref::kind::temp, t});
                    cg::gemm_request c = r;
                    c.n_slots = n_slots();
                    add_step(cg::emit_gemm_combine(c, r.k_chunks, g.n_inputs + t), dest);
                    return true;
                }
                add_step(cg::emit_gemm(r), dest);
                return true;
            }

            // ---------------------------------------------------------
            // row programs
            // ---------------------------------------------------------
            // Collects the row reductions under `id` (through elementwise
            // and view nodes).  Every reduction must reduce the last axis of
            // `row_shape` with keepdim and be consumed directly by a
            // broadcast back to `row_shape` that sits on an elementwise-only
            // path from a row-space root.  Returns false if the region does
            // not have that form.
            bool collect_row(int id, const std::vector<int64_t>& row_shape,
                             std::set<int>& reductions,
                             std::set<std::pair<int, bool>>& seen,
                             bool elementwise_path) {
                if (id < 0 || temp_of.count(id)) return true;
                // A node is checked once per kind of path that reaches it:
                // a reduction reached through a view must not be bound to
                // the row value.
                if (!seen.insert({id, elementwise_path}).second) return true;
                const ir::node& n = g.at(id);
                if (is_product(n.kind)) return true; // materialised
                if (ir::is_reduction(n.kind)) return false; // not via broadcast
                if (n.kind == ir::op::broadcast && elementwise_path &&
                    n.out == row_shape) {
                    const ir::node& child = g.at(n.lhs);
                    if (ir::is_reduction(child.kind) && !temp_of.count(n.lhs)) {
                        const ir::node& src = g.at(child.lhs);
                        const size_t last = row_shape.size() - 1;
                        if (!child.keepdim || src.out != row_shape ||
                            static_cast<size_t>(child.axis) != last)
                            return false;
                        if (!reductions.count(n.lhs)) {
                            reductions.insert(n.lhs);
                            std::set<std::pair<int, bool>> inner_seen;
                            if (!collect_row(child.lhs, row_shape, reductions,
                                             inner_seen, true))
                                return false;
                        }
                        return true;
                    }
                }
                const bool keeps = is_elementwise(n.kind);
                if (n.lhs >= 0 &&
                    !collect_row(n.lhs, row_shape, reductions, seen,
                                 elementwise_path && keeps))
                    return false;
                if (n.rhs >= 0 &&
                    !collect_row(n.rhs, row_shape, reductions, seen,
                                 elementwise_path && keeps))
                    return false;
                return true;
            }

            bool try_row(int id, arg_ref dest) {
                const ir::node& n = g.at(id);
                const bool reduce_output = ir::is_reduction(n.kind);
                const int producer = reduce_output ? n.lhs : id;
                const std::vector<int64_t> row_shape = g.at(producer).out;
                if (row_shape.empty()) return false;
                if (reduce_output &&
                    static_cast<size_t>(n.axis) != row_shape.size() - 1)
                    return false;
                std::set<int> reductions;
                std::set<std::pair<int, bool>> seen;
                if (!collect_row(producer, row_shape, reductions, seen, true)) return false;
                if (reductions.empty() && !reduce_output) return false;
                // Matmuls inside become temporaries first.
                std::set<int> mms;
                {
                    std::set<int> all;
                    boundaries(producer, all, {}, false);
                    for (const int r : reductions) boundaries(g.at(r).lhs, all, {}, false);
                    for (const int b : all) {
                        if (is_product(g.at(b).kind)) mms.insert(b);
                        else if (!reductions.count(b)) return false;
                    }
                }
                for (const int mm : mms) ensure_temp(mm);

                cg::kexpr k;
                cg::lowering low(g, k, row_shape);
                bind_inputs(low);
                std::vector<int> order(reductions.begin(), reductions.end());
                std::sort(order.begin(), order.end());
                for (size_t i = 0; i < order.size(); ++i) {
                    cg::binding b;
                    b.what = cg::binding::kind::row_value;
                    b.row = static_cast<int>(i);
                    low.bound[order[i]] = b;
                }
                cg::row_request r;
                r.expr = &k;
                r.shape = row_shape;
                for (const int red : order) {
                    cg::row_reduction rr;
                    rr.is_max = g.at(red).kind == ir::op::max;
                    // Lower the producer without the reduction's own binding
                    // in scope for itself (bindings only replace the
                    // reduction node, not its operand).
                    rr.producer = low.at(g.at(red).lhs, low.identity());
                    r.reductions.push_back(rr);
                }
                r.reduce_output = reduce_output;
                r.output_is_max = reduce_output && n.kind == ir::op::max;
                r.output = low.at(producer, low.identity());
                r.n_slots = n_slots();
                r.width = width;
                r.compute_units = compute_units;
                const int64_t pieces = cg::row_partial_parts(r);
                if (pieces > 1) {
                    // Few long rows folded into one value each: partials of
                    // the rows' pieces into a temporary, then per row.
                    int64_t rows = 1;
                    for (size_t d = 0; d + 1 < row_shape.size(); ++d) rows *= row_shape[d];
                    const int t = static_cast<int>(plan.temp_elems.size());
                    plan.temp_elems.push_back(rows * pieces);
                    add_step(cg::emit_row_partial(r), {arg_ref::kind::temp, t});
                    cg::row_request c = r;
                    c.n_slots = n_slots();
                    add_step(cg::emit_row_combine(c, g.n_inputs + t), dest);
                    return true;
                }
                const int64_t parts = cg::row_split_parts(r);
                if (parts > 0) {
                    // Rows split over workgroups exchange partials through a
                    // temporary that must read zero when the kernel starts.
                    const int t = static_cast<int>(plan.temp_elems.size());
                    plan.temp_elems.push_back(cg::row_split_temp_floats(r));
                    emit_zero_fill(t);
                    r.split_slot = g.n_inputs + t;
                    r.split_parts = parts;
                    r.n_slots = n_slots();
                    add_step(cg::emit_row_split(r), dest);
                    return true;
                }
                add_step(cg::emit_row(r), dest);
                return true;
            }

            // Zeros into temporary `t` with a fill kernel (not a memset, so
            // that a captured graph replays it like any other step).
            void emit_zero_fill(int t) {
                cg::kexpr k;
                cg::knode c;
                c.op = cg::kop::constant;
                c.value = 0.0F;
                cg::pointwise_request r;
                r.expr = &k;
                r.root = k.add(c);
                r.shape = {plan.temp_elems[static_cast<size_t>(t)]};
                r.n_slots = n_slots();
                r.width = width;
                r.compute_units = compute_units;
                add_step(cg::emit_pointwise(r), {arg_ref::kind::temp, t});
            }

            // ---------------------------------------------------------
            // softmax along a non-last axis
            // ---------------------------------------------------------
            // For a max node M = max(f, axis, keepdim) along a non-last
            // axis that is read only as exp(f - broadcast(M)), itself summed
            // along the same axis with keepdim (softmax's form, ops.cpp):
            // that sum node, else -1.  M then matters only through
            // exp(f - M), so the order-free max serves (emit_column_softmax).
            int column_softmax_sum(int max_id) const {
                const ir::node& m = g.at(max_id);
                if (m.kind != ir::op::max || !m.keepdim) return -1;
                const ir::node& f = g.at(m.lhs);
                if (f.out.size() < 2 || static_cast<size_t>(m.axis) + 1 == f.out.size()) return -1;
                auto only_user = [&](int x) {
                    const std::vector<int>& u = users[static_cast<size_t>(x)];
                    return u.size() == 1 ? u[0] : -1;
                };
                const int b = only_user(max_id);
                if (b < 0 || g.at(b).kind != ir::op::broadcast || g.at(b).out != f.out) return -1;
                const int d = only_user(b);
                if (d < 0 || g.at(d).kind != ir::op::subtract || g.at(d).lhs != m.lhs || g.at(d).rhs != b) return -1;
                const int e = only_user(d);
                if (e < 0 || g.at(e).kind != ir::op::exp) return -1;
                for (const int sum : users[static_cast<size_t>(e)]) {
                    const ir::node& sn = g.at(sum);
                    if (sn.kind == ir::op::sum && sn.lhs == e && sn.axis == m.axis && sn.keepdim && sum != g.root())
                        return sum;
                }
                return -1;
            }

            // The sum node of that form into temporary `dest`, with its max
            // beside it: M at [0, outputs), S at [outputs, 2 outputs).
            bool try_column_softmax(int id, arg_ref dest) {
                if (dest.what != arg_ref::kind::temp) return false;
                const ir::node& n = g.at(id);
                if (n.kind != ir::op::sum) return false;
                const ir::node& e = g.at(n.lhs);
                if (e.kind != ir::op::exp) return false;
                const ir::node& d = g.at(e.lhs);
                if (d.kind != ir::op::subtract || d.rhs < 0 || g.at(d.rhs).kind != ir::op::broadcast) return false;
                const int max_id = g.at(d.rhs).lhs;
                if (column_softmax_sum(max_id) != id || temp_of.count(max_id)) return false;
                const int f = g.at(max_id).lhs;
                std::set<int> inner;
                boundaries(f, inner, {}, false);
                for (const int b : inner) ensure_temp(b);
                const std::vector<int64_t>& shape = g.at(f).out;
                cg::kexpr k;
                cg::lowering low(g, k, shape);
                bind_inputs(low);
                cg::column_reduce_request r;
                r.expr = &k;
                r.producer = low.at(f, low.identity());
                r.shape = shape;
                r.axis = static_cast<size_t>(n.axis);
                r.n_slots = n_slots();
                r.width = width;
                const int64_t outputs = ir::numel(n.out);
                const int64_t parts = cg::column_reduce_parts(r, compute_units);
                plan.temp_elems[static_cast<size_t>(dest.index)] = 2 * outputs;
                if (parts < 2) {
                    add_step(cg::emit_column_softmax(r, -1), dest);
                }
                else {
                    r.parts = parts;
                    const int partial = static_cast<int>(plan.temp_elems.size());
                    plan.temp_elems.push_back(3 * parts * outputs);
                    add_step(cg::emit_column_softmax(r, -1), {arg_ref::kind::temp, partial});
                    cg::column_reduce_request c = r;
                    c.shape = {parts, outputs};
                    c.axis = 0;
                    c.parts = 1;
                    c.n_slots = n_slots();
                    // each strand merges at most 4 parts, as for the column
                    // reductions' second pass
                    c.max_cols = 64;
                    while (c.max_cols > 1 && (256 / c.max_cols) * 4 < parts) c.max_cols /= 2;
                    add_step(cg::emit_column_softmax(c, g.n_inputs + partial), dest);
                }
                temp_of[max_id] = dest.index;
                offset_of[max_id] = 0;
                offset_of[id] = outputs;
                return true;
            }

            // ---------------------------------------------------------
            // other reductions, pointwise
            // ---------------------------------------------------------
            void emit_reduction(int id, arg_ref dest) {
                if (try_column_softmax(id, dest)) return;
                const ir::node& n = g.at(id);
                std::set<int> inner;
                boundaries(n.lhs, inner, {}, false);
                for (const int b : inner) ensure_temp(b);
                const std::vector<int64_t>& shape = g.at(n.lhs).out;
                cg::kexpr k;
                cg::lowering low(g, k, shape);
                bind_inputs(low);
                const int producer = low.at(n.lhs, low.identity());
                if (static_cast<size_t>(n.axis) == shape.size() - 1) {
                    cg::row_request r;
                    r.expr = &k;
                    r.shape = shape;
                    r.reduce_output = true;
                    r.output_is_max = n.kind == ir::op::max;
                    r.output = producer;
                    r.n_slots = n_slots();
                    r.width = width;
                    r.compute_units = compute_units;
                    add_step(cg::emit_row(r), dest);
                    return;
                }
                cg::column_reduce_request r;
                r.expr = &k;
                r.producer = producer;
                r.shape = shape;
                r.axis = static_cast<size_t>(n.axis);
                r.is_max = n.kind == ir::op::max;
                r.n_slots = n_slots();
                r.width = width;
                // Few outputs over a long axis: fold chunks of the axis in
                // separate workgroups, then combine the partials.
                const int64_t outputs = ir::numel(n.out);
                const int64_t parts = cg::column_reduce_parts(r, compute_units);
                if (parts < 2) {
                    if (r.is_max) {
                        r.exact_expr = &k;
                        r.exact_producer = producer;
                        r.exact_shape = shape;
                        r.exact_axis = r.axis;
                    }
                    add_step(cg::emit_column_reduce(r), dest);
                    return;
                }
                r.parts = parts;
                const int partial = static_cast<int>(plan.temp_elems.size());
                plan.temp_elems.push_back(parts * outputs);
                add_step(cg::emit_column_reduce(r), {arg_ref::kind::temp, partial});
                // Second pass: fold the partials [parts, outputs] in order.
                cg::kexpr k2;
                cg::knode load;
                load.op = cg::kop::load;
                load.slot = g.n_inputs + partial;
                load.index = cg::ival::constant(0, 2);
                load.index.w = {outputs, 1};
                load.box = {{0, parts}, {0, outputs}};
                cg::column_reduce_request c;
                c.expr = &k2;
                c.producer = k2.add(load);
                c.shape = {parts, outputs};
                c.axis = 0;
                c.is_max = r.is_max;
                c.n_slots = n_slots();
                c.width = width;
                // Enough strands that each folds at most 4 partials: the
                // pass is a few dependent loads long instead of parts /
                // strands (a single workgroup over [1024, 256] partials
                // took 23.5 us).
                c.max_cols = 64;
                while (c.max_cols > 1 && (256 / c.max_cols) * 4 < parts) c.max_cols /= 2;
                if (r.is_max) {
                    c.exact_expr = &k;
                    c.exact_producer = producer;
                    c.exact_shape = shape;
                    c.exact_axis = r.axis;
                }
                add_step(cg::emit_column_reduce(c), dest);
            }

            void emit_pointwise(int id, arg_ref dest) {
                std::set<int> inner;
                boundaries(id, inner, {}, true);
                for (const int b : inner) ensure_temp(b);
                const std::vector<int64_t>& shape = g.at(id).out;
                cg::kexpr k;
                cg::lowering low(g, k, shape);
                bind_inputs(low);
                cg::pointwise_request r;
                r.expr = &k;
                r.root = low.at(id, low.identity());
                r.shape = shape;
                r.n_slots = n_slots();
                r.slot_elems = slot_elems();
                r.width = width;
                r.compute_units = compute_units;
                add_step(cg::emit_pointwise(r), dest);
            }

            // A reduction over an empty axis is its identity everywhere:
            // 0.0f for sum, -FLT_MAX for max (the values the reference's
            // block reduction starts from, src/tensor.cpp:900-901).
            void emit_identity_fill(int id, arg_ref dest) {
                const ir::node& n = g.at(id);
                cg::kexpr k;
                cg::knode c;
                c.op = cg::kop::constant;
                c.value = n.kind == ir::op::sum ? 0.0F : -3.40282346638528859812e+38F;
                cg::pointwise_request r;
                r.expr = &k;
                r.root = k.add(c);
                r.shape = n.out;
                r.n_slots = n_slots();
                r.width = width;
                add_step(cg::emit_pointwise(r), dest);
            }

            void emit(int id, arg_ref dest) {
                const ir::node& n = g.at(id);
                if (ir::numel(n.out) == 0) return;
                if (ir::is_reduction(n.kind) && ir::numel(g.at(n.lhs).out) == 0) {
                    emit_identity_fill(id, dest);
                    return;
                }
                if (try_gemm(id, dest)) return;
                if (try_row(id, dest)) return;
                if (ir::is_reduction(n.kind)) {
                    emit_reduction(id, dest);
                    return;
                }
                emit_pointwise(id, dest);
            }
        };

        struct plan_cache {
            std::mutex mutex;
            std::unordered_map<std::string, std::shared_ptr<graph_plan>> entries;
        };
        plan_cache& cache() {
            static plan_cache* instance = new plan_cache();
            return *instance;
        }

        int planning_compute_units() {
            try {
                return rt::device().compute_units;
            }
            catch (...) {
                return 256; // MI355X
            }
        }

    } // namespace

    std::string graph_plan::describe() const {
        std::ostringstream os;
        os << "{\"out_shape\":[";
        for (size_t i = 0; i < out_shape.size(); ++i) os << (i ? "," : "") << out_shape[i];
        os << "],\"temps\":[";
        for (size_t i = 0; i < temp_elems.size(); ++i) os << (i ? "," : "") << temp_elems[i];
        os << "],\"kernels\":[";
        for (size_t i = 0; i < steps.size(); ++i) {
            const step& s = steps[i];
            os << (i ? "," : "") << "{\"kind\":\"" << s.code.kind << "\",\"name\":\""
               << s.code.name << "\",\"grid\":[" << s.code.grid_x << ","
               << s.code.grid_y << "," << s.code.grid_z << "],\"block\":" << s.code.block
               << ",\"slots\":" << s.code.n_slots << ",\"dest\":\""
               << (s.dest.what == arg_ref::kind::output
                       ? std::string("output")
                       : "temp" + std::to_string(s.dest.index))
               << "\",\"source_bytes\":" << s.code.source.size()
               << ",\"code_bytes\":" << (s.object ? s.object->bytes.size() : 0) << "}";
        }
        os << "],\"codegen_ms\":" << codegen_ms << ",\"compile_ms\":" << compile_ms << "}";
        return os.str();
    }

    std::shared_ptr<graph_plan> build(const ir::graph& g, int compute_units) {
        const auto start = std::chrono::steady_clock::now();
        auto plan = std::make_shared<graph_plan>();
        const ir::node& root = g.at(g.root());
        plan->out_shape = root.out;
        plan->n_inputs = g.n_inputs;
        plan->input_elems.assign(static_cast<size_t>(g.n_inputs), 0);
        for (const ir::node& n : g.nodes) {
            if (n.kind == ir::op::input) {
                int64_t& need = plan->input_elems[static_cast<size_t>(n.input)];
                need = std::max(need, ir::numel(n.shape));
            }
        }
        builder b(g, *plan, compute_units);
        if (ir::numel(root.out) > 0) b.emit(g.root(), {arg_ref::kind::output, 0});
        plan->codegen_ms = rt::elapsed_ms(start);
        return plan;
    }

    void compile(graph_plan& plan) {
        const auto start = std::chrono::steady_clock::now();
        for (step& s : plan.steps) {
            if (!s.object) s.object = rt::compile(s.code.source, {});
        }
        plan.compile_ms = rt::elapsed_ms(start);
    }

    std::shared_ptr<graph_plan> lookup(const ir::graph& g, bool* hit) {
        const std::string key = ir::canonical_key(g);
        {
            std::scoped_lock lock{cache().mutex};
            auto found = cache().entries.find(key);
            if (found != cache().entries.end()) {
                if (hit) *hit = true;
                return found->second;
            }
        }
        if (hit) *hit = false;
        std::shared_ptr<graph_plan> plan = build(g, planning_compute_units());
        compile(*plan);
        {
            std::scoped_lock lock{rt::counters_mutex()};
            rt::counters().codegen_ms += plan->codegen_ms;
        }
        std::scoped_lock lock{cache().mutex};
        // Bounded like the code-object cache; plans in use stay alive
        // through their shared owners.
        if (cache().entries.size() >= 4096) cache().entries.clear();
        auto [it, inserted] = cache().entries.emplace(key, plan);
        return it->second;
    }

    void clear_cache() {
        std::scoped_lock lock{cache().mutex};
        cache().entries.clear();
    }

    namespace {
        void check_inputs(const graph_plan& plan, const std::vector<rt::buffer_state*>& inputs) {
            if (static_cast<int>(inputs.size()) < plan.n_inputs) {
            throw std::invalid_argument("graph needs more input buffers");
        }
            for (int i = 0; i < plan.n_inputs; ++i) {
                const int64_t need = plan.input_elems[static_cast<size_t>(i)];
                const rt::buffer_state* in = inputs[static_cast<size_t>(i)];
                const size_t have = in == nullptr ? 0 : in->bytes;
                if (need > 0 && have < static_cast<size_t>(need) * sizeof(float)) {
                    throw std::invalid_argument(
                        have == 0 ? "GPU kernel input is empty"
                                  : "input device buffer is too small"
                    );
                }
            }
        }

        // Loads the plan's modules (once) and orders the inputs' producers
        // before work on `s`.
        void prepare_launch(graph_plan& plan, const std::vector<rt::buffer_state*>& inputs,
                            const std::shared_ptr<rt::stream>& s) {
            {
                std::scoped_lock lock{plan.load_mutex};
                if (!plan.loaded) {
                    for (step& st : plan.steps)
                        st.kernel = rt::load_kernel(st.object, st.code.name);
                    plan.loaded = true;
                }
            }
            for (int i = 0; i < plan.n_inputs; ++i) {
                rt::buffer_state* in = inputs[static_cast<size_t>(i)];
                if (in != nullptr && in->bytes > 0) in->before_read(s);
            }
        }

        // The plan's kernels in order: slot i < n_inputs is input i, the
        // rest are the temporaries at `temps`, and each step writes `out`
        // or a temporary.
        void launch_steps(const graph_plan& plan, const std::vector<rt::buffer_state*>& inputs,
                          void* out, const std::vector<void*>& temps, const rt::stream& s,
                          hip::event_t start, hip::event_t stop) {
            std::vector<void*> pointers;
            std::vector<void*> params;
            for (size_t index = 0; index < plan.steps.size(); ++index) {
                const step& st = plan.steps[index];
                const int slots = st.code.n_slots;
                pointers.assign(static_cast<size_t>(slots) + 1, nullptr);
                for (int i = 0; i < slots; ++i) {
                    if (i < plan.n_inputs) {
                        rt::buffer_state* in = inputs[static_cast<size_t>(i)];
                        pointers[i] = in == nullptr ? nullptr : in->ptr;
                    }
                    else {
                        const size_t t = static_cast<size_t>(i - plan.n_inputs);
                        pointers[i] = t < temps.size() ? temps[t] : nullptr;
                    }
                }
                pointers[slots] = st.dest.what == arg_ref::kind::output
                                      ? out
                                      : temps[static_cast<size_t>(st.dest.index)];
                params.assign(pointers.size(), nullptr);
                for (size_t i = 0; i < pointers.size(); ++i) params[i] = &pointers[i];
                rt::launch(st.kernel, st.code.grid_x, st.code.grid_y, st.code.grid_z,
                           st.code.block, 0, params.data(), s,
                           index == 0 ? start : nullptr,
                           index + 1 == plan.steps.size() ? stop : nullptr);
            }
        }
    } // namespace

    std::shared_ptr<rt::buffer_state> run(
        graph_plan& plan, const std::vector<rt::buffer_state*>& inputs,
        const std::function<std::shared_ptr<rt::buffer_state>(size_t)>& allocate,
        hip::event_t start, hip::event_t stop
    ) {
        check_inputs(plan, inputs);
        const size_t out_bytes =
            static_cast<size_t>(ir::numel(plan.out_shape)) * sizeof(float);
        if (out_bytes == 0) return allocate(0);

        std::shared_ptr<rt::stream> s = rt::current_stream();
        prepare_launch(plan, inputs, s);
        std::shared_ptr<rt::buffer_state> out = allocate(out_bytes);
        std::vector<std::shared_ptr<rt::buffer_state>> temps;
        std::vector<void*> temp_ptrs;
        temps.reserve(plan.temp_elems.size());
        for (const int64_t elems : plan.temp_elems) {
            temps.push_back(std::make_shared<rt::buffer_state>(
                static_cast<size_t>(std::max<int64_t>(elems, 1)) * sizeof(float)
            ));
            temp_ptrs.push_back(temps.back()->ptr);
        }
        launch_steps(plan, inputs, out->ptr, temp_ptrs, *s, start, stop);
        out->after_write(s);
        // Temporaries are freed stream-ordered after the launches above.
        return out;
    }

    std::vector<size_t> workspace_layout(const graph_plan& plan, size_t* total) {
        std::vector<size_t> offsets;
        size_t at = 0;
        for (const int64_t elems : plan.temp_elems) {
            offsets.push_back(at);
            const size_t bytes = static_cast<size_t>(std::max<int64_t>(elems, 1)) * sizeof(float);
            at += (bytes + 255) / 256 * 256;
        }
        *total = at;
        return offsets;
    }

    void run_in_workspace(graph_plan& plan, const std::vector<rt::buffer_state*>& inputs,
                          rt::buffer_state& out, char* workspace, size_t workspace_bytes) {
        check_inputs(plan, inputs);
        const size_t out_bytes =
            static_cast<size_t>(ir::numel(plan.out_shape)) * sizeof(float);
        if (out_bytes == 0) return;
        if (out.bytes < out_bytes) throw std::invalid_argument("output device buffer is too small");
        size_t need = 0;
        const std::vector<size_t> offsets = workspace_layout(plan, &need);
        if (need > workspace_bytes)
            throw std::invalid_argument("the graph's temporaries need " + std::to_string(need) +
                                        " bytes of device workspace; " + std::to_string(workspace_bytes) +
                                        " are available");
        std::vector<void*> temp_ptrs;
        for (const size_t offset : offsets) temp_ptrs.push_back(workspace + offset);
        std::shared_ptr<rt::stream> s = rt::current_stream();
        prepare_launch(plan, inputs, s);
        // The output may still be read or written by work on other streams.
        out.before_write(s);
        launch_steps(plan, inputs, out.ptr, temp_ptrs, *s, nullptr, nullptr);
        out.after_write(s);
    }

} // namespace porch::plan
