// Pointwise kernel classes: flat (vectorised), tiled (LDS transpose) and
// scalar.  The reference launches one thread per output element with scalar
// loads and 64-bit div/mod index chains for every view (reference
// src/tensor.cpp:874-894, launched at src/cuda_jit.cpp:841-866); these
// kernels choose their shape from the composed leaf strides instead.

#include "codegen.hpp"
#include "emit_expr.hpp"

#include <algorithm>
#include <stdexcept>

namespace porch::cg {
    namespace {

        constexpr int block_threads = 256;
        constexpr int64_t max_grid = int64_t{1} << 22;

        std::vector<std::string> coordinate_names(size_t rank) {
            std::vector<std::string> names;
            for (size_t d = 0; d < rank; ++d) names.push_back("q" + std::to_string(d));
            return names;
        }

        std::string output_index(const std::vector<int64_t>& shape) {
            const std::vector<int64_t> strides = ir::contiguous_strides(shape);
            std::string s;
            for (size_t d = 0; d < shape.size(); ++d) {
                if (shape[d] == 1) continue;
                if (!s.empty()) s += " + ";
                s += "q" + std::to_string(d);
                if (strides[d] != 1) s += " * " + std::to_string(strides[d]);
            }
            return s.empty() ? "0" : s;
        }

        unsigned grid_for(int64_t items) {
            const int64_t blocks = (items + block_threads - 1) / block_threads;
            return static_cast<unsigned>(std::clamp<int64_t>(blocks, 1, max_grid));
        }

        // ---------------------------------------------------------------
        // scalar: one output per lane, any index map
        // ---------------------------------------------------------------
        kernel_code emit_scalar(const pointwise_request& r) {
            const size_t rank = r.shape.size();
            const int64_t count = ir::numel(r.shape);
            kernel_code kc;
            kc.kind = "pointwise.scalar";
            kc.name = "porch_pointwise";
            kc.n_slots = r.n_slots;
            kc.block = block_threads;
            kc.grid_x = grid_for(count);
            const char* T = r.width.type();
            std::string& s = kc.source;
            s = kernel_prologue(r.n_slots, T);
            s += "extern \"C\" __global__ void __launch_bounds__(256) porch_pointwise(" +
                 kernel_params(r.n_slots) + ") {\n";
            s += "    for (idx_t f = (idx_t)blockIdx.x * 256 + threadIdx.x; f < " +
                 std::to_string(count) + "; f += (idx_t)gridDim.x * 256) {\n";
            const std::vector<bool> used = used_coordinates(*r.expr, r.root, rank);
            s += decompose("f", r.shape, used, T, "        ");
            std::string body;
            emitter em(*r.expr, body, 1);
            em.indent = "        ";
            const std::vector<std::string> names = coordinate_names(rank);
            em.load = [&](int id) {
                const knode& n = r.expr->at(id);
                return std::vector<std::string>{
                    "a" + std::to_string(n.slot) + "[" + index_text(n.index, names) + "]"
                };
            };
            em.condition = [&](const kcond& c) {
                return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
            };
            em.row_value = [](int) -> std::string {
                throw std::logic_error("row value in a pointwise kernel");
            };
            const std::string v = em.emit(r.root)[0];
            s += body;
            s += "        out[f] = " + v + ";\n";
            s += "    }\n}\n";
            return kc;
        }

        // ---------------------------------------------------------------
        // flat: 4 consecutive outputs per lane, 128-bit where aligned
        // ---------------------------------------------------------------
        enum class flat_mode { none, row_vector, contiguous };

        flat_mode choose_flat(const pointwise_request& r) {
            const size_t rank = r.shape.size();
            const int64_t inner = r.shape[rank - 1];
            const std::vector<int64_t> ostrides = ir::contiguous_strides(r.shape);
            bool all_affine = true;
            bool contiguous_everywhere = true;
            bool uniform_selects = true;
            for (const int id : r.expr->postorder(r.root)) {
                const knode& n = r.expr->at(id);
                if (n.op == kop::load) {
                    if (!n.index.is_affine) {
                        all_affine = false;
                        continue;
                    }
                    if (n.index.is_constant()) continue;
                    for (size_t d = 0; d < rank; ++d) {
                        if (r.shape[d] != 1 && n.index.w[d] != ostrides[d])
                            contiguous_everywhere = false;
                    }
                }
                if (n.op == kop::select) {
                    contiguous_everywhere = false;
                    if (!n.cond.lhs.is_affine || n.cond.lhs.w[rank - 1] != 0)
                        uniform_selects = false;
                }
            }
            if (!all_affine) return flat_mode::none;
            if (inner % 4 == 0 && uniform_selects) return flat_mode::row_vector;
            if (contiguous_everywhere) return flat_mode::contiguous;
            return flat_mode::none;
        }

        kernel_code emit_flat(const pointwise_request& r, flat_mode mode) {
            const size_t rank = r.shape.size();
            const int64_t count = ir::numel(r.shape);
            const int64_t groups = count / 4;
            const int64_t tail = count % 4;
            const std::vector<int64_t> ostrides = ir::contiguous_strides(r.shape);
            kernel_code kc;
            kc.kind = "pointwise.flat";
            kc.name = "porch_pointwise";
            kc.n_slots = r.n_slots;
            kc.block = block_threads;
            kc.grid_x = grid_for(std::max<int64_t>(groups, 1));
            const char* T = r.width.type();
            const std::vector<std::string> names = coordinate_names(rank);
            std::string& s = kc.source;
            s = kernel_prologue(r.n_slots, T);
            s += "extern \"C\" __global__ void __launch_bounds__(256) porch_pointwise(" +
                 kernel_params(r.n_slots) + ") {\n";
            s += "    for (idx_t g = (idx_t)blockIdx.x * 256 + threadIdx.x; g < " +
                 std::to_string(groups) + "; g += (idx_t)gridDim.x * 256) {\n";
            s += "        const idx_t f = g * 4;\n";
            const std::vector<bool> used = used_coordinates(*r.expr, r.root, rank);
            if (mode == flat_mode::row_vector)
                s += decompose("f", r.shape, used, T, "        ");

            std::string body;
            emitter em(*r.expr, body, 4);
            em.indent = "        ";
            em.condition = [&](const kcond& c) {
                return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
            };
            em.row_value = [](int) -> std::string {
                throw std::logic_error("row value in a pointwise kernel");
            };
            em.load = [&](int id) {
                const knode& n = r.expr->at(id);
                const std::string base = "a" + std::to_string(n.slot);
                std::vector<std::string> lanes(4);
                if (n.index.is_constant()) {
                    const std::string v = em.fresh("u");
                    em.line("const float " + v + " = " + base + "[" +
                            std::to_string(n.index.c0) + "];");
                    for (auto& lane : lanes) lane = v;
                    return lanes;
                }
                std::string idx;
                int64_t step = 0;
                bool aligned = false;
                if (mode == flat_mode::contiguous) {
                    idx = n.index.c0 == 0 ? "f"
                                          : "(f + " + std::to_string(n.index.c0) + ")";
                    step = 1;
                    aligned = n.index.c0 % 4 == 0;
                }
                else {
                    idx = index_text(n.index, names);
                    step = n.index.w[rank - 1];
                    aligned = step == 1 && n.index.c0 % 4 == 0;
                    for (size_t d = 0; d + 1 < rank && aligned; ++d) {
                        if (n.index.w[d] % 4 != 0) aligned = false;
                    }
                }
                if (step == 0) {
                    const std::string v = em.fresh("u");
                    em.line("const float " + v + " = " + base + "[" + idx + "];");
                    for (auto& lane : lanes) lane = v;
                    return lanes;
                }
                if (step == 1 && aligned) {
                    const std::string v = em.fresh("w");
                    em.line("const float4 " + v + " = *reinterpret_cast<const float4*>(" +
                            base + " + " + idx + ");");
                    lanes = {v + ".x", v + ".y", v + ".z", v + ".w"};
                    return lanes;
                }
                const std::string p = em.fresh("p");
                em.line("const float* " + p + " = " + base + " + " + idx + ";");
                for (int e = 0; e < 4; ++e) {
                    lanes[e] = p + "[" + std::to_string(step * e) + "]";
                }
                return lanes;
            };
            const std::vector<std::string> v = em.emit(r.root);
            s += body;
            s += "        *reinterpret_cast<float4*>(out + f) = make_float4(" + v[0] +
                 ", " + v[1] + ", " + v[2] + ", " + v[3] + ");\n";
            s += "    }\n";
            if (tail != 0) {
                // Remaining count % 4 outputs, one per lane.
                s += "    if (blockIdx.x == 0 && threadIdx.x < " + std::to_string(tail) +
                     ") {\n";
                s += "        const idx_t f = " + std::to_string(groups * 4) +
                     " + threadIdx.x;\n";
                s += decompose("f", r.shape, used, T, "        ");
                std::string tail_body;
                emitter te(*r.expr, tail_body, 1);
                te.indent = "        ";
                te.condition = em.condition;
                te.row_value = em.row_value;
                te.load = [&](int id) {
                    const knode& n = r.expr->at(id);
                    return std::vector<std::string>{
                        "a" + std::to_string(n.slot) + "[" + index_text(n.index, names) + "]"
                    };
                };
                const std::string tv = te.emit(r.root)[0];
                s += tail_body;
                s += "        out[f] = " + tv + ";\n";
                s += "    }\n";
            }
            s += "}\n";
            return kc;
        }

        // ---------------------------------------------------------------
        // tiled: LDS transpose for leaves strided along the output's
        // contiguous dimension
        // ---------------------------------------------------------------
        constexpr int tile = 64;

        struct tiling {
            int p = -1;                 // coordinate the staged leaves run along
            std::vector<int> staged;    // kexpr roots evaluated in phase 1
        };

        tiling choose_tiling(const pointwise_request& r) {
            tiling t;
            const size_t rank = r.shape.size();
            if (rank < 2) return t;
            const size_t q = rank - 1;
            if (r.shape[q] < 2) return t;
            // Score each candidate p by the transposed leaves it makes
            // contiguous-ish (|w_p| <= 4).
            int best = -1;
            int best_score = 0;
            for (size_t p = 0; p < q; ++p) {
                if (r.shape[p] < 2) continue;
                int score = 0;
                for (const int id : r.expr->loads(r.root)) {
                    const ival& x = r.expr->at(id).index;
                    if (!x.is_affine) continue;
                    if (x.w[q] == 0 || x.w[q] == 1) continue;
                    if (x.w[p] >= 1 && x.w[p] <= 4) ++score;
                }
                if (score > best_score ||
                    (score == best_score && score > 0 && static_cast<int>(p) > best)) {
                    best = static_cast<int>(p);
                    best_score = score;
                }
            }
            if (best < 0 || best_score == 0) return t;
            t.p = best;
            const size_t p = static_cast<size_t>(best);
            // friendly: every load below is not unit-stride along q (and
            // affine); beneficial: some load is transposed and close along p.
            const std::vector<int> order = r.expr->postorder(r.root);
            std::vector<char> friendly(r.expr->nodes.size(), 0);
            std::vector<char> beneficial(r.expr->nodes.size(), 0);
            for (const int id : order) {
                const knode& n = r.expr->at(id);
                switch (n.op) {
                    case kop::load: {
                        const ival& x = n.index;
                        friendly[id] = x.is_affine && x.w[q] != 1;
                        beneficial[id] = x.is_affine && x.w[q] != 0 && x.w[q] != 1 &&
                                         x.w[p] >= 1 && x.w[p] <= 4;
                        break;
                    }
                    case kop::constant:
                        friendly[id] = 1;
                        break;
                    case kop::row_value:
                        friendly[id] = 0;
                        break;
                    default: {
                        bool f = true;
                        bool b = false;
                        if (n.a >= 0) {
                            f = f && friendly[n.a];
                            b = b || beneficial[n.a];
                        }
                        if (n.b >= 0) {
                            f = f && friendly[n.b];
                            b = b || beneficial[n.b];
                        }
                        if (n.op == kop::select && !n.cond.lhs.is_affine) f = false;
                        friendly[id] = f;
                        beneficial[id] = b;
                    }
                }
            }
            // Maximal friendly+beneficial subtrees, from the root down.
            std::vector<int> stack{r.root};
            std::vector<char> visited(r.expr->nodes.size(), 0);
            while (!stack.empty()) {
                const int id = stack.back();
                stack.pop_back();
                if (id < 0 || visited[id]) continue;
                visited[id] = 1;
                if (friendly[id] && beneficial[id]) {
                    t.staged.push_back(id);
                    continue;
                }
                const knode& n = r.expr->at(id);
                stack.push_back(n.a);
                stack.push_back(n.b);
            }
            if (t.staged.empty() || t.staged.size() > 8) t.p = -1;
            return t;
        }

        kernel_code emit_tiled(const pointwise_request& r, const tiling& t) {
            const size_t rank = r.shape.size();
            const size_t q = rank - 1;
            const size_t p = static_cast<size_t>(t.p);
            const int64_t ntq = (r.shape[q] + tile - 1) / tile;
            const int64_t ntp = (r.shape[p] + tile - 1) / tile;
            std::vector<int64_t> other_shape;
            std::vector<size_t> other_dims;
            for (size_t d = 0; d < rank; ++d) {
                if (d == p || d == q) continue;
                other_shape.push_back(r.shape[d]);
                other_dims.push_back(d);
            }
            const int64_t others = ir::numel(other_shape);
            kernel_code kc;
            kc.kind = "pointwise.tiled";
            kc.name = "porch_tiled";
            kc.n_slots = r.n_slots;
            kc.block = block_threads;
            kc.grid_x = static_cast<unsigned>(ntq * ntp * others);
            const char* T = r.width.type();
            const std::vector<std::string> names = coordinate_names(rank);
            const std::string qs = "q" + std::to_string(q);
            const std::string ps = "q" + std::to_string(p);
            const size_t n_stage = t.staged.size();

            std::string& s = kc.source;
            s = kernel_prologue(r.n_slots, T);
            s += "extern \"C\" __global__ void __launch_bounds__(256) porch_tiled(" +
                 kernel_params(r.n_slots) + ") {\n";
            s += "    __shared__ float stage[" + std::to_string(n_stage) + "][" +
                 std::to_string(tile) + "][" + std::to_string(tile + 1) + "];\n";
            s += "    const idx_t tile_id = blockIdx.x;\n";
            s += "    const idx_t tq = tile_id % " + std::to_string(ntq) + ";\n";
            s += "    const idx_t tp = (tile_id / " + std::to_string(ntq) + ") % " +
                 std::to_string(ntp) + ";\n";
            s += "    const idx_t rest = tile_id / " + std::to_string(ntq * ntp) + ";\n";
            // Coordinates of the other dimensions, from `rest`.
            {
                const std::vector<int64_t> ostr = ir::contiguous_strides(other_shape);
                for (size_t i = 0; i < other_dims.size(); ++i) {
                    std::string value;
                    if (other_shape[i] == 1) value = "0";
                    else if (i == 0) value = "rest / " + std::to_string(ostr[i]);
                    else
                        value = "(rest / " + std::to_string(ostr[i]) + ") % " +
                                std::to_string(other_shape[i]);
                    s += "    const idx_t q" + std::to_string(other_dims[i]) + " = " +
                         value + ";\n";
                }
                if (other_dims.empty()) s += "    (void)rest;\n";
            }
            s += "    const int tid = threadIdx.x;\n";

            auto load_fn = [&](emitter& em) {
                return [&r, &names, &em](int id) {
                    (void)em;
                    const knode& n = r.expr->at(id);
                    return std::vector<std::string>{
                        "a" + std::to_string(n.slot) + "[" + index_text(n.index, names) + "]"
                    };
                };
            };
            auto cond_fn = [&](const kcond& c) {
                return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
            };
            auto in_range = ps + " < " + std::to_string(r.shape[p]) + " && " + qs +
                            " < " + std::to_string(r.shape[q]);

            // Phase 1: lanes along p (the staged leaves' near-contiguous dim).
            s += "    #pragma unroll 4\n";
            s += "    for (int it = 0; it < " + std::to_string(tile * tile / block_threads) +
                 "; ++it) {\n";
            s += "        const int pl = tid & " + std::to_string(tile - 1) + ";\n";
            s += "        const int ql = (tid >> 6) + it * " +
                 std::to_string(block_threads / tile) + ";\n";
            s += "        const idx_t " + ps + " = tp * " + std::to_string(tile) + " + pl;\n";
            s += "        const idx_t " + qs + " = tq * " + std::to_string(tile) + " + ql;\n";
            s += "        if (" + in_range + ") {\n";
            {
                std::string body;
                emitter em(*r.expr, body, 1);
                em.indent = "            ";
                em.load = load_fn(em);
                em.condition = cond_fn;
                em.row_value = [](int) -> std::string {
                    throw std::logic_error("row value in a pointwise kernel");
                };
                for (size_t i = 0; i < n_stage; ++i) {
                    const std::string v = em.emit(t.staged[i])[0];
                    em.line("stage[" + std::to_string(i) + "][pl][ql] = " + v + ";");
                }
                s += body;
            }
            s += "        }\n    }\n";
            s += "    __syncthreads();\n";
            // Phase 2: lanes along q (the output's contiguous dim).
            s += "    #pragma unroll 4\n";
            s += "    for (int it = 0; it < " + std::to_string(tile * tile / block_threads) +
                 "; ++it) {\n";
            s += "        const int ql = tid & " + std::to_string(tile - 1) + ";\n";
            s += "        const int pl = (tid >> 6) + it * " +
                 std::to_string(block_threads / tile) + ";\n";
            s += "        const idx_t " + ps + " = tp * " + std::to_string(tile) + " + pl;\n";
            s += "        const idx_t " + qs + " = tq * " + std::to_string(tile) + " + ql;\n";
            s += "        if (" + in_range + ") {\n";
            {
                std::string body;
                emitter em(*r.expr, body, 1);
                em.indent = "            ";
                em.load = load_fn(em);
                em.condition = cond_fn;
                em.row_value = [](int) -> std::string {
                    throw std::logic_error("row value in a pointwise kernel");
                };
                em.override_node = [&](int id) -> std::vector<std::string> {
                    for (size_t i = 0; i < n_stage; ++i) {
                        if (t.staged[i] == id)
                            return {"stage[" + std::to_string(i) + "][pl][ql]"};
                    }
                    return {};
                };
                const std::string v = em.emit(r.root)[0];
                s += body;
                s += "            out[" + output_index(r.shape) + "] = " + v + ";\n";
            }
            s += "        }\n    }\n}\n";
            return kc;
        }

    } // namespace

    kernel_code emit_pointwise(const pointwise_request& r) {
        if (r.shape.empty()) throw std::logic_error("pointwise kernel of rank 0");
        const tiling t = choose_tiling(r);
        if (t.p >= 0) return emit_tiled(r, t);
        const flat_mode mode = choose_flat(r);
        if (mode != flat_mode::none && ir::numel(r.shape) >= 4) return emit_flat(r, mode);
        return emit_scalar(r);
    }

} // namespace porch::cg
