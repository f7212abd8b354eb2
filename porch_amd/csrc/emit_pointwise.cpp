// Pointwise kernel classes: flat (vectorised), tiled (LDS transpose) and
// scalar.  The reference launches one thread per output element with scalar
// loads and 64-bit div/mod index chains for every view (reference
// src/tensor.cpp:874-894, launched at src/cuda_jit.cpp:841-866); these
// kernels choose their shape from the composed leaf strides instead.

#include "codegen.hpp"
#include "emit_expr.hpp"

#include <algorithm>
#include <functional>
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
                 std::to_string(count) + "; f += " + std::to_string(int64_t{kc.grid_x} * 256) + ") {\n";
            const std::vector<bool> used = used_coordinates(*r.expr, r.root, rank);
            s += decompose("f", r.shape, used, T, "        ");
            std::string body;
            emitter em(*r.expr, body, 1);
            em.indent = "        ";
            em.declare_roots({r.root});
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

        bool uniform_over(const kcond& c, size_t d, int64_t v);

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
                    // the same branch for each group of 4 along the row (a
                    // concat along the last axis at a multiple of 4): the
                    // condition is evaluated once, at the group's first
                    // element
                    if (!uniform_over(n.cond, rank - 1, 4)) uniform_selects = false;
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
            // the stride is the launch's lane count, a constant: no
            // implicit kernel argument is read, and a grid that covers every
            // group runs the body once
            s += "    for (idx_t g = (idx_t)blockIdx.x * 256 + threadIdx.x; g < " +
                 std::to_string(groups) + "; g += " + std::to_string(int64_t{kc.grid_x} * 256) + ") {\n";
            const std::string ind = "        ";
            s += ind + "const idx_t f = g * 4;\n";
            const std::vector<bool> used = used_coordinates(*r.expr, r.root, rank);
            if (mode == flat_mode::row_vector)
                s += decompose("f", r.shape, used, T, ind);

            std::string body;
            emitter em(*r.expr, body, 4);
            em.indent = ind;
            em.declare_roots({r.root});
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
                    // A leaf read once per element (no broadcast dimension)
                    // streams: a non-temporal load keeps it from displacing
                    // reused lines (a 256 MiB copy measured 86.2 -> 76.2 us).
                    bool streaming = true;
                    for (size_t d = 0; d < rank; ++d) {
                        if (r.shape[d] > 1 && n.index.w[d] == 0) streaming = false;
                    }
                    if (streaming)
                        em.line("const porch_v4f " + v + " = __builtin_nontemporal_load(" +
                                "reinterpret_cast<const porch_v4f*>(" + base + " + " + idx + "));");
                    else
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
            s += ind + "*reinterpret_cast<float4*>(out + f) = make_float4(" + v[0] +
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
                te.declare_roots({r.root});
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
        // Tiles are 64 (q) x 64 or 128 (p) outputs; see emit_tiled.
        constexpr int tile_q = 64;

        struct tiling {
            int p = -1;                 // coordinate the staged leaves run along
            std::vector<int> staged;    // kexpr roots evaluated in phase 1
            // Per staged root: the selects above it and the branch each must
            // take (true: the first operand) for its value to be used.
            std::vector<std::vector<std::pair<kcond, bool>>> guards;
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
            if (t.staged.empty() || t.staged.size() > 8) {
                t.p = -1;
                return t;
            }
            // Phase 1 computes the staged values ahead of the selects above
            // them, so each is computed only where those selects take its
            // branch: elsewhere its loads may fall outside their buffers.
            // A staged root reached along more than one path, or through a
            // select with a non-affine condition, is not staged.
            t.guards.assign(t.staged.size(), {});
            std::vector<char> reached(t.staged.size(), 0);
            std::vector<std::pair<kcond, bool>> path;
            int visits = 0;
            bool ok = true;
            std::function<void(int)> walk = [&](int id) {
                if (!ok || id < 0) return;
                if (++visits > 4096) {
                    ok = false;
                    return;
                }
                for (size_t i = 0; i < t.staged.size(); ++i) {
                    if (t.staged[i] != id) continue;
                    if (reached[i]) ok = false;
                    reached[i] = 1;
                    t.guards[i] = path;
                    return;
                }
                const knode& n = r.expr->at(id);
                if (n.op == kop::select) {
                    if (!n.cond.lhs.is_affine) {
                        ok = ok && r.expr->loads(id).empty();
                        return;
                    }
                    path.emplace_back(n.cond, true);
                    walk(n.a);
                    path.back().second = false;
                    walk(n.b);
                    path.pop_back();
                    return;
                }
                walk(n.a);
                walk(n.b);
            };
            walk(r.root);
            if (!ok) t.p = -1;
            return t;
        }

        // Nodes of the staged subtrees (phase 1) and of the rest (phase 2).
        std::vector<char> staged_mask(const kexpr& k, const tiling& t) {
            std::vector<char> in(k.nodes.size(), 0);
            for (const int root : t.staged)
                for (const int id : k.postorder(root)) in[id] = 1;
            return in;
        }

        // Is select condition `c` the same for the `v` consecutive values
        // q_d = v*j .. v*j + v-1 of coordinate d, wherever it is evaluated?
        bool uniform_over(const kcond& c, size_t d, int64_t v) {
            if (!c.lhs.is_affine) return false;
            const int64_t w = c.lhs.w[d];
            if (w == 0 || v == 1) return true;
            if (w != 1) return false;
            for (size_t e = 0; e < c.lhs.w.size(); ++e)
                if (e != d && c.lhs.w[e] % v != 0) return false;
            return ((c.bound - c.lhs.c0) % v + v) % v == 0;
        }

        // A load of `v` elements spaced w[d] apart along coordinate d (the
        // first at a multiple of v) read as one aligned float2/float4.
        struct vector_load {
            bool ok = false;
            int width = 1;   // floats per vector load
            int64_t m = 0;   // offset of the first element inside the vector
            int64_t step = 0;
        };

        vector_load plan_vector_load(const knode& n, size_t d, int64_t v,
                                     const std::vector<int64_t>& slot_elems) {
            vector_load out;
            const ival& x = n.index;
            if (!x.is_affine || v == 1) return out;
            const int64_t s = x.w[d];
            if (s <= 0) return out;
            const int64_t wv = s * v;
            if (wv != 2 && wv != 4) return out;
            for (size_t e = 0; e < x.w.size(); ++e)
                if (e != d && x.w[e] % wv != 0) return out;
            const int64_t m = ((x.c0 % wv) + wv) % wv;
            if (m + s * (v - 1) > wv - 1) return out;
            // Every vector read stays inside the slot's buffer: evaluate the
            // index over the load's box with q_d at multiples of v.
            if (n.slot < 0 || static_cast<size_t>(n.slot) >= slot_elems.size()) return out;
            int64_t lo = x.c0;
            int64_t hi = x.c0;
            for (size_t e = 0; e < x.w.size(); ++e) {
                int64_t a = n.box[e].first;
                int64_t b = n.box[e].second - 1;
                if (e == d) {
                    a = (a + v - 1) / v * v;
                    b = b / v * v;
                }
                if (b < a) return out;
                lo += std::min(x.w[e] * a, x.w[e] * b);
                hi += std::max(x.w[e] * a, x.w[e] * b);
            }
            if (lo - m < 0 || hi - m + wv - 1 > slot_elems[static_cast<size_t>(n.slot)] - 1)
                return out;
            out.ok = true;
            out.width = static_cast<int>(wv);
            out.m = m;
            out.step = s;
            return out;
        }

        const char* lane_name(int64_t i) {
            static const char* names[] = {".x", ".y", ".z", ".w"};
            return names[i];
        }

        kernel_code emit_tiled(const pointwise_request& r, const tiling& t) {
            const kexpr& k = *r.expr;
            const size_t rank = r.shape.size();
            const size_t q = rank - 1;
            const size_t p = static_cast<size_t>(t.p);
            const int64_t extent_p = r.shape[p];
            const int64_t extent_q = r.shape[q];
            const size_t n_stage = t.staged.size();
            std::vector<int64_t> other_shape;
            std::vector<size_t> other_dims;
            for (size_t d = 0; d < rank; ++d) {
                if (d == p || d == q) continue;
                other_shape.push_back(r.shape[d]);
                other_dims.push_back(d);
            }
            const int64_t others = ir::numel(other_shape);
            const std::vector<char> in_stage = staged_mask(k, t);
            std::vector<int> tiled_roots(t.staged.begin(), t.staged.end());
            tiled_roots.push_back(r.root);

            // Phase 1 width: elements per lane along p.
            int64_t V = 1;
            for (const int64_t v : {int64_t{4}, int64_t{2}}) {
                if (extent_p % v != 0) continue;
                bool uniform = true;
                for (const auto& guard : t.guards)
                    for (const auto& [c, branch] : guard)
                        if (!uniform_over(c, p, v)) uniform = false;
                bool useful = false;
                for (size_t id = 0; id < k.nodes.size(); ++id) {
                    if (!in_stage[id]) continue;
                    const knode& n = k.at(static_cast<int>(id));
                    if (n.op == kop::select && !uniform_over(n.cond, p, v)) uniform = false;
                    if (n.op == kop::load && !n.index.is_affine) uniform = false;
                    if (n.op == kop::load && plan_vector_load(n, p, v, r.slot_elems).ok)
                        useful = true;
                }
                if (uniform && useful) {
                    V = v;
                    break;
                }
            }
            // 128 outputs along p where phase 1 reads one unit-stride leaf
            // (128-bit loads) into one stage: it then reads 512 B of each
            // source row per tile instead of 256 B, and the stage (33 KB)
            // still leaves room for four workgroups per compute unit.
            // Measured (trace means): x^T over [4096, 4096] 27.0 -> 23.2 us,
            // x^T + y 40.4 -> 36.8, x^T * y + z 54.7 -> 51.9.  Not with two
            // transposed leaves (x^T + y^T: 38.4 -> 41.5) nor stride-2 reads,
            // which already cover 512 B (the view chain: 18.0 -> 22.4).
            int phase1_leaves = 0;
            for (size_t id = 0; id < k.nodes.size(); ++id) {
                const knode& n = k.at(static_cast<int>(id));
                if (in_stage[id] && n.op == kop::load && (!n.index.is_affine || n.index.w[p] != 0)) ++phase1_leaves;
            }
            const int64_t tile_p = (n_stage == 1 && V == 4 && phase1_leaves == 1 && extent_p >= 128) ? 128 : 64;
            const int64_t ntq = (extent_q + tile_q - 1) / tile_q;
            const int64_t ntp = (extent_p + tile_p - 1) / tile_p;

            // Phase 2 width: outputs per lane along q (128-bit stores).
            int64_t W = (extent_q % 4 == 0) ? 4 : 1;
            {
                std::vector<char> phase2(k.nodes.size(), 0);
                std::vector<int> stack{r.root};
                while (!stack.empty()) {
                    const int id = stack.back();
                    stack.pop_back();
                    if (id < 0 || phase2[id]) continue;
                    bool staged_root = false;
                    for (const int sroot : t.staged) staged_root = staged_root || sroot == id;
                    phase2[id] = 1;
                    if (staged_root) continue;
                    const knode& n = k.at(id);
                    if (n.op == kop::select && !uniform_over(n.cond, q, W)) W = 1;
                    if (n.op == kop::load && !n.index.is_affine) W = 1;
                    stack.push_back(n.a);
                    stack.push_back(n.b);
                }
            }
            // Selects of the staged subtrees decided once per tile (up to 2).
            std::vector<int> hoisted;
            for (size_t id = 0; id < k.nodes.size() && hoisted.size() < 2; ++id) {
                const knode& n = k.at(static_cast<int>(id));
                if (in_stage[id] && n.op == kop::select && n.cond.lhs.is_affine)
                    hoisted.push_back(static_cast<int>(id));
            }

            // A leaf whose every element is read once by this kernel (no
            // broadcast dimension) streams past the caches: non-temporal
            // loads keep it from evicting data that is reused.
            auto streaming = [&](const knode& n) {
                if (!n.index.is_affine) return false;
                for (size_t d = 0; d < rank; ++d) {
                    if (r.shape[d] > 1 && n.index.w[d] == 0) return false;
                }
                return true;
            };

            kernel_code kc;
            kc.kind = "pointwise.tiled";
            kc.name = "porch_tiled";
            kc.n_slots = r.n_slots;
            kc.block = block_threads;
            // Persistent workgroups (at most four per compute unit) walk the
            // tiles: a workgroup's reads of its next tile overlap other
            // workgroups' stores instead of the whole chip reading, then
            // writing, in step.
            const int64_t tiles = ntq * ntp * others;
            const int64_t resident = static_cast<int64_t>(std::max(r.compute_units, 1)) * 4;
            const bool persistent = tiles > resident;
            kc.grid_x = static_cast<unsigned>(persistent ? resident : tiles);
            const char* T = r.width.type();
            const std::vector<std::string> names = coordinate_names(rank);
            const std::string qs = "q" + std::to_string(q);
            const std::string ps = "q" + std::to_string(p);

            std::string& s = kc.source;
            s = kernel_prologue(r.n_slots, T);
            s += "extern \"C\" __global__ void __launch_bounds__(256) porch_tiled(" +
                 kernel_params(r.n_slots) + ") {\n";
            s += "    __shared__ float stage[" + std::to_string(n_stage) + "][" + std::to_string(tile_p) + "][" +
                 std::to_string(tile_q + 1) + "];\n";
            // Consecutive workgroups walk along p: neighbouring tiles read
            // neighbouring segments of the same source rows.
            if (persistent)
                s += "    for (idx_t tile_id = blockIdx.x; tile_id < " + std::to_string(tiles) +
                     "; tile_id += gridDim.x) {\n";
            else
                s += "    { const idx_t tile_id = blockIdx.x;\n";
            s += "    const idx_t tp = tile_id % " + std::to_string(ntp) + ";\n";
            s += "    const idx_t tq = (tile_id / " + std::to_string(ntp) + ") % " +
                 std::to_string(ntq) + ";\n";
            s += "    const idx_t rest = tile_id / " + std::to_string(ntq * ntp) + ";\n";
            {
                const std::vector<int64_t> ostr = ir::contiguous_strides(other_shape);
                for (size_t i = 0; i < other_dims.size(); ++i) {
                    std::string value;
                    if (other_shape[i] == 1) value = "0";
                    else if (i == 0) value = "rest / " + std::to_string(ostr[i]);
                    else
                        value = "(rest / " + std::to_string(ostr[i]) + ") % " +
                                std::to_string(other_shape[i]);
                    s += "    const idx_t q" + std::to_string(other_dims[i]) + " = " + value + ";\n";
                }
                if (other_dims.empty()) s += "    (void)rest;\n";
            }
            s += "    const idx_t pbase = tp * " + std::to_string(tile_p) + ";\n";
            s += "    const idx_t qbase = tq * " + std::to_string(tile_q) + ";\n";
            s += "    const int tid = threadIdx.x;\n";

            // Per-tile decision of the hoisted selects: 1 = first branch on
            // the whole tile, 2 = second branch, 0 = mixed.
            for (size_t h = 0; h < hoisted.size(); ++h) {
                const kcond& c = k.at(hoisted[h]).cond;
                std::string lo = std::to_string(c.lhs.c0);
                std::string hi = lo;
                for (size_t d = 0; d < rank; ++d) {
                    const int64_t w = c.lhs.w[d];
                    if (w == 0) continue;
                    std::string a, b;
                    if (d == p) {
                        a = "pbase";
                        b = "(pbase + " + std::to_string(tile_p - 1) + " < " + std::to_string(extent_p) +
                            " ? pbase + " + std::to_string(tile_p - 1) + " : (idx_t)" +
                            std::to_string(extent_p - 1) + ")";
                    }
                    else if (d == q) {
                        a = "qbase";
                        b = "(qbase + " + std::to_string(tile_q - 1) + " < " + std::to_string(extent_q) +
                            " ? qbase + " + std::to_string(tile_q - 1) + " : (idx_t)" +
                            std::to_string(extent_q - 1) + ")";
                    }
                    else {
                        a = b = "q" + std::to_string(d);
                    }
                    const std::string ws = std::to_string(w);
                    lo += " + " + ws + " * " + (w > 0 ? a : b);
                    hi += " + " + ws + " * " + (w > 0 ? b : a);
                }
                const std::string H = std::to_string(h);
                s += "    const idx_t lo" + H + " = " + lo + ";\n";
                s += "    const idx_t hi" + H + " = " + hi + ";\n";
                s += "    const int mode" + H + " = (hi" + H + " < " + std::to_string(c.bound) +
                     ") ? 1 : ((lo" + H + " >= " + std::to_string(c.bound) + ") ? 2 : 0);\n";
            }

            auto cond_fn = [&](const kcond& c) {
                return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
            };
            const bool full_p = extent_p % tile_p == 0;
            const bool full_q = extent_q % tile_q == 0;

            // Phase 2 layout: lanes along q, W outputs per lane.
            const int64_t lanes_q = tile_q / W;
            const int64_t rows2 = block_threads / lanes_q;
            const int64_t passes2 = tile_p / rows2;
            auto phase2_coords = [&](const std::string& ind) {
                return ind + "const int ql = (tid % " + std::to_string(lanes_q) + ") * " + std::to_string(W) + ";\n" +
                       ind + "const int pl = tid / " + std::to_string(lanes_q) + " + it * " + std::to_string(rows2) +
                       ";\n" + ind + "const idx_t " + ps + " = pbase + pl;\n" + ind + "const idx_t " + qs +
                       " = qbase + ql;\n";
            };
            // ---- phase 1: lanes along p, V elements per lane ----
            const int64_t lanes_p = tile_p / V;
            const int64_t rows1 = block_threads / lanes_p;
            const int64_t passes1 = tile_q / rows1;
            auto phase1_body = [&](const std::vector<int>& modes) {
                std::string code;
                code += "        #pragma unroll\n";
                code += "        for (int it = 0; it < " + std::to_string(passes1) + "; ++it) {\n";
                code += "            const int pl = (tid % " + std::to_string(lanes_p) + ") * " +
                        std::to_string(V) + ";\n";
                code += "            const int ql = tid / " + std::to_string(lanes_p) + " + it * " +
                        std::to_string(rows1) + ";\n";
                code += "            const idx_t " + ps + " = pbase + pl;\n";
                code += "            const idx_t " + qs + " = qbase + ql;\n";
                std::string guard;
                if (!full_p) guard += ps + " < " + std::to_string(extent_p);
                if (!full_q) guard += std::string(guard.empty() ? "" : " && ") + qs + " < " +
                                      std::to_string(extent_q);
                std::string indent = "            ";
                if (!guard.empty()) {
                    code += indent + "if (" + guard + ") {\n";
                    indent += "    ";
                }
                std::string body;
                emitter em(k, body, static_cast<int>(V));
                em.indent = indent;
                em.declare_roots(tiled_roots);
                em.condition = cond_fn;
                em.row_value = [](int) -> std::string {
                    throw std::logic_error("row value in a pointwise kernel");
                };
                em.forced_branch = [&](int id) {
                    for (size_t h = 0; h < hoisted.size(); ++h) {
                        if (hoisted[h] == id) return modes[h] == 1 ? 0 : (modes[h] == 2 ? 1 : -1);
                    }
                    return -1;
                };
                em.load = [&](int id) {
                    const knode& n = k.at(id);
                    const std::string base = "a" + std::to_string(n.slot);
                    const std::string idx = index_text(n.index, names);
                    std::vector<std::string> lanes(static_cast<size_t>(V));
                    const int64_t step = n.index.is_affine ? n.index.w[p] : 0;
                    if (V > 1 && step == 0) {
                        const std::string u = em.fresh("u");
                        em.line("const float " + u + " = " + base + "[" + idx + "];");
                        for (auto& lane : lanes) lane = u;
                        return lanes;
                    }
                    const vector_load vl = plan_vector_load(n, p, V, r.slot_elems);
                    if (vl.ok) {
                        const std::string w = em.fresh("w");
                        const std::string type = vl.width == 4 ? "float4" : "float2";
                        const std::string addr = base + " + " + idx + " - " + std::to_string(vl.m);
                        if (vl.width == 4 && streaming(n))
                            em.line("const porch_v4f " + w + " = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" +
                                    addr + "));");
                        else
                            em.line("const " + type + " " + w + " = *reinterpret_cast<const " + type +
                                    "*>(" + addr + ");");
                        for (int64_t e = 0; e < V; ++e) lanes[e] = w + lane_name(vl.m + vl.step * e);
                        return lanes;
                    }
                    if (V == 1) return std::vector<std::string>{base + "[" + idx + "]"};
                    const std::string ptr = em.fresh("p");
                    em.line("const float* " + ptr + " = " + base + " + " + idx + ";");
                    for (int64_t e = 0; e < V; ++e)
                        lanes[e] = ptr + "[" + std::to_string(step * e) + "]";
                    return lanes;
                };
                for (size_t i = 0; i < n_stage; ++i) {
                    std::string guard;
                    for (const auto& [c, branch] : t.guards[i]) {
                        if (!guard.empty()) guard += " && ";
                        guard += branch ? cond_fn(c) : "!(" + cond_fn(c) + ")";
                    }
                    if (!guard.empty()) em.open_scope(guard);
                    const std::vector<std::string> v = em.emit(t.staged[i]);
                    for (int64_t e = 0; e < V; ++e)
                        em.line("stage[" + std::to_string(i) + "][pl + " + std::to_string(e) +
                                "][ql] = " + v[e] + ";");
                    if (!guard.empty()) em.close_scope();
                }
                code += body;
                if (!guard.empty()) code += "            }\n";
                code += "        }\n";
                return code;
            };
            // One version of phase 1 per combination of hoisted-select modes.
            std::vector<std::vector<int>> combos{{}};
            for (size_t h = 0; h < hoisted.size(); ++h) {
                std::vector<std::vector<int>> next;
                for (const auto& c : combos)
                    for (const int m : {1, 2, 0}) {
                        auto d = c;
                        d.push_back(m);
                        next.push_back(d);
                    }
                combos = next;
            }
            for (size_t c = 0; c < combos.size(); ++c) {
                std::string test;
                for (size_t h = 0; h < hoisted.size(); ++h) {
                    if (!test.empty()) test += " && ";
                    test += "mode" + std::to_string(h) + " == " + std::to_string(combos[c][h]);
                }
                if (combos.size() == 1) s += "    {\n";
                else if (c == 0) s += "    if (" + test + ") {\n";
                else if (c + 1 == combos.size()) s += "    } else {\n";
                else s += "    } else if (" + test + ") {\n";
                s += phase1_body(combos[c]);
            }
            s += "    }\n";
            s += "    __syncthreads();\n";

            // ---- phase 2: lanes along q, W outputs per lane ----
            s += "    #pragma unroll\n";
            s += "    for (int it = 0; it < " + std::to_string(passes2) + "; ++it) {\n";
            s += phase2_coords("        ");
            std::string guard;
            if (!full_p) guard += ps + " < " + std::to_string(extent_p);
            if (!full_q) guard += std::string(guard.empty() ? "" : " && ") + qs + " < " +
                                  std::to_string(extent_q);
            std::string indent = "        ";
            if (!guard.empty()) {
                s += indent + "if (" + guard + ") {\n";
                indent += "    ";
            }
            {
                std::string body;
                emitter em(k, body, static_cast<int>(W));
                em.indent = indent;
                em.declare_roots(tiled_roots);
                em.condition = cond_fn;
                em.row_value = [](int) -> std::string {
                    throw std::logic_error("row value in a pointwise kernel");
                };
                em.override_node = [&](int id) -> std::vector<std::string> {
                    for (size_t i = 0; i < n_stage; ++i) {
                        if (t.staged[i] != id) continue;
                        std::vector<std::string> out;
                        for (int64_t e = 0; e < W; ++e)
                            out.push_back("stage[" + std::to_string(i) + "][pl][ql + " +
                                          std::to_string(e) + "]");
                        return out;
                    }
                    return {};
                };
                em.load = [&](int id) {
                    const knode& n = k.at(id);
                    const std::string base = "a" + std::to_string(n.slot);
                    const std::string idx = index_text(n.index, names);
                    if (W == 1) return std::vector<std::string>{base + "[" + idx + "]"};
                    std::vector<std::string> lanes(static_cast<size_t>(W));
                    const int64_t step = n.index.w[q];
                    if (step == 0) {
                        const std::string u = em.fresh("u");
                        em.line("const float " + u + " = " + base + "[" + idx + "];");
                        for (auto& lane : lanes) lane = u;
                        return lanes;
                    }
                    const vector_load vl = plan_vector_load(n, q, W, r.slot_elems);
                    if (vl.ok && vl.width == 4 && vl.m == 0 && vl.step == 1) {
                        const std::string w = em.fresh("w");
                        if (streaming(n))
                            em.line("const porch_v4f " + w + " = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" +
                                    base + " + " + idx + "));");
                        else
                            em.line("const float4 " + w + " = *reinterpret_cast<const float4*>(" +
                                    base + " + " + idx + ");");
                        return std::vector<std::string>{w + ".x", w + ".y", w + ".z", w + ".w"};
                    }
                    const std::string ptr = em.fresh("p");
                    em.line("const float* " + ptr + " = " + base + " + " + idx + ";");
                    for (int64_t e = 0; e < W; ++e)
                        lanes[e] = ptr + "[" + std::to_string(step * e) + "]";
                    return lanes;
                };
                const std::vector<std::string> v = em.emit(r.root);
                s += body;
                if (W == 4)
                    s += indent + "*reinterpret_cast<float4*>(out + " + output_index(r.shape) +
                         ") = make_float4(" + v[0] + ", " + v[1] + ", " + v[2] + ", " + v[3] + ");\n";
                else
                    s += indent + "out[" + output_index(r.shape) + "] = " + v[0] + ";\n";
            }
            if (!guard.empty()) s += "        }\n";
            s += "    }\n";
            // The next tile's phase 1 overwrites the stage phase 2 just read.
            if (persistent) s += "    __syncthreads();\n";
            s += "    }\n}\n";
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
