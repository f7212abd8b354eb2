// Row programs.  The reference materialises every nested reduction as its
// own kernel (reference src/tensor.cpp:970-989) and reduces each output with
// a 256-thread block and a shared-memory tree (896-962): softmax becomes
// four launches and about four reads of the input.  A row program runs the
// whole row-space graph in one kernel: one wave64 per row (a workgroup per
// long row, a segment of a wave per short row), the row's leaves read once into
// registers, each reduction folded in registers and finished with a wave
// butterfly (plus LDS across waves in workgroup mode), and the outputs - or
// the row's final reduction - written in the same pass.

#include "codegen.hpp"
#include "emit_expr.hpp"

#include <algorithm>
#include <functional>
#include <memory>
#include <set>
#include <stdexcept>

namespace porch::cg {
    namespace {

        std::vector<std::string> coordinate_names(size_t rank) {
            std::vector<std::string> names;
            for (size_t d = 0; d < rank; ++d) names.push_back("q" + std::to_string(d));
            return names;
        }

        bool depends_on_column(const kexpr& k, int root, size_t col) {
            for (const int id : k.postorder(root)) {
                const knode& n = k.at(id);
                if (n.op == kop::load) {
                    if (!n.index.is_affine) return true;
                    if (n.index.w[col] != 0) return true;
                }
                if (n.op == kop::select) {
                    if (!n.cond.lhs.is_affine || n.cond.lhs.w[col] != 0) return true;
                }
            }
            return false;
        }

        bool row_invariant(const ival& x, size_t rank) {
            if (!x.is_affine) return false;
            for (size_t d = 0; d + 1 < rank; ++d) {
                if (x.w[d] != 0) return false;
            }
            return true;
        }

        // Nodes under a select (either branch) from `root`.
        void mark_under_select(const kexpr& k, int root, std::vector<char>& under) {
            std::function<void(int, bool)> walk = [&](int id, bool inside) {
                if (id < 0) return;
                if (inside) {
                    if (under[id]) return;
                    under[id] = 1;
                }
                const knode& n = k.at(id);
                const bool child_inside = inside || n.op == kop::select;
                walk(n.a, child_inside);
                walk(n.b, child_inside);
            };
            walk(root, false);
        }

    } // namespace

    kernel_code emit_row(const row_request& r) {
        const kexpr& k = *r.expr;
        const size_t rank = r.shape.size();
        const size_t col = rank - 1;
        const int64_t length = r.shape[col];
        std::vector<int64_t> row_shape(r.shape.begin(), r.shape.end() - 1);
        const int64_t rows = ir::numel(row_shape);
        // Rows of 2048 or more are spread over a whole workgroup (at least
        // 8 values per lane): a quarter of the registers per lane of the
        // wave-per-row form, so four times the resident rows to overlap
        // loads, arithmetic and stores.  A single fold of rows under 4096
        // (one value per row, nothing cached) stays with a wave per row: no
        // workgroup barrier per row (logistic row sum [16384, 2048]: 25.1 ->
        // 24.1 us, A/B in one process).
        const bool single_fold = r.reduce_output && r.reductions.empty();
        const bool block_mode = length >= 2048 && !(single_fold && length < 4096);

        // Pass roots: each reduction's producer, then the output.
        std::vector<int> pass_roots;
        for (const row_reduction& red : r.reductions) pass_roots.push_back(red.producer);
        pass_roots.push_back(r.output);
        const size_t n_pass = pass_roots.size();

        bool all_affine = true;
        bool uniform_selects = true;
        for (const int root : pass_roots) {
            for (const int id : k.postorder(root)) {
                const knode& n = k.at(id);
                if (n.op == kop::load && !n.index.is_affine) all_affine = false;
                if (n.op == kop::select &&
                    (!n.cond.lhs.is_affine || n.cond.lhs.w[col] != 0))
                    uniform_selects = false;
            }
        }
        const int width = (all_affine && uniform_selects && length % 4 == 0) ? 4 : 1;
        // Lanes per row: the workgroup, or the wave - or, for rows shorter
        // than a wave's 64 values (x width), the smallest power-of-two
        // segment of lanes that covers the row, with 64 / seg rows per wave
        // at once (softmax [262144, 32]: 8 rows per wave instead of 1, with
        // 3 butterfly steps per reduction instead of 6).
        int seg = 64;
        if (!block_mode) {
            seg = 1;
            while (seg < 64 && static_cast<int64_t>(seg) * width < length) seg *= 2;
        }
        // Waves per workgroup in workgroup mode: 4, or up to 16 for rows
        // beyond 16384 so that a lane holds at most 64 of the row's values
        // and the row fits the register cache (read once).  Softmax
        // [1024, 65536] otherwise reads every row three times.
        int block_waves = 4;
        if (block_mode) {
            while (block_waves < 16 && length > static_cast<int64_t>(block_waves) * 64 * 64) block_waves *= 2;
        }
        const int lanes = block_mode ? 64 * block_waves : seg;
        const int rows_per_seg_wave = block_mode ? 1 : 64 / seg; // rows a wave holds at once
        const int64_t per_chunk = static_cast<int64_t>(lanes) * width;
        const int64_t chunks = (length + per_chunk - 1) / per_chunk;
        const bool ragged = length % per_chunk != 0;

        // Nodes under a select are never cached (their values exist only on
        // the taken branch).
        std::vector<char> under(k.nodes.size(), 0);
        for (size_t p = 0; p < n_pass; ++p) mark_under_select(k, pass_roots[p], under);

        // Row-invariant, column-varying loads are hoisted out of the row loop.
        std::vector<int> hoisted;
        const int64_t per_value = chunks * width;
        // Cached floats per lane: 128, or 64 with 16-wave workgroups (four
        // waves per SIMD leave 128 VGPRs in all; softmax [1024, 131072]
        // cached 128 and spilled 49 of them to scratch).
        const int64_t budget = block_waves == 16 ? 64 : 128;
        if (rows > 1) {
            std::set<int> seen;
            for (const int root : pass_roots) {
                for (const int id : k.postorder(root)) {
                    const knode& n = k.at(id);
                    if (n.op != kop::load || under[id] || seen.count(id)) continue;
                    if (row_invariant(n.index, rank) && depends_on_column(k, id, col)) {
                        hoisted.push_back(id);
                        seen.insert(id);
                    }
                }
            }
            if (static_cast<int64_t>(hoisted.size()) * per_value > budget / 2) hoisted.clear();
        }
        auto is_hoisted = [&](int id) {
            return std::find(hoisted.begin(), hoisted.end(), id) != hoisted.end();
        };

        // Register caches across passes.  Pass p walks its root; a
        // column-varying node already computed by an earlier pass is read
        // from its cache (and not descended into), so a value and its
        // operands are never both kept.  `allow` limits what may be cached.
        std::vector<int> cached;
        std::vector<size_t> first_pass(k.nodes.size(), 0);
        std::vector<size_t> last_pass(k.nodes.size(), 0);
        auto plan_caches = [&](bool loads_only) {
            cached.clear();
            std::vector<int> computed(k.nodes.size(), -1);
            std::vector<char> is_cached(k.nodes.size(), 0);
            for (size_t p = 0; p < n_pass; ++p) {
                std::vector<char> visited(k.nodes.size(), 0);
                std::function<void(int)> walk = [&](int id) {
                    if (id < 0 || visited[id]) return;
                    visited[id] = 1;
                    const knode& n = k.at(id);
                    const bool cacheable =
                        !under[id] && !is_hoisted(id) && n.op != kop::constant &&
                        n.op != kop::row_value && depends_on_column(k, id, col) &&
                        (!loads_only || n.op == kop::load);
                    if (cacheable && computed[id] >= 0 && static_cast<size_t>(computed[id]) < p) {
                        if (!is_cached[id]) {
                            is_cached[id] = 1;
                            cached.push_back(id);
                            first_pass[id] = static_cast<size_t>(computed[id]);
                        }
                        last_pass[id] = p;
                        return;
                    }
                    if (computed[id] < 0) computed[id] = static_cast<int>(p);
                    walk(n.a);
                    walk(n.b);
                };
                walk(pass_roots[p]);
            }
            // Peak number of cached values alive across a pass boundary.
            int64_t peak = 0;
            for (size_t b = 0; b + 1 < n_pass; ++b) {
                int64_t live = 0;
                for (const int id : cached)
                    if (first_pass[id] <= b && last_pass[id] > b) ++live;
                peak = std::max(peak, live);
            }
            return (peak + static_cast<int64_t>(hoisted.size())) * per_value <= budget;
        };
        if (!plan_caches(false) && !plan_caches(true)) cached.clear();

        const int64_t rows_per_group = block_mode ? 1 : 4 * rows_per_seg_wave;
        int64_t rows_per_wave = 1;
        if (!hoisted.empty()) {
            // Enough workgroups to fill the machine several times over; each
            // loads the hoisted values once.
            const int64_t target =
                static_cast<int64_t>(r.compute_units) * (block_mode ? 16 : 8) * rows_per_group;
            rows_per_wave = std::max<int64_t>(1, rows / std::max<int64_t>(target, 1));
        }
        const int64_t groups =
            std::max<int64_t>(1, (rows + rows_per_group * rows_per_wave - 1) /
                                     (rows_per_group * rows_per_wave));

        kernel_code kc;
        kc.kind = "row";
        kc.name = "porch_row";
        kc.n_slots = r.n_slots;
        kc.block = block_mode ? static_cast<unsigned>(lanes) : 256;
        kc.grid_x = static_cast<unsigned>(std::min<int64_t>(groups, int64_t{1} << 22));
        const char* T = r.width.type();
        const std::vector<std::string> names = coordinate_names(rank);
        const std::string qc = "q" + std::to_string(col);

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(" + std::to_string(kc.block) + ") porch_row(" +
             kernel_params(r.n_slots) + ") {\n";
        s += "    const int lane = threadIdx.x & 63;\n";
        s += "    const int wave = threadIdx.x >> 6;\n";
        const size_t n_reductions = r.reductions.size() + (r.reduce_output ? 1 : 0);
        if (block_mode) {
            // One slot per reduction per wave, in two sets alternating by row
            // iteration: a slot is rewritten two rows later, and every row
            // passes at least one barrier in between, so one barrier per
            // reduction suffices.
            s += "    __shared__ float red[2][" + std::to_string(std::max<size_t>(n_reductions, 1)) +
                 "][" + std::to_string(block_waves) + "];\n";
            s += "    const int tl = threadIdx.x;\n";
            s += "    int it = 0;\n";
            bool any_max = r.reduce_output && r.output_is_max;
            for (const row_reduction& red : r.reductions) any_max = any_max || red.is_max;
            // Virtual-lane partials of a max taken in the reference's order.
            if (any_max) s += "    __shared__ float ex[257];\n";
        }
        else if (seg == 64) {
            s += "    const int tl = lane;\n";
        }
        else {
            s += "    const int tl = lane & " + std::to_string(seg - 1) + ";\n";
            s += "    const int sub = lane / " + std::to_string(seg) + ";\n";
        }
        // With several rows per wave the last iteration may hold fewer rows
        // than segments: `live` guards every access of a segment without one
        // (the loop itself stays uniform across the wave).
        const bool segmented = !block_mode && seg < 64;
        const std::string W = std::to_string(width);
        const std::string NC = std::to_string(chunks);
        for (const int id : cached) {
            s += "    float c" + std::to_string(id) + "[" + NC + "][" + W + "];\n";
        }

        // Chunk loops unroll fully when values live in per-chunk register
        // arrays (cached or hoisted); otherwise by 8: a fully unrolled loop
        // over many chunks issues all its loads at once and spills (softmax
        // [512, 262144], 64 chunks: 68 VGPRs spilled).
        const bool partial_unroll = cached.empty() && hoisted.empty() && chunks > 16;
        // Rows read from memory once per pass walk their chunks in
        // alternate directions, so each pass starts on the chunks the
        // previous one read last, which are the likeliest still cached.
        int memory_passes = 0;
        auto chunk_open = [&](std::string& code, const std::string& indent, bool row_pass = false) {
            const bool reverse = row_pass && partial_unroll && memory_passes++ % 2 == 1;
            code += indent + (partial_unroll ? "#pragma unroll 8\n" : "#pragma unroll\n");
            if (reverse)
                code += indent + "for (int j = " + std::to_string(chunks - 1) + "; j >= 0; --j) {\n";
            else
                code += indent + "for (int j = 0; j < " + NC + "; ++j) {\n";
            code += indent + "    const " + T + " " + qc + " = (" + T + ")(j * " +
                    std::to_string(lanes) + " + tl) * " + W + ";\n";
            if (ragged && segmented)
                code += indent + "    if (live && " + qc + " < " + std::to_string(length) + ") {\n";
            else if (ragged)
                code += indent + "    if (" + qc + " < " + std::to_string(length) + ") {\n";
            else if (segmented)
                code += indent + "    if (live) {\n";
        };
        const bool guarded = ragged || segmented;
        auto chunk_close = [&](std::string& code, const std::string& indent) {
            if (guarded) code += indent + "    }\n";
            code += indent + "}\n";
        };

        // A leaf whose every element is read exactly once by this kernel
        // (no broadcast dimension, and held in registers or read by one
        // pass only) streams past the caches: non-temporal loads keep it
        // from evicting data that is reused.  A leaf that several passes
        // read again (a row too long for the register cache) uses ordinary
        // loads, so the later passes can hit L2 and the Infinity Cache.
        std::vector<int> passes_reading(k.nodes.size(), 0);
        for (const row_reduction& red : r.reductions)
            for (const int id : k.postorder(red.producer)) ++passes_reading[id];
        if (r.output >= 0)
            for (const int id : k.postorder(r.output)) ++passes_reading[id];
        auto streaming = [&](int id) {
            const knode& n = k.at(id);
            if (!n.index.is_affine) return false;
            for (size_t d = 0; d < rank; ++d) {
                if (r.shape[d] > 1 && n.index.w[d] == 0) return false;
            }
            return passes_reading[id] <= 1 || std::find(cached.begin(), cached.end(), id) != cached.end();
        };
        // Outputs use ordinary stores: with non-temporal loads already
        // keeping the inputs out of the way, non-temporal stores measured
        // 3-5% slower on softmax [8192, 4096] (A/B in one process).

        auto load_text = [&](emitter& em, int id) {
            const knode& n = k.at(id);
            const std::string base = "a" + std::to_string(n.slot);
            std::vector<std::string> out(static_cast<size_t>(width));
            if (width == 1) {
                out[0] = base + "[" + index_text(n.index, names) + "]";
                return out;
            }
            const int64_t step = n.index.w[col];
            const std::string idx = index_text(n.index, names);
            if (step == 0) {
                const std::string v = em.fresh("u");
                em.line("const float " + v + " = " + base + "[" + idx + "];");
                for (auto& lane_value : out) lane_value = v;
                return out;
            }
            bool aligned = step == 1 && n.index.c0 % 4 == 0;
            for (size_t d = 0; d + 1 < rank && aligned; ++d) {
                if (n.index.w[d] % 4 != 0) aligned = false;
            }
            if (aligned) {
                const std::string v = em.fresh("w");
                if (streaming(id)) {
                    em.line("const porch_v4f " + v + " = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" +
                            base + " + " + idx + "));");
                }
                else {
                    em.line("const float4 " + v + " = *reinterpret_cast<const float4*>(" + base +
                            " + " + idx + ");");
                }
                return std::vector<std::string>{v + ".x", v + ".y", v + ".z", v + ".w"};
            }
            const std::string p = em.fresh("p");
            em.line("const float* " + p + " = " + base + " + " + idx + ";");
            for (int e = 0; e < width; ++e) out[e] = p + "[" + std::to_string(step * e) + "]";
            return out;
        };

        // Hoisted row-invariant loads.
        for (const int id : hoisted) {
            s += "    float h" + std::to_string(id) + "[" + NC + "][" + W + "];\n";
        }
        if (!hoisted.empty()) {
            std::string code;
            if (segmented) code += "    const bool live = true;\n";
            chunk_open(code, "    ");
            std::string body;
            emitter em(k, body, width);
            em.indent = "        ";
            for (const int id : hoisted) {
                const std::vector<std::string> v = load_text(em, id);
                for (int e = 0; e < width; ++e)
                    em.line("h" + std::to_string(id) + "[j][" + std::to_string(e) +
                            "] = " + v[e] + ";");
            }
            code += body;
            chunk_close(code, "    ");
            s += code;
        }

        const std::string row_step = std::to_string(rows_per_group);
        if (block_mode) {
            s += "    for (idx_t row = blockIdx.x; row < " + std::to_string(rows) +
                 "; row += gridDim.x) {\n";
        }
        else if (!segmented) {
            s += "    for (idx_t row = (idx_t)blockIdx.x * 4 + wave; row < " +
                 std::to_string(rows) + "; row += (idx_t)gridDim.x * 4) {\n";
        }
        else {
            const std::string G = std::to_string(rows_per_seg_wave);
            s += "    for (idx_t first = ((idx_t)blockIdx.x * 4 + wave) * " + G + "; first < " +
                 std::to_string(rows) + "; first += (idx_t)gridDim.x * " + std::to_string(4 * rows_per_seg_wave) +
                 ") {\n";
            s += "        const idx_t row = first + sub;\n";
            s += "        const bool live = row < " + std::to_string(rows) + ";\n";
        }
        {
            std::vector<bool> needed(row_shape.size(), true);
            s += decompose("row", row_shape, needed, T, "        ");
        }

        size_t next_slot = 0;
        // Lane reduction, lowest distance first: within a row of 16 lanes
        // by DPP (quad permutations for distances 1 and 2, then the half-row
        // and row mirrors, which pair lanes across groups that already hold
        // one value each), across rows by ds_bpermute (__shfl_xor).  Both
        // combines are commutative (a + b == b + a; porch_fmax orders -0
        // below +0 and returns NaN for any NaN), so every lane of a row ends
        // with the same value, up to the payload of a NaN.
        auto reduce_lanes = [&](const std::string& acc, bool is_max) {
            std::string code;
            auto combine = [&](const std::string& partner) {
                return is_max ? "porch_fmax(" + acc + ", " + partner + ")" : acc + " + " + partner;
            };
            const int span = std::min(lanes, 64);
            const char* dpp[] = {"0xB1", "0x4E", "0x141", "0x140"}; // distances 1, 2, 4, 8
            for (int m = 1, i = 0; m < span; m *= 2, ++i) {
                const std::string partner =
                    m <= 8 ? "__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, " + acc +
                                 "), " + dpp[i] + ", 0xF, 0xF, false))"
                           : "__shfl_xor(" + acc + ", " + std::to_string(m) + ", 64)";
                code += "        " + acc + " = " + combine(partner) + ";\n";
            }
            if (block_mode) {
                const std::string slot = "red[it & 1][" + std::to_string(next_slot++) + "]";
                code += "        if (lane == 0) " + slot + "[wave] = " + acc + ";\n";
                code += "        __syncthreads();\n";
                // Pairwise over the wave partials, in a fixed order.
                std::vector<std::string> terms;
                for (int w = 0; w < block_waves; ++w) terms.push_back(slot + "[" + std::to_string(w) + "]");
                while (terms.size() > 1) {
                    std::vector<std::string> next;
                    for (size_t t = 0; t + 1 < terms.size(); t += 2)
                        next.push_back(is_max ? "porch_fmax(" + terms[t] + ", " + terms[t + 1] + ")"
                                              : "(" + terms[t] + " + " + terms[t + 1] + ")");
                    terms = next;
                }
                code += "        " + acc + " = " + terms[0] + ";\n";
            }
            return code;
        };

        std::vector<int> row_roots;
        for (const row_reduction& red : r.reductions) row_roots.push_back(red.producer);
        if (r.output >= 0) row_roots.push_back(r.output);

        // Nodes that reach the result only through its final sum: every
        // user is itself such a node, and no other pass (reduction) reads
        // them.  Operands precede users in the arena, so one backward sweep.
        std::vector<char> relaxed(k.nodes.size(), 0);
        if (r.reduce_output && !r.output_is_max && r.output >= 0) {
            std::vector<char> other(k.nodes.size(), 0);
            for (const row_reduction& red : r.reductions)
                for (const int id : k.postorder(red.producer)) other[id] = 1;
            std::vector<char> in_output(k.nodes.size(), 0);
            for (const int id : k.postorder(r.output)) in_output[id] = 1;
            for (size_t i = k.nodes.size(); i-- > 0;) {
                if (!in_output[i] || other[i]) continue;
                if (static_cast<int>(i) == r.output) {
                    relaxed[i] = 1;
                    continue;
                }
                bool all = true;
                int users = 0;
                for (size_t u = i + 1; u < k.nodes.size(); ++u) {
                    const knode& n = k.nodes[u];
                    if (n.a != static_cast<int>(i) && n.b != static_cast<int>(i)) continue;
                    ++users;
                    if (!relaxed[u]) all = false;
                }
                relaxed[i] = (all && users > 0) ? 1 : 0;
            }
        }

        auto make_emitter = [&](std::string& body, size_t pass) {
            auto em = std::make_unique<emitter>(k, body, width);
            em->indent = guarded ? "                " : "            ";
            em->declare_roots(row_roots);
            em->relaxed = [&](int id) { return relaxed[static_cast<size_t>(id)] != 0; };
            emitter* self = em.get();
            em->load = [&, self](int id) {
                for (const int h : hoisted) {
                    if (h == id) {
                        std::vector<std::string> out;
                        for (int e = 0; e < width; ++e)
                            out.push_back("h" + std::to_string(id) + "[j][" + std::to_string(e) + "]");
                        return out;
                    }
                }
                return load_text(*self, id);
            };
            em->override_node = [&, pass](int id) -> std::vector<std::string> {
                for (const int c : cached) {
                    if (c == id && first_pass[id] < pass) {
                        std::vector<std::string> out;
                        for (int e = 0; e < width; ++e)
                            out.push_back("c" + std::to_string(id) + "[j][" + std::to_string(e) + "]");
                        return out;
                    }
                }
                return {};
            };
            em->row_value = [](int row) { return "rv" + std::to_string(row); };
            em->condition = [&](const kcond& c) {
                return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
            };
            return em;
        };

        // A max whose order-free result may differ from the reference's
        // (porch_max_order_matters: a NaN in the row, or a +0 maximum) is
        // recomputed in the reference's block order (src/tensor.cpp:896-962):
        // 256 virtual lanes, virtual lane t folding columns t, t + 256, ...
        // with t = t > v ? t : v from -FLT_MAX, then the tree with strides
        // 128, 64, ..., 1.  Lane tl of a row's `seg` lanes takes virtual
        // lanes tl, tl + seg, ...: the tree's strides of seg and more combine
        // within the lane, the smaller ones across lanes.  A workgroup row
        // stages its 256 virtual partials in LDS and finishes in wave 0.  The
        // branch is uniform over the row's lanes, and the result is the
        // row leader's, so every lane holds the same bits.
        auto leaf_fold = [&](const std::string& first, int root, const std::string& f,
                             const std::string& indent, bool guard_live) {
            std::string code = indent + "float " + f + " = -PORCH_FLT_MAX;\n";
            if (guard_live) code += indent + "if (live)\n";
            code += indent + "for (" + T + " " + qc + " = " + first + "; " + qc + " < " + std::to_string(length) +
                    "; " + qc + " += 256) {\n";
            std::string body;
            emitter em(k, body, 1);
            em.indent = indent + "    ";
            em.declare_roots(row_roots);
            em.relaxed = [&](int id) { return relaxed[static_cast<size_t>(id)] != 0; };
            em.load = [&](int id) {
                const knode& n = k.at(id);
                return std::vector<std::string>{"a" + std::to_string(n.slot) + "[" + index_text(n.index, names) + "]"};
            };
            em.row_value = [](int row) { return "rv" + std::to_string(row); };
            em.condition = [&](const kcond& c) {
                return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
            };
            const std::vector<std::string> v = em.emit(root);
            em.line(f + " = porch_refmax(" + f + ", " + v[0] + ");");
            code += body + indent + "}\n";
            return code;
        };
        // The reference's tree over virtual lanes lo, lo + step, ... (n of
        // them, n a power of two) held in `leaf`: strides n/2, ..., 1 in
        // units of `step`.  Leaves named "" are empty virtual lanes
        // (-FLT_MAX); a pair of them folds away at generation time.
        int tree_counter = 0;
        auto lane_tree = [&](std::vector<std::string> leaf, const std::string& indent, std::string& code) {
            for (size_t h = leaf.size() / 2; h >= 1; h /= 2) {
                for (size_t i = 0; i < h; ++i) {
                    if (leaf[i].empty() && leaf[i + h].empty()) continue;
                    const std::string a = leaf[i].empty() ? "-PORCH_FLT_MAX" : leaf[i];
                    const std::string b = leaf[i + h].empty() ? "-PORCH_FLT_MAX" : leaf[i + h];
                    const std::string t = "xt" + std::to_string(tree_counter++);
                    code += indent + "const float " + t + " = porch_refmax(" + a + ", " + b + ");\n";
                    leaf[i] = t;
                }
            }
            return leaf[0].empty() ? std::string("-PORCH_FLT_MAX") : leaf[0];
        };
        auto exact_max = [&](int root, const std::string& acc) {
            // Rows sharing a wave take the path together when any of them
            // needs it (its cross-lane steps then run with the whole wave
            // active), and keep the result only where they do.
            std::string code = segmented
                ? "        if (__ballot(porch_max_order_matters(" + acc + ")) != 0) {\n"
                  "            const bool xflag = porch_max_order_matters(" + acc + ");\n"
                : "        if (porch_max_order_matters(" + acc + ")) {\n";
            const std::string in = "            ";
            if (block_mode) {
                code += in + "if (threadIdx.x < 256) {\n";
                code += leaf_fold("(" + std::string(T) + ")threadIdx.x", root, "xf", in + "    ", false);
                code += in + "    ex[threadIdx.x] = xf;\n" + in + "}\n";
                code += in + "__syncthreads();\n";
                code += in + "if (wave == 0) {\n";
                std::vector<std::string> leaf;
                for (int r = 0; r < 4; ++r) {
                    leaf.push_back("xl" + std::to_string(r));
                    code += in + "    const float xl" + std::to_string(r) + " = ex[lane + " + std::to_string(64 * r) + "];\n";
                }
                code += in + "    float xh = " + lane_tree(leaf, in + "    ", code) + ";\n";
                for (int m = 32; m >= 1; m /= 2)
                    code += in + "    xh = porch_refmax(xh, __shfl_xor(xh, " + std::to_string(m) + ", 64));\n";
                code += in + "    if (lane == 0) ex[256] = xh;\n" + in + "}\n";
                code += in + "__syncthreads();\n";
                code += in + acc + " = ex[256];\n";
            }
            else {
                // Virtual lane tl + seg * r holds columns only while
                // seg * r < length.
                const int per_lane = 256 / seg;
                std::vector<std::string> leaf(static_cast<size_t>(per_lane));
                for (int r = 0; r < per_lane; ++r) {
                    if (static_cast<int64_t>(seg) * r >= length) break;
                    const std::string f = "xf" + std::to_string(r);
                    code += leaf_fold("tl + " + std::to_string(seg * r), root, f, in, segmented);
                    leaf[static_cast<size_t>(r)] = f;
                }
                code += in + "float xh = " + lane_tree(leaf, in, code) + ";\n";
                for (int m = seg / 2; m >= 1; m /= 2)
                    code += in + "xh = porch_refmax(xh, __shfl_xor(xh, " + std::to_string(m) + ", 64));\n";
                const std::string result = "__shfl(xh, " + (seg == 64 ? std::string("0") : "lane & " + std::to_string(64 - seg)) + ", 64)";
                if (segmented) {
                    code += in + "const float xr = " + result + ";\n";
                    code += in + "if (xflag) " + acc + " = xr;\n";
                }
                else {
                    code += in + acc + " = " + result + ";\n";
                }
            }
            code += "        }\n";
            return code;
        };

        auto store_caches = [&](emitter& em, size_t pass, int root) {
            for (const int c : cached) {
                if (first_pass[c] != pass) continue;
                bool reached = false;
                for (const int id : k.postorder(root)) reached = reached || id == c;
                if (!reached) continue;
                const std::vector<std::string> v = em.emit(c);
                for (int e = 0; e < width; ++e)
                    em.line("c" + std::to_string(c) + "[j][" + std::to_string(e) + "] = " + v[e] + ";");
            }
        };

        auto fold_pass = [&](size_t pass, int root, bool is_max, const std::string& acc) {
            std::string code;
            code += "        float " + acc + " = " + (is_max ? "-PORCH_FLT_MAX" : "0.0f") + ";\n";
            chunk_open(code, "        ", true);
            std::string body;
            auto em = make_emitter(body, pass);
            // A relaxed sum of reciprocals 1/d with d proven in [2^-31, 2^31]
            // (the logistic's 1 + exp(-v) lies in [1, 2]): four terms as
            // ((d0 + d1) d2 d3 + (d2 + d3) d0 d1) / (d0 d1 d2 d3), one
            // reciprocal instead of four; every product stays normal and
            // finite, and each group is within a few ulp of the four terms.
            const knode& rn = k.at(root);
            const bool paired = !is_max && width == 4 && relaxed[static_cast<size_t>(root)] &&
                                rn.op == kop::reciprocal &&
                                std::find(cached.begin(), cached.end(), root) == cached.end() &&
                                em->range_of(rn.a).within(0x1p-31F, 0x1p31F);
            if (paired) {
                const std::vector<std::string> d = em->emit(rn.a);
                store_caches(*em, pass, root);
                const std::string p0 = em->fresh("xp"), p1 = em->fresh("xp");
                const std::string s0 = em->fresh("xs"), s1 = em->fresh("xs");
                em->line("const float " + p0 + " = " + d[0] + " * " + d[1] + ";");
                em->line("const float " + p1 + " = " + d[2] + " * " + d[3] + ";");
                em->line("const float " + s0 + " = " + d[0] + " + " + d[1] + ";");
                em->line("const float " + s1 + " = " + d[2] + " + " + d[3] + ";");
                em->line(acc + " = __builtin_fmaf(__builtin_fmaf(" + s0 + ", " + p1 + ", " + s1 + " * " + p0 +
                         "), __builtin_amdgcn_rcpf(" + p0 + " * " + p1 + "), " + acc + ");");
            }
            else {
                const std::vector<std::string> v = em->emit(root);
                store_caches(*em, pass, root);
                for (int e = 0; e < width; ++e) {
                    if (is_max) em->line(acc + " = porch_fmax(" + acc + ", " + v[e] + ");");
                    else em->line(acc + " += " + v[e] + ";");
                }
            }
            code += body;
            chunk_close(code, "        ");
            code += reduce_lanes(acc, is_max);
            if (is_max) code += exact_max(root, acc);
            return code;
        };

        // A row too long for the register cache reads its leaves once per
        // pass.  A max of f followed by a sum of exp(f - that max) (softmax)
        // then runs as one pass.  Each lane keeps the exact running max and
        // a sum of exp(f - a) against an anchor a of its own, moved (and
        // the sum rescaled) only when a value exceeds it by more than 64,
        // so that no term overflows.  After the pass the max is reduced as
        // before, each lane rescales its sum once by exp(a - max), and the
        // sums are reduced as before: each term carries one extra rounding
        // of the reference's exp(f - max), not one per merge of partial
        // sums (a running-max form that rescaled at every merge measured
        // 1.05e-6 relative error at [40, 200004]).
        int online = -1;
        if (block_mode && cached.empty()) {
            for (size_t i = 0; i + 1 < r.reductions.size() && online < 0; ++i) {
                if (!r.reductions[i].is_max || r.reductions[i + 1].is_max) continue;
                const knode& g = k.at(r.reductions[i + 1].producer);
                if (g.op != kop::exp) continue;
                const knode& d = k.at(g.a);
                if (d.op != kop::subtract || d.a != r.reductions[i].producer) continue;
                const knode& rv = k.at(d.b);
                if (rv.op == kop::row_value && rv.row == static_cast<int>(i)) online = static_cast<int>(i);
            }
        }
        auto online_pass = [&](size_t pass, int root) {
            std::string code;
            code += "        float acc_m = -PORCH_FLT_MAX;\n        float acc_a = -PORCH_FLT_MAX;\n"
                    "        float acc_s = 0.0f;\n";
            chunk_open(code, "        ", true);
            std::string body;
            auto em = make_emitter(body, pass);
            const std::vector<std::string> v = em->emit(root);
            std::string cm = v[0];
            for (int e = 1; e < width; ++e) cm = "porch_fmax(" + cm + ", " + v[e] + ")";
            em->line("const float cm = " + cm + ";");
            em->line("acc_m = porch_fmax(acc_m, cm);");
            em->line("if (cm > acc_a + 64.0f) {");
            em->line("    acc_s = acc_s * porch_exp(acc_a - cm);");
            em->line("    acc_a = cm;");
            em->line("}");
            for (int e = 0; e < width; ++e) em->line("acc_s += porch_exp(" + v[e] + " - acc_a);");
            code += body;
            chunk_close(code, "        ");
            code += reduce_lanes("acc_m", true);
            code += exact_max(root, "acc_m");
            code += "        acc_s = acc_s * porch_exp(acc_a - acc_m);\n";
            code += reduce_lanes("acc_s", false);
            return code;
        };

        for (size_t i = 0; i < r.reductions.size(); ++i) {
            if (static_cast<int>(i) == online) {
                s += online_pass(i, r.reductions[i].producer);
                s += "        const float rv" + std::to_string(i) + " = acc_m;\n";
                s += "        const float rv" + std::to_string(i + 1) + " = acc_s;\n";
                ++i;
                continue;
            }
            const std::string acc = "acc" + std::to_string(i);
            s += fold_pass(i, r.reductions[i].producer, r.reductions[i].is_max, acc);
            s += "        const float rv" + std::to_string(i) + " = " + acc + ";\n";
        }
        const size_t out_pass = n_pass - 1;
        if (r.reduce_output) {
            s += fold_pass(out_pass, r.output, r.output_is_max, "acc_out");
            if (block_mode) s += "        if (threadIdx.x == 0) out[row] = acc_out;\n";
            else if (segmented) s += "        if (tl == 0 && live) out[row] = acc_out;\n";
            else s += "        if (lane == 0) out[row] = acc_out;\n";
        }
        else {
            std::string code;
            chunk_open(code, "        ", true);
            std::string body;
            auto em = make_emitter(body, out_pass);
            const std::vector<std::string> v = em->emit(r.output);
            const std::string base = "row * " + std::to_string(length) + " + " + qc;
            if (width == 4) {
                em->line("*reinterpret_cast<float4*>(out + " + base + ") = make_float4(" + v[0] +
                         ", " + v[1] + ", " + v[2] + ", " + v[3] + ");");
            }
            else {
                em->line("out[" + base + "] = " + v[0] + ";");
            }
            code += body;
            chunk_close(code, "        ");
            s += code;
        }
        if (block_mode) s += "        ++it;\n";
        s += "    }\n}\n";
        return kc;
    }

} // namespace porch::cg
