// A reduction over the last axis into few outputs (a full sum of a long
// vector, say), spread over the machine in two kernels instead of one
// workgroup per output.  The row program row_request describes (a single
// fold of an elementwise value over each row, no inner row reductions) is
// split into `parts` contiguous pieces per row:
//
//   row.partial   one 256-lane workgroup per (row, piece): each lane folds
//                 its strided values, then the wave butterfly and the four
//                 waves through LDS give the piece's partial, written to a
//                 temporary [rows, parts];
//   row.combine   one wave per row folds the row's partials.
//
// Sums are order-free within their tolerance.  A max is folded with
// porch_fmax (commutative, NaN-propagating, -0 below +0); where its result
// may differ from the reference's block order (NaN, or a +0 maximum) the
// combining wave recomputes it in that order over the whole row
// (src/tensor.cpp:896-962: 256 virtual lanes folding positions t, t + 256,
// ... with t = t > v ? t : v from -FLT_MAX, then the stride tree).

#include "codegen.hpp"
#include "emit_expr.hpp"

#include <algorithm>
#include <stdexcept>

namespace porch::cg {
    namespace {

        // Values a piece holds at least, and workgroups aimed at per
        // compute unit over all pieces.
        constexpr int64_t min_piece = 8192;
        constexpr int64_t groups_per_cu = 4;

        struct partial_shape {
            int64_t rows = 0;
            int64_t parts = 0;
            int64_t piece = 0; // values per piece, a multiple of 256 x width
            int width = 1;
        };

        bool column_uniform_selects_and_affine(const kexpr& k, int root, size_t col) {
            for (const int id : k.postorder(root)) {
                const knode& n = k.at(id);
                if (n.op == kop::load && !n.index.is_affine) return false;
                if (n.op == kop::select && (!n.cond.lhs.is_affine || n.cond.lhs.w[col] != 0)) return false;
            }
            return true;
        }

        partial_shape analyze(const row_request& r) {
            partial_shape sh;
            if (!r.reduce_output || !r.reductions.empty() || r.output < 0) return sh;
            const size_t col = r.shape.size() - 1;
            const int64_t length = r.shape[col];
            int64_t rows = 1;
            for (size_t d = 0; d < col; ++d) rows *= r.shape[d];
            const int64_t cus = std::max(r.compute_units, 8);
            // Only rows that one workgroup each would leave most of the
            // machine idle on, long enough to split.
            if (rows >= cus || length < 4 * min_piece) return sh;
            sh.width = column_uniform_selects_and_affine(*r.expr, r.output, col) && length % 4 == 0 ? 4 : 1;
            const int64_t quantum = 256 * static_cast<int64_t>(sh.width);
            int64_t parts = std::min((length + min_piece - 1) / min_piece, (groups_per_cu * cus + rows - 1) / rows);
            if (parts < 2) return sh;
            int64_t piece = (length + parts - 1) / parts;
            piece = (piece + quantum - 1) / quantum * quantum;
            parts = (length + piece - 1) / piece;
            if (parts < 2) return sh;
            sh.rows = rows;
            sh.parts = parts;
            sh.piece = piece;
            return sh;
        }

        // Values of the row program's output at column `qc` (width lanes),
        // the leaves read as emit_row reads them.
        std::vector<std::string> output_values(const row_request& r, std::string& body, int width,
                                               const std::vector<std::string>& names, const std::string& indent) {
            const kexpr& k = *r.expr;
            const size_t rank = r.shape.size();
            const size_t col = rank - 1;
            emitter em(k, body, width);
            em.indent = indent;
            em.declare_roots({r.output});
            em.load = [&](int id) {
                const knode& n = k.at(id);
                const std::string base = "a" + std::to_string(n.slot);
                std::vector<std::string> out(static_cast<size_t>(width));
                const std::string idx = index_text(n.index, names);
                if (width == 1) {
                    out[0] = base + "[" + idx + "]";
                    return out;
                }
                const int64_t step = n.index.w[col];
                if (step == 0) {
                    const std::string v = em.fresh("u");
                    em.line("const float " + v + " = " + base + "[" + idx + "];");
                    for (auto& lane_value : out) lane_value = v;
                    return out;
                }
                bool aligned = step == 1 && n.index.c0 % 4 == 0;
                for (size_t d = 0; d + 1 < rank && aligned; ++d)
                    if (n.index.w[d] % 4 != 0) aligned = false;
                if (aligned) {
                    const std::string v = em.fresh("w");
                    em.line("const porch_v4f " + v + " = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" +
                            base + " + " + idx + "));");
                    return std::vector<std::string>{v + ".x", v + ".y", v + ".z", v + ".w"};
                }
                const std::string p = em.fresh("p");
                em.line("const float* " + p + " = " + base + " + " + idx + ";");
                for (int e = 0; e < width; ++e) out[e] = p + "[" + std::to_string(step * e) + "]";
                return out;
            };
            em.row_value = [](int) -> std::string {
                throw std::logic_error("emit_row_partial: a row value in a single fold");
            };
            em.condition = [&](const kcond& c) {
                return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
            };
            return em.emit(r.output);
        }

        std::vector<std::string> coordinate_names(size_t rank) {
            std::vector<std::string> names;
            for (size_t d = 0; d < rank; ++d) names.push_back("q" + std::to_string(d));
            return names;
        }

        std::string wave_fold(bool is_max, const std::string& v) {
            std::string c;
            for (int d = 32; d >= 1; d /= 2) {
                const std::string other = "__shfl_xor(" + v + ", " + std::to_string(d) + ", 64)";
                c += "        " + v + " = " + (is_max ? "porch_fmax(" + v + ", " + other + ")" : v + " + " + other) + ";\n";
            }
            return c;
        }

    } // namespace

    int64_t row_partial_parts(const row_request& r) { return analyze(r).parts; }

    kernel_code emit_row_partial(const row_request& r) {
        const partial_shape sh = analyze(r);
        if (sh.parts < 2) throw std::logic_error("emit_row_partial: the reduction is not split");
        const size_t rank = r.shape.size();
        const size_t col = rank - 1;
        const int64_t length = r.shape[col];
        const std::vector<int64_t> row_shape(r.shape.begin(), r.shape.end() - 1);
        const char* T = r.width.type();
        const std::vector<std::string> names = coordinate_names(rank);
        const std::string qc = names[col];
        const bool is_max = r.output_is_max;
        const std::string W = std::to_string(sh.width);
        const std::string identity = is_max ? "-PORCH_FLT_MAX" : "0.0f";

        kernel_code kc;
        kc.kind = "row.partial";
        kc.name = "porch_row";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>(sh.rows * sh.parts);

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(256) porch_row(" + kernel_params(r.n_slots) + ") {\n";
        s += "    const int tl = threadIdx.x;\n    const int lane = tl & 63;\n    const int wave = tl >> 6;\n";
        s += "    __shared__ float xred[4];\n";
        s += "    const idx_t row = (idx_t)blockIdx.x / " + std::to_string(sh.parts) + ";\n";
        s += "    const idx_t part = (idx_t)blockIdx.x % " + std::to_string(sh.parts) + ";\n";
        std::vector<bool> needed(row_shape.size(), true);
        s += decompose("row", row_shape, needed, T, "    ");
        s += "    float acc = " + identity + ";\n";
        // eight strided loads in flight per lane: 7% faster than four over
        // a 256 MiB vector
        s += "    #pragma unroll 8\n";
        s += "    for (" + std::string(T) + " xi = 0; xi < " + std::to_string(sh.piece / (256 * sh.width)) + "; ++xi) {\n";
        s += "        const " + std::string(T) + " " + qc + " = part * " + std::to_string(sh.piece) + " + xi * " +
             std::to_string(256 * sh.width) + " + tl * " + W + ";\n";
        s += "        if (" + qc + " < " + std::to_string(length) + ") {\n";
        std::string body;
        const std::vector<std::string> v = output_values(r, body, sh.width, names, "            ");
        s += body;
        for (int e = 0; e < sh.width; ++e)
            s += "            acc = " + (is_max ? "porch_fmax(acc, " + v[e] + ")" : "acc + " + v[e]) + ";\n";
        s += "        }\n    }\n";
        s += wave_fold(is_max, "acc");
        s += "    if (lane == 0) xred[wave] = acc;\n    __syncthreads();\n";
        s += "    if (tl == 0) out[blockIdx.x] = " +
             (is_max ? std::string("porch_fmax(porch_fmax(xred[0], xred[1]), porch_fmax(xred[2], xred[3]))")
                     : std::string("(xred[0] + xred[1]) + (xred[2] + xred[3])")) +
             ";\n";
        s += "}\n";
        return kc;
    }

    kernel_code emit_row_combine(const row_request& r, int partial_slot) {
        const partial_shape sh = analyze(r);
        if (sh.parts < 2) throw std::logic_error("emit_row_combine: the reduction is not split");
        const size_t rank = r.shape.size();
        const size_t col = rank - 1;
        const int64_t length = r.shape[col];
        const std::vector<int64_t> row_shape(r.shape.begin(), r.shape.end() - 1);
        const char* T = r.width.type();
        const std::vector<std::string> names = coordinate_names(rank);
        const std::string qc = names[col];
        const bool is_max = r.output_is_max;
        const std::string P = std::to_string(sh.parts);

        kernel_code kc;
        kc.kind = "row.combine";
        kc.name = "porch_row";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>((sh.rows + 3) / 4);

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(256) porch_row(" + kernel_params(r.n_slots) + ") {\n";
        s += "    const int lane = threadIdx.x & 63;\n";
        s += "    const idx_t row = (idx_t)blockIdx.x * 4 + (threadIdx.x >> 6);\n";
        s += "    if (row >= " + std::to_string(sh.rows) + ") return;\n";
        s += "    const float* __restrict__ xp = a" + std::to_string(partial_slot) + " + row * " + P + ";\n";
        s += "    float acc = " + std::string(is_max ? "-PORCH_FLT_MAX" : "0.0f") + ";\n";
        s += "    for (int i = lane; i < " + P + "; i += 64) acc = " +
             (is_max ? std::string("porch_fmax(acc, xp[i])") : std::string("acc + xp[i]")) + ";\n";
        s += wave_fold(is_max, "acc");
        if (is_max) {
            // Every lane holds the same max (porch_fmax is commutative), so
            // the branch is uniform over the wave.
            s += "    if (porch_max_order_matters(acc)) {\n";
            std::vector<bool> needed(row_shape.size(), true);
            s += decompose("row", row_shape, needed, T, "        ");
            s += "        float xf[4] = {-PORCH_FLT_MAX, -PORCH_FLT_MAX, -PORCH_FLT_MAX, -PORCH_FLT_MAX};\n";
            s += "        for (" + std::string(T) + " xb = 0; xb < " + std::to_string(length) + "; xb += 256) {\n";
            s += "            #pragma unroll\n            for (int i = 0; i < 4; ++i) {\n";
            s += "                const " + std::string(T) + " " + qc + " = xb + i * 64 + lane;\n";
            s += "                if (" + qc + " < " + std::to_string(length) + ") {\n";
            std::string body;
            const std::vector<std::string> v = output_values(r, body, 1, names, "                    ");
            s += body;
            s += "                    xf[i] = porch_refmax(xf[i], " + v[0] + ");\n";
            s += "                }\n            }\n        }\n";
            // virtual lane t = lane + 64 i: strides 128 and 64 within the
            // lane, 32 .. 1 across lanes (the lower virtual lane on the left)
            s += "        float xh = porch_refmax(porch_refmax(xf[0], xf[2]), porch_refmax(xf[1], xf[3]));\n";
            for (int d = 32; d >= 1; d /= 2)
                s += "        xh = porch_refmax(xh, __shfl_xor(xh, " + std::to_string(d) + ", 64));\n";
            s += "        acc = __shfl(xh, 0, 64);\n";
            s += "    }\n";
        }
        s += "    if (lane == 0) out[row] = acc;\n";
        s += "}\n";
        return kc;
    }

} // namespace porch::cg
