// Reductions over a non-last axis.  Lanes run along the output's contiguous
// dimension, so each step of a fold is a coalesced read (the reference
// instead gives every output its own 256-thread block,
// src/tensor.cpp:896-962).  When there are fewer than 64 output groups per
// workgroup, the spare lanes become strands that fold interleaved rows of
// the same outputs, and the strands' partials are combined through LDS.
// When the outputs alone cannot fill the machine, the axis is split into
// chunks folded by separate workgroups (grid y) into partial results,
// which a second pass combines.

#include "codegen.hpp"
#include "emit_expr.hpp"

#include <algorithm>
#include <stdexcept>

namespace porch::cg {

    namespace {
        // Can each lane take 4 consecutive outputs along the innermost
        // output dimension, with 128-bit loads (leaves unit-stride and
        // 4-aligned along it, or invariant) and selects uniform over them?
        bool vectorizable(const column_reduce_request& r, size_t inner) {
            const kexpr& k = *r.expr;
            if (r.shape[inner] % 4 != 0) return false;
            for (const int id : k.postorder(r.producer)) {
                const knode& n = k.at(id);
                if (n.op == kop::load) {
                    const ival& x = n.index;
                    if (!x.is_affine) return false;
                    if (x.w[inner] == 0) continue;
                    if (x.w[inner] != 1 || x.c0 % 4 != 0) return false;
                    for (size_t d = 0; d < x.w.size(); ++d)
                        if (d != inner && x.w[d] % 4 != 0) return false;
                }
                if (n.op == kop::select) {
                    const ival& c = n.cond.lhs;
                    if (!c.is_affine) return false;
                    if (c.w[inner] != 0) {
                        if (c.w[inner] != 1 || ((n.cond.bound - c.c0) % 4 + 4) % 4 != 0) return false;
                        for (size_t d = 0; d < c.w.size(); ++d)
                            if (d != inner && c.w[d] % 4 != 0) return false;
                    }
                }
            }
            return true;
        }
        size_t inner_dim(const column_reduce_request& r) {
            return r.axis + 1 == r.shape.size() ? r.axis : r.shape.size() - 1;
        }

        int lanes_width(const column_reduce_request& r) {
            const size_t inner = inner_dim(r);
            return (inner != r.axis && vectorizable(r, inner)) ? 4 : 1;
        }
    } // namespace

    namespace {
        // Workgroup layout: `cols` lanes along the output groups (a power of
        // two up to 64, fewer when there are fewer groups) times
        // 256 / cols strands, each strand folding every strands-th row of
        // the axis.
        int layout_cols(int64_t groups, int max_cols = 64) {
            int cols = 1;
            while (cols < max_cols && cols < groups) cols *= 2;
            return cols;
        }
    } // namespace

    namespace {
        // The producer's values at axis position `row_expr` (coordinate
        // variable `qa`) into `dst`[0..width), as a C block: 128-bit loads
        // for leaves unit-stride along the inner output dimension, one
        // load broadcast for leaves invariant along it.
        std::string row_values(const column_reduce_request& r, const std::vector<std::string>& names, size_t inner,
                               int width, const char* T, const std::string& qa, const std::string& row_expr,
                               const std::string& dst, const std::string& ind) {
            const kexpr& k = *r.expr;
            std::string c = ind + "{\n" + ind + "    const " + T + " " + qa + " = " + row_expr + ";\n";
            std::string body;
            emitter em(k, body, width);
            em.indent = ind + "    ";
            em.declare_roots({r.producer});
            em.load = [&](int id) {
                const knode& n = k.at(id);
                const std::string b = "a" + std::to_string(n.slot);
                const std::string idx = index_text(n.index, names);
                if (width == 1) return std::vector<std::string>{b + "[" + idx + "]"};
                if (n.index.w[inner] == 0) {
                    const std::string u = em.fresh("u");
                    em.line("const float " + u + " = " + b + "[" + idx + "];");
                    return std::vector<std::string>(4, u);
                }
                const std::string w = em.fresh("w");
                em.line("const float4 " + w + " = *reinterpret_cast<const float4*>(" + b + " + " + idx + ");");
                return std::vector<std::string>{w + ".x", w + ".y", w + ".z", w + ".w"};
            };
            em.condition = [&](const kcond& cd) { return index_text(cd.lhs, names) + " < " + std::to_string(cd.bound); };
            em.row_value = [](int) -> std::string { throw std::logic_error("row value in a column reduction"); };
            const std::vector<std::string> v = em.emit(r.producer);
            c += body;
            for (int e = 0; e < width; ++e)
                c += ind + "    " + dst + "[" + std::to_string(e) + "] = " + v[static_cast<size_t>(e)] + ";\n";
            return c + ind + "}\n";
        }

    } // namespace

    namespace {
        // Outputs whose order-free max may differ from the reference's
        // (porch_max_order_matters: a NaN, or a +0 maximum) are recomputed
        // by the whole workgroup in the reference's block order
        // (src/tensor.cpp:896-962): thread t folds axis positions t,
        // t + 256, ... with t = t > v ? t : v from -FLT_MAX, and the 256
        // partials go through the tree with strides 128, 64, ..., 1 (the
        // first two within each lane of wave 0, the rest across its lanes).
        // Every wave ballots the flags from the combined results in LDS, so
        // the loop over flagged outputs is uniform; the result replaces the
        // combined value before the store.
        std::string exact_column_max(const column_reduce_request& r, const std::string& W,
                                     const std::string& C, const char* T) {
            const kexpr& k = *r.exact_expr;
            const size_t rank = r.exact_shape.size();
            std::vector<int64_t> out_shape;
            std::vector<size_t> out_dims;
            for (size_t d = 0; d < rank; ++d) {
                if (d == r.exact_axis) continue;
                out_shape.push_back(r.exact_shape[d]);
                out_dims.push_back(d);
            }
            std::vector<std::string> names;
            for (size_t d = 0; d < rank; ++d) names.push_back("q" + std::to_string(d));
            const std::string qa = "q" + std::to_string(r.exact_axis);
            std::string s;
            s += "        #pragma unroll\n        for (int e = 0; e < " + W + "; ++e) {\n";
            s += "            const bool xflag = lane < " + C + " && base + lane < " + std::to_string(
                     ir::numel(out_shape) / std::stoll(W)) + " && porch_max_order_matters(partial[0][lane][e]);\n";
            s += "            unsigned long long xmask = __ballot(xflag);\n";
            s += "            while (xmask) {\n";
            s += "                const int u = __builtin_ctzll(xmask);\n";
            s += "                xmask &= xmask - 1;\n";
            s += "                const idx_t xo = (base + u) * " + W + " + e;\n";
            const std::vector<int64_t> ostr = ir::contiguous_strides(out_shape);
            for (size_t i = 0; i < out_dims.size(); ++i) {
                std::string value;
                if (out_shape[i] == 1) value = "0";
                else if (i == 0) value = "xo / " + std::to_string(ostr[i]);
                else if (ostr[i] == 1) value = "xo % " + std::to_string(out_shape[i]);
                else value = "(xo / " + std::to_string(ostr[i]) + ") % " + std::to_string(out_shape[i]);
                s += std::string("                const ") + T + " q" + std::to_string(out_dims[i]) + " = " + value + ";\n";
            }
            s += "                float xf = -PORCH_FLT_MAX;\n";
            s += std::string("                for (") + T + " " + qa + " = threadIdx.x; " + qa + " < " +
                 std::to_string(r.exact_shape[r.exact_axis]) + "; " + qa + " += 256) {\n";
            std::string body;
            emitter em(k, body, 1);
            em.indent = "                    ";
            em.declare_roots({r.exact_producer});
            em.load = [&](int id) {
                const knode& n = k.at(id);
                return std::vector<std::string>{"a" + std::to_string(n.slot) + "[" + index_text(n.index, names) + "]"};
            };
            em.condition = [&](const kcond& c) {
                return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
            };
            em.row_value = [](int) -> std::string {
                throw std::logic_error("row value in a column reduction");
            };
            const std::vector<std::string> v = em.emit(r.exact_producer);
            em.line("xf = porch_refmax(xf, " + v[0] + ");");
            s += body + "                }\n";
            s += "                ex[threadIdx.x] = xf;\n";
            s += "                __syncthreads();\n";
            s += "                if (wave == 0) {\n";
            s += "                    float xh = porch_refmax(porch_refmax(ex[lane], ex[lane + 128]),\n"
                 "                                            porch_refmax(ex[lane + 64], ex[lane + 192]));\n";
            for (int m = 32; m >= 1; m /= 2)
                s += "                    xh = porch_refmax(xh, __shfl_xor(xh, " + std::to_string(m) + ", 64));\n";
            s += "                    if (lane == 0) partial[0][u][e] = xh;\n";
            s += "                }\n";
            s += "                __syncthreads();\n";
            s += "            }\n";
            s += "        }\n";
            return s;
        }
    } // namespace

    int64_t column_reduce_parts(const column_reduce_request& r, int compute_units) {
        const int64_t extent = r.shape[r.axis];
        const int64_t outputs = ir::numel(r.shape) / std::max<int64_t>(extent, 1);
        if (extent < 256 || outputs * extent < (int64_t{1} << 20)) return 1;
        const int64_t groups = outputs / lanes_width(r);
        const int cols = layout_cols(groups);
        const int64_t strands = 256 / cols;
        const int64_t workgroups = (groups + cols - 1) / cols;
        const int64_t target = static_cast<int64_t>(compute_units) * 4;
        // at least 4 rows per strand in each part
        const int64_t parts = std::min(target / std::max<int64_t>(workgroups, 1), extent / (4 * strands));
        return std::max<int64_t>(parts, 1);
    }

    kernel_code emit_column_reduce(const column_reduce_request& r) {
        const size_t rank = r.shape.size();
        std::vector<int64_t> out_shape;
        std::vector<size_t> out_dims;
        for (size_t d = 0; d < rank; ++d) {
            if (d == r.axis) continue;
            out_shape.push_back(r.shape[d]);
            out_dims.push_back(d);
        }
        const int64_t outputs = ir::numel(out_shape);
        const int64_t extent = r.shape[r.axis];
        // 4 outputs per lane (128-bit loads and stores) where the leaves
        // allow.
        const size_t inner = inner_dim(r);
        const int width = lanes_width(r);
        const int64_t groups = outputs / width;
        const int cols = layout_cols(groups, std::clamp(r.max_cols, 1, 64));
        const int strands = 256 / cols;
        kernel_code kc;
        kc.kind = "reduce.column";
        kc.name = "porch_reduce";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>(
            std::clamp<int64_t>((groups + cols - 1) / cols, 1, int64_t{1} << 22)
        );
        const int64_t parts = std::max<int64_t>(r.parts, 1);
        const int64_t chunk = (extent + parts - 1) / parts;
        kc.grid_y = static_cast<unsigned>(parts);
        const char* T = r.width.type();
        std::vector<std::string> names;
        for (size_t d = 0; d < rank; ++d) names.push_back("q" + std::to_string(d));
        const std::string W = std::to_string(width);
        const std::string C = std::to_string(cols);
        const std::string S = std::to_string(strands);

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(256) porch_reduce(" +
             kernel_params(r.n_slots) + ") {\n";
        if (strands > 1) s += "    __shared__ float partial[" + S + "][" + C + "][" + W + "];\n";
        const bool exact = r.is_max && r.exact_expr != nullptr;
        if (exact) {
            if (strands < 2) throw std::logic_error("exact column max needs the strand partials in LDS");
            s += "    __shared__ float ex[257];\n";
            s += "    const int lane = threadIdx.x & 63;\n";
            s += "    const int wave = threadIdx.x >> 6;\n";
        }
        s += "    const int cl = threadIdx.x % " + C + ";\n";
        s += "    const int strand = threadIdx.x / " + C + ";\n";
        // The group loop is uniform across the workgroup (barriers inside);
        // `live` marks lanes past the last group.
        s += "    for (idx_t base = (idx_t)blockIdx.x * " + C + "; base < " + std::to_string(groups) +
             "; base += (idx_t)gridDim.x * " + C + ") {\n";
        s += "        const idx_t g = base + cl;\n";
        s += "        const bool live = g < " + std::to_string(groups) + ";\n";
        s += "        const idx_t o = g * " + W + ";\n";
        const std::vector<int64_t> ostr = ir::contiguous_strides(out_shape);
        for (size_t i = 0; i < out_dims.size(); ++i) {
            std::string value;
            if (out_shape[i] == 1) value = "0";
            else if (i == 0) value = "o / " + std::to_string(ostr[i]);
            else if (ostr[i] == 1) value = "o % " + std::to_string(out_shape[i]);
            else
                value = "(o / " + std::to_string(ostr[i]) + ") % " +
                        std::to_string(out_shape[i]);
            s += std::string("        const ") + T + " q" + std::to_string(out_dims[i]) +
                 " = " + value + ";\n";
        }
        const std::string init = r.is_max ? "-PORCH_FLT_MAX" : "0.0f";
        s += "        float acc[" + W + "];\n";
        s += "        #pragma unroll\n        for (int e = 0; e < " + W + "; ++e) acc[e] = " + init + ";\n";
        // Each strand folds rows strand, strand + strands, ... of its chunk
        // in order.
        const std::string qa = "q" + std::to_string(r.axis);
        const std::string first = parts > 1 ? "(" + std::string(T) + ")blockIdx.y * " + std::to_string(chunk) : "0";
        if (parts > 1) {
            s += std::string("        const ") + T + " first = " + first + ";\n";
            s += std::string("        const ") + T + " last = first + " + std::to_string(chunk) + " < " +
                 std::to_string(extent) + " ? first + " + std::to_string(chunk) + " : " +
                 std::to_string(extent) + ";\n";
        }
        else {
            s += std::string("        const ") + T + " first = 0;\n";
            s += std::string("        const ") + T + " last = " + std::to_string(extent) + ";\n";
        }
        // Max folds are order-free (porch_fmax); outputs where the order
        // can matter are recomputed in the reference's order below.
        auto combine = [&](const std::string& a, const std::string& b) {
            return r.is_max ? "porch_fmax(" + a + ", " + b + ")" : a + " + " + b;
        };
        // One row a step, without an unroll pragma: loading 4, 8 or 16 rows
        // a step (their loads in flight together) was slower on max over
        // axis 0 of [8192, 8192] (54.7, 57.7, 49.4 against 48.3 us) and
        // within 7% either way on sums over [4096, 4096], [1048576, 4],
        // [65536, 64], [8192, 300] and over axis 1 of [64, 4096, 64].
        s += "        if (live) {\n";
        s += std::string("        for (") + T + " qb = first + strand; qb < last; qb += " + S + ") {\n";
        s += "            float rt[" + W + "];\n";
        s += row_values(r, names, inner, width, T, qa, "qb", "rt", "            ");
        s += "            #pragma unroll\n            for (int e = 0; e < " + W + "; ++e) acc[e] = " +
             combine("acc[e]", "rt[e]") + ";\n";
        s += "        }\n        }\n";
        const std::string dst = parts > 1 ? "(idx_t)blockIdx.y * " + std::to_string(outputs) + " + o" : "o";
        std::string result = "acc";
        if (strands > 1) {
            // Strand partials combined pairwise through LDS, in a fixed order.
            s += "        #pragma unroll\n        for (int e = 0; e < " + W + "; ++e) partial[strand][cl][e] = acc[e];\n";
            s += "        __syncthreads();\n";
            s += "        #pragma unroll\n";
            s += "        for (int h = " + std::to_string(strands / 2) + "; h >= 1; h >>= 1) {\n";
            s += "            if (strand < h) {\n";
            s += "                #pragma unroll\n                for (int e = 0; e < " + W + "; ++e)\n";
            s += "                    partial[strand][cl][e] = " +
                 combine("partial[strand][cl][e]", "partial[strand + h][cl][e]") + ";\n";
            s += "            }\n            __syncthreads();\n        }\n";
            result = "partial[0][cl]";
        }
        if (exact) s += exact_column_max(r, W, C, T);
        s += std::string("        if (") + (strands > 1 ? "strand == 0 && " : "") + "live) {\n";
        if (width == 4)
            s += "            *reinterpret_cast<float4*>(out + " + dst + ") = make_float4(" + result + "[0], " +
                 result + "[1], " + result + "[2], " + result + "[3]);\n";
        else
            s += "            out[" + dst + "] = " + result + "[0];\n";
        s += "        }\n";
        if (strands > 1) s += "        __syncthreads();\n";
        s += "    }\n}\n";
        return kc;
    }

    namespace {
        // The combination of column softmax partial triples [3][parts][outputs]
        // (m, a, t per part and output) into [2][outputs]: first M, the max
        // of the parts' m (order-free), then S = sum t exp(a - M) (each
        // anchor a is a value of its part, so a <= M and every factor is at
        // most 1).  Lanes along the outputs (4 per lane where the outputs
        // allow), the rest of the workgroup strands over the parts; each
        // strand's values go through a fixed pairwise tree in LDS.  Two
        // plain trees (a max, then a sum) instead of one of merges: no chain
        // of dependent exps.
        kernel_code emit_softmax_combine(const column_reduce_request& r, int partial_slot) {
            const int64_t parts = r.shape[0];
            const int64_t outputs = r.shape[1];
            const int width = outputs % 4 == 0 ? 4 : 1;
            const int64_t groups = outputs / width;
            const int cols = layout_cols(groups, std::clamp(r.max_cols, 1, 64));
            const int strands = 256 / cols;
            kernel_code kc;
            kc.kind = "reduce.column_softmax_combine";
            kc.name = "porch_reduce";
            kc.n_slots = r.n_slots;
            kc.block = 256;
            kc.grid_x = static_cast<unsigned>(std::clamp<int64_t>((groups + cols - 1) / cols, 1, int64_t{1} << 22));
            const char* T = r.width.type();
            const std::string W = std::to_string(width);
            const std::string C = std::to_string(cols);
            const std::string S = std::to_string(strands);
            const std::string O = std::to_string(outputs);
            const std::string P = std::to_string(parts);
            const std::string slot = "a" + std::to_string(partial_slot);
            std::string& s = kc.source;
            s = kernel_prologue(r.n_slots, T);
            s += "extern \"C\" __global__ void __launch_bounds__(256) porch_reduce(" + kernel_params(r.n_slots) + ") {\n";
            s += "    __shared__ float red[" + S + "][" + C + "][" + W + "];\n";
            s += "    const int cl = threadIdx.x % " + C + ";\n";
            s += "    const int strand = threadIdx.x / " + C + ";\n";
            s += "    for (idx_t base = (idx_t)blockIdx.x * " + C + "; base < " + std::to_string(groups) +
                 "; base += (idx_t)gridDim.x * " + C + ") {\n";
            s += "        const idx_t g = base + cl;\n";
            s += "        const bool live = g < " + std::to_string(groups) + ";\n";
            s += "        const idx_t o = g * " + W + ";\n";
            auto load = [&](int j, const std::string& name) {
                const std::string at = slot + " + ((idx_t)" + std::to_string(j) + " * " + P + " + qp) * " + O + " + o";
                if (width == 4)
                    return "                const float4 " + name + "4 = *reinterpret_cast<const float4*>(" + at + ");\n" +
                           "                const float " + name + "[4] = {" + name + "4.x, " + name + "4.y, " + name +
                           "4.z, " + name + "4.w};\n";
                return "                const float " + name + "[1] = {*(" + at + ")};\n";
            };
            auto tree = [&](const std::string& acc, bool is_max) {
                std::string c;
                c += "        #pragma unroll\n        for (int e = 0; e < " + W + "; ++e) red[strand][cl][e] = " + acc + "[e];\n";
                c += "        __syncthreads();\n";
                c += "        #pragma unroll\n        for (int h = " + std::to_string(strands / 2) + "; h >= 1; h >>= 1) {\n";
                c += "            if (strand < h) {\n";
                c += "                #pragma unroll\n                for (int e = 0; e < " + W + "; ++e)\n";
                c += std::string("                    red[strand][cl][e] = ") +
                     (is_max ? "porch_fmax(red[strand][cl][e], red[strand + h][cl][e]);\n"
                             : "red[strand][cl][e] + red[strand + h][cl][e];\n");
                c += "            }\n            __syncthreads();\n        }\n";
                c += "        #pragma unroll\n        for (int e = 0; e < " + W + "; ++e) " + acc + "[e] = red[0][cl][e];\n";
                c += "        __syncthreads();\n";
                return c;
            };
            s += "        float m[" + W + "], t[" + W + "];\n";
            s += "        #pragma unroll\n        for (int e = 0; e < " + W + "; ++e) { m[e] = -PORCH_FLT_MAX; t[e] = 0.0f; }\n";
            s += "        if (live) {\n";
            s += "            #pragma unroll 4\n";
            s += std::string("            for (") + T + " qp = strand; qp < " + P + "; qp += " + S + ") {\n";
            s += load(0, "pm");
            s += "                #pragma unroll\n                for (int e = 0; e < " + W + "; ++e) m[e] = porch_fmax(m[e], pm[e]);\n";
            s += "            }\n        }\n";
            s += tree("m", true);
            s += "        if (live) {\n";
            s += "            #pragma unroll 4\n";
            s += std::string("            for (") + T + " qp = strand; qp < " + P + "; qp += " + S + ") {\n";
            s += load(1, "pa");
            s += load(2, "pt");
            s += "                #pragma unroll\n                for (int e = 0; e < " + W +
                 "; ++e) t[e] += pt[e] * porch_exp(pa[e] - m[e]);\n";
            s += "            }\n        }\n";
            s += tree("t", false);
            s += "        if (strand == 0 && live) {\n";
            if (width == 4) {
                s += "            *reinterpret_cast<float4*>(out + o) = make_float4(m[0], m[1], m[2], m[3]);\n";
                s += "            *reinterpret_cast<float4*>(out + " + O + " + o) = make_float4(t[0], t[1], t[2], t[3]);\n";
            }
            else {
                s += "            out[o] = m[0];\n            out[" + O + " + o] = t[0];\n";
            }
            s += "        }\n    }\n}\n";
            return kc;
        }
    } // namespace

    // Softmax statistics along a non-last axis in one read: for each
    // output column, the max M of f and S = sum exp(f - M), where the
    // reference reads f twice (a max, then a sum of exp(f - max)).
    //
    // Each lane folds its values into a triple (m, a, t): m the order-free
    // max (porch_fmax, from -FLT_MAX as the reference's fold starts), a an
    // anchor and t = sum exp(f - a).  The anchor starts at -FLT_MAX and
    // moves to a value only when that value exceeds it by more than 1 (t
    // rescaled by exp(a_old - a_new)), so it stays within 1 below the max:
    // the large terms are then exp of small differences f - a, whose float
    // rounding (relative to |f - a|) stays at the reference's level.  (With
    // the anchor up to 64 below the max, as for rows, the largest terms
    // carried that rounding times |f - a| ~ 20 on N(0, 9) columns: 1.3e-6
    // against the oracle on [8, 300, 64] over axis 1.)  Each move shrinks
    // the earlier terms by e^-1 or more, so the rescales' own roundings
    // fade geometrically.  Triples merge as m = max, a = the larger
    // anchor, t = t1 exp(a1 - a) + t2 exp(a2 - a); the statistics are
    // M = m and S = t exp(a - M).  NaN in the column gives S = NaN, +inf
    // gives exp(inf - inf) = NaN, a column of -inf gives M = -FLT_MAX and
    // S = 0: the reference's values for the softmax built on them.  (M is
    // order-free: it may differ from the reference's max in the sign of a
    // zero or by being NaN where the reference's is not, which changes no
    // value of exp(f - M) / S.)
    //
    // partial_slot < 0: the first pass over `r.producer`, chunks of the
    // axis per grid y when r.parts > 1, each (chunk, output) triple to out
    // as [3][parts][outputs]; with one part, M and S directly to out as
    // [2][outputs].  partial_slot >= 0: the combination of such triples
    // (r.shape = {parts, outputs}) into [2][outputs] (emit_softmax_combine).
    kernel_code emit_column_softmax(const column_reduce_request& r, int partial_slot) {
        if (partial_slot >= 0) return emit_softmax_combine(r, partial_slot);
        const size_t rank = r.shape.size();
        std::vector<int64_t> out_shape;
        std::vector<size_t> out_dims;
        for (size_t d = 0; d < rank; ++d) {
            if (d == r.axis) continue;
            out_shape.push_back(r.shape[d]);
            out_dims.push_back(d);
        }
        const int64_t outputs = ir::numel(out_shape);
        const int64_t extent = r.shape[r.axis];
        const size_t inner = inner_dim(r);
        const int width = lanes_width(r);
        const int64_t groups = outputs / width;
        const int cols = layout_cols(groups, std::clamp(r.max_cols, 1, 64));
        const int strands = 256 / cols;
        const int64_t parts = std::max<int64_t>(r.parts, 1);
        const int64_t chunk = (extent + parts - 1) / parts;
        kernel_code kc;
        kc.kind = "reduce.column_softmax";
        kc.name = "porch_reduce";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>(std::clamp<int64_t>((groups + cols - 1) / cols, 1, int64_t{1} << 22));
        kc.grid_y = static_cast<unsigned>(parts);
        const char* T = r.width.type();
        std::vector<std::string> names;
        for (size_t d = 0; d < rank; ++d) names.push_back("q" + std::to_string(d));
        const std::string W = std::to_string(width);
        const std::string C = std::to_string(cols);
        const std::string S = std::to_string(strands);
        const std::string O = std::to_string(outputs);

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        // Merges triple (m2, a2, t2) into (m, a, t).
        s += "__device__ __forceinline__ void porch_softmax_merge(float& m, float& a, float& t, float m2, float a2, "
             "float t2) {\n";
        s += "    m = porch_fmax(m, m2);\n";
        s += "    const float an = a2 > a ? a2 : a;\n";
        s += "    t = t * porch_exp(a - an) + t2 * porch_exp(a2 - an);\n";
        s += "    a = an;\n";
        s += "}\n";
        s += "extern \"C\" __global__ void __launch_bounds__(256) porch_reduce(" + kernel_params(r.n_slots) + ") {\n";
        if (strands > 1) {
            for (const char* x : {"pm", "pa", "pt"})
                s += std::string("    __shared__ float ") + x + "[" + S + "][" + C + "][" + W + "];\n";
        }
        s += "    const int cl = threadIdx.x % " + C + ";\n";
        s += "    const int strand = threadIdx.x / " + C + ";\n";
        s += "    for (idx_t base = (idx_t)blockIdx.x * " + C + "; base < " + std::to_string(groups) +
             "; base += (idx_t)gridDim.x * " + C + ") {\n";
        s += "        const idx_t g = base + cl;\n";
        s += "        const bool live = g < " + std::to_string(groups) + ";\n";
        s += "        const idx_t o = g * " + W + ";\n";
        {
            const std::vector<int64_t> ostr = ir::contiguous_strides(out_shape);
            for (size_t i = 0; i < out_dims.size(); ++i) {
                std::string value;
                if (out_shape[i] == 1) value = "0";
                else if (i == 0) value = "o / " + std::to_string(ostr[i]);
                else if (ostr[i] == 1) value = "o % " + std::to_string(out_shape[i]);
                else value = "(o / " + std::to_string(ostr[i]) + ") % " + std::to_string(out_shape[i]);
                s += std::string("        const ") + T + " q" + std::to_string(out_dims[i]) + " = " + value + ";\n";
            }
        }
        s += "        float m[" + W + "], a[" + W + "], t[" + W + "];\n";
        s += "        #pragma unroll\n        for (int e = 0; e < " + W +
             "; ++e) { m[e] = -PORCH_FLT_MAX; a[e] = -PORCH_FLT_MAX; t[e] = 0.0f; }\n";
        const std::string qa = "q" + std::to_string(r.axis);
        if (parts > 1) {
            s += std::string("        const ") + T + " first = (" + T + ")blockIdx.y * " + std::to_string(chunk) + ";\n";
            s += std::string("        const ") + T + " last = first + " + std::to_string(chunk) + " < " +
                 std::to_string(extent) + " ? first + " + std::to_string(chunk) + " : " + std::to_string(extent) + ";\n";
        }
        else {
            s += std::string("        const ") + T + " first = 0;\n";
            s += std::string("        const ") + T + " last = " + std::to_string(extent) + ";\n";
        }
        s += "        if (live) {\n";
        {
            auto values_at = [&](const std::string& row_expr, const std::string& dst, const std::string& ind) {
                return row_values(r, names, inner, width, T, qa, row_expr, dst, ind);
            };
            // Four rows a step: their loads issued together, then one
            // anchor decision per output for the four (branch-free: a step
            // that keeps the anchor rescales by exp(0) = 1).
            s += std::string("        ") + T + " qb = first + strand;\n";
            s += "        for (; qb + " + std::to_string(3 * strands) + " < last; qb += " + std::to_string(4 * strands) + ") {\n";
            s += "            float rb0[" + W + "], rb1[" + W + "], rb2[" + W + "], rb3[" + W + "];\n";
            for (int j = 0; j < 4; ++j)
                s += values_at("qb + " + std::to_string(j * strands), "rb" + std::to_string(j), "            ");
            s += "            #pragma unroll\n            for (int e = 0; e < " + W + "; ++e) {\n";
            s += "                const float bm = porch_fmax(porch_fmax(rb0[e], rb1[e]), porch_fmax(rb2[e], rb3[e]));\n";
            s += "                m[e] = porch_fmax(m[e], bm);\n";
            s += "                const float an = bm > a[e] + 1.0f ? bm : a[e];\n";
            s += "                t[e] = t[e] * porch_exp(a[e] - an) + ((porch_exp(rb0[e] - an) + porch_exp(rb1[e] - an)) + "
                 "(porch_exp(rb2[e] - an) + porch_exp(rb3[e] - an)));\n";
            s += "                a[e] = an;\n";
            s += "            }\n";
            s += "        }\n";
            // the last rows, one at a time
            s += "        for (; qb < last; qb += " + S + ") {\n";
            s += "            float rt[" + W + "];\n";
            s += values_at("qb", "rt", "            ");
            s += "            #pragma unroll\n            for (int e = 0; e < " + W + "; ++e) {\n";
            s += "                m[e] = porch_fmax(m[e], rt[e]);\n";
            s += "                const float an = rt[e] > a[e] + 1.0f ? rt[e] : a[e];\n";
            s += "                t[e] = t[e] * porch_exp(a[e] - an) + porch_exp(rt[e] - an);\n";
            s += "                a[e] = an;\n";
            s += "            }\n";
            s += "        }\n";
        }
        s += "        }\n";
        if (strands > 1) {
            // Strand triples merged pairwise through LDS, in a fixed order.
            s += "        #pragma unroll\n        for (int e = 0; e < " + W +
                 "; ++e) { pm[strand][cl][e] = m[e]; pa[strand][cl][e] = a[e]; pt[strand][cl][e] = t[e]; }\n";
            s += "        __syncthreads();\n";
            s += "        #pragma unroll\n";
            s += "        for (int h = " + std::to_string(strands / 2) + "; h >= 1; h >>= 1) {\n";
            s += "            if (strand < h) {\n";
            s += "                #pragma unroll\n                for (int e = 0; e < " + W + "; ++e) {\n";
            s += "                    float mm = pm[strand][cl][e], aa = pa[strand][cl][e], tt = pt[strand][cl][e];\n";
            s += "                    porch_softmax_merge(mm, aa, tt, pm[strand + h][cl][e], pa[strand + h][cl][e], "
                 "pt[strand + h][cl][e]);\n";
            s += "                    pm[strand][cl][e] = mm; pa[strand][cl][e] = aa; pt[strand][cl][e] = tt;\n";
            s += "                }\n";
            s += "            }\n            __syncthreads();\n        }\n";
            s += "        #pragma unroll\n        for (int e = 0; e < " + W +
                 "; ++e) { m[e] = pm[0][cl][e]; a[e] = pa[0][cl][e]; t[e] = pt[0][cl][e]; }\n";
        }
        s += std::string("        if (") + (strands > 1 ? "strand == 0 && " : "") + "live) {\n";
        auto store = [&](const std::string& at, const std::string& arr) {
            if (width == 4)
                s += "            *reinterpret_cast<float4*>(out + " + at + ") = make_float4(" + arr + "[0], " + arr + "[1], " +
                     arr + "[2], " + arr + "[3]);\n";
            else
                s += "            out[" + at + "] = " + arr + "[0];\n";
        };
        if (parts > 1) {
            const std::string PO = std::to_string(parts * outputs);
            store("(idx_t)blockIdx.y * " + O + " + o", "m");
            store(PO + " + (idx_t)blockIdx.y * " + O + " + o", "a");
            store("(idx_t)2 * " + PO + " + (idx_t)blockIdx.y * " + O + " + o", "t");
        }
        else {
            s += "            float sum[" + W + "];\n";
            s += "            #pragma unroll\n            for (int e = 0; e < " + W +
                 "; ++e) sum[e] = t[e] * porch_exp(a[e] - m[e]);\n";
            store("o", "m");
            store(O + " + o", "sum");
        }
        s += "        }\n";
        if (strands > 1) s += "        __syncthreads();\n";
        s += "    }\n}\n";
        return kc;
    }

} // namespace porch::cg
