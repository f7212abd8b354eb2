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
        const kexpr& k = *r.expr;
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
        // in order; unrolled so that several rows' loads are in flight.
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
        s += "        if (live) {\n";
        s += "        #pragma unroll 4\n";
        s += std::string("        for (") + T + " " + qa + " = first + strand; " + qa + " < last; " + qa +
             " += " + S + ") {\n";
        std::string body;
        emitter em(k, body, width);
        em.indent = "            ";
        em.declare_roots({r.producer});
        em.load = [&](int id) {
            const knode& n = k.at(id);
            const std::string base = "a" + std::to_string(n.slot);
            const std::string idx = index_text(n.index, names);
            if (width == 1) return std::vector<std::string>{base + "[" + idx + "]"};
            if (n.index.w[inner] == 0) {
                const std::string u = em.fresh("u");
                em.line("const float " + u + " = " + base + "[" + idx + "];");
                return std::vector<std::string>(4, u);
            }
            const std::string w = em.fresh("w");
            em.line("const float4 " + w + " = *reinterpret_cast<const float4*>(" + base + " + " + idx + ");");
            return std::vector<std::string>{w + ".x", w + ".y", w + ".z", w + ".w"};
        };
        em.condition = [&](const kcond& c) {
            return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
        };
        em.row_value = [](int) -> std::string {
            throw std::logic_error("row value in a column reduction");
        };
        const std::vector<std::string> v = em.emit(r.producer);
        s += body;
        // Max folds are order-free (porch_fmax); outputs where the order
        // can matter are recomputed in the reference's order below.
        auto combine = [&](const std::string& a, const std::string& b) {
            return r.is_max ? "porch_fmax(" + a + ", " + b + ")" : a + " + " + b;
        };
        for (int e = 0; e < width; ++e) {
            const std::string a = "acc[" + std::to_string(e) + "]";
            s += "            " + a + " = " + combine(a, v[e]) + ";\n";
        }
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

} // namespace porch::cg
