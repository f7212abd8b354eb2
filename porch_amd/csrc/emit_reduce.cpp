// Reductions over a non-last axis.  One lane per output element folds the
// axis sequentially; lanes run along the output's contiguous dimension, so
// each step of the fold is a coalesced read (the reference instead gives
// every output its own 256-thread block, src/tensor.cpp:896-962).  When the
// outputs alone cannot fill the machine, the axis is split into chunks
// folded by separate workgroups (grid y) into partial results, which a
// second pass combines in chunk order.

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

    int64_t column_reduce_parts(const column_reduce_request& r, int compute_units) {
        const int64_t extent = r.shape[r.axis];
        const int64_t outputs = ir::numel(r.shape) / std::max<int64_t>(extent, 1);
        if (extent < 256 || outputs * extent < (int64_t{1} << 20)) return 1;
        const int64_t groups = (outputs / lanes_width(r) + 255) / 256;
        const int64_t target = static_cast<int64_t>(compute_units) * 4;
        const int64_t parts = std::min(target / std::max<int64_t>(groups, 1), extent / 32);
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
        // allow; the fold order per output is unchanged.
        const size_t inner = inner_dim(r);
        const int width = lanes_width(r);
        const int64_t groups = outputs / width;
        kernel_code kc;
        kc.kind = "reduce.column";
        kc.name = "porch_reduce";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>(
            std::clamp<int64_t>((groups + 255) / 256, 1, int64_t{1} << 22)
        );
        const int64_t parts = std::max<int64_t>(r.parts, 1);
        const int64_t chunk = (extent + parts - 1) / parts;
        kc.grid_y = static_cast<unsigned>(parts);
        const char* T = r.width.type();
        std::vector<std::string> names;
        for (size_t d = 0; d < rank; ++d) names.push_back("q" + std::to_string(d));

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(256) porch_reduce(" +
             kernel_params(r.n_slots) + ") {\n";
        s += "    for (idx_t g = (idx_t)blockIdx.x * 256 + threadIdx.x; g < " +
             std::to_string(groups) + "; g += (idx_t)gridDim.x * 256) {\n";
        s += "        const idx_t o = g * " + std::to_string(width) + ";\n";
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
        s += "        float acc[" + std::to_string(width) + "];\n";
        s += "        #pragma unroll\n        for (int e = 0; e < " + std::to_string(width) +
             "; ++e) acc[e] = " + init + ";\n";
        // Unrolled so that several rows' loads are in flight at once; the
        // fold itself stays in row order.
        const std::string qa = "q" + std::to_string(r.axis);
        if (parts > 1) {
            s += std::string("        const ") + T + " first = (" + T + ")blockIdx.y * " +
                 std::to_string(chunk) + ";\n";
            s += std::string("        const ") + T + " last = first + " + std::to_string(chunk) + " < " +
                 std::to_string(extent) + " ? first + " + std::to_string(chunk) + " : " +
                 std::to_string(extent) + ";\n";
            s += "        #pragma unroll 8\n";
            s += std::string("        for (") + T + " " + qa + " = first; " + qa + " < last; ++" + qa + ") {\n";
        }
        else {
            s += "        #pragma unroll 8\n";
            s += std::string("        for (") + T + " " + qa + " = 0; " + qa + " < " +
                 std::to_string(extent) + "; ++" + qa + ") {\n";
        }
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
        for (int e = 0; e < width; ++e) {
            const std::string a = "acc[" + std::to_string(e) + "]";
            if (r.is_max) s += "            " + a + " = " + a + " > " + v[e] + " ? " + a + " : " + v[e] + ";\n";
            else s += "            " + a + " += " + v[e] + ";\n";
        }
        s += "        }\n";
        const std::string dst = parts > 1 ? "(idx_t)blockIdx.y * " + std::to_string(outputs) + " + o" : "o";
        if (width == 4)
            s += "        *reinterpret_cast<float4*>(out + " + dst + ") = make_float4(acc[0], acc[1], acc[2], acc[3]);\n";
        else
            s += "        out[" + dst + "] = acc[0];\n";
        s += "    }\n}\n";
        return kc;
    }

} // namespace porch::cg
