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
        kernel_code kc;
        kc.kind = "reduce.column";
        kc.name = "porch_reduce";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>(
            std::clamp<int64_t>((outputs + 255) / 256, 1, int64_t{1} << 22)
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
        s += "    for (idx_t o = (idx_t)blockIdx.x * 256 + threadIdx.x; o < " +
             std::to_string(outputs) + "; o += (idx_t)gridDim.x * 256) {\n";
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
        s += std::string("        float acc = ") + (r.is_max ? "-PORCH_FLT_MAX" : "0.0f") +
             ";\n";
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
        emitter em(k, body, 1);
        em.indent = "            ";
        em.declare_roots({r.producer});
        em.load = [&](int id) {
            const knode& n = k.at(id);
            return std::vector<std::string>{
                "a" + std::to_string(n.slot) + "[" + index_text(n.index, names) + "]"
            };
        };
        em.condition = [&](const kcond& c) {
            return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
        };
        em.row_value = [](int) -> std::string {
            throw std::logic_error("row value in a column reduction");
        };
        const std::string v = em.emit(r.producer)[0];
        s += body;
        if (r.is_max) s += "            acc = acc > " + v + " ? acc : " + v + ";\n";
        else s += "            acc += " + v + ";\n";
        s += "        }\n";
        if (parts > 1) s += "        out[(idx_t)blockIdx.y * " + std::to_string(outputs) + " + o] = acc;\n";
        else s += "        out[o] = acc;\n";
        s += "    }\n}\n";
        return kc;
    }

} // namespace porch::cg
