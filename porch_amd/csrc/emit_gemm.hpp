#pragma once

// Helpers shared by the matmul emitters (emit_gemm.cpp, emit_gemm_skinny.cpp).

#include "codegen.hpp"
#include "emit_expr.hpp"

#include <string>
#include <vector>

namespace porch::cg {

    // Element index of operand `op` at (row, col) of batch entry `batch`
    // (empty: not batched), as C text.
    std::string operand_index(const gemm_operand& op, const std::string& row, const std::string& col,
                              const std::string& batch = "");

    // Sets up `em` to emit the request's epilogue at coordinates `names`
    // with the accumulated product `acc` as row value 0.
    void epilogue_emitter(emitter& em, const gemm_request& r, const std::vector<std::string>& names,
                          const std::string& acc);

} // namespace porch::cg
