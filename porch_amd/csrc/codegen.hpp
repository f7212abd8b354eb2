#pragma once

// Emitters of gfx950 HIP source for fused regions.  Each emitter takes a
// lowered kernel expression (lower.hpp) and produces one kernel with its
// launch geometry.  Kernel classes:
//
//   pointwise.flat   wave64 grid loop, 4 outputs per lane with 128-bit loads
//                    and stores wherever every leaf is unit-stride (or
//                    invariant) along the innermost output dimension;
//   pointwise.tiled  64x64 output tiles whose transposed leaves are read with
//                    lanes along the leaf's contiguous dimension, staged in
//                    LDS (padded rows, conflict-free) and written with lanes
//                    along the output's contiguous dimension;
//   pointwise.scalar one output per lane, any index map (div/mod allowed);
//   row              one wave (or workgroup) per row: the row's leaves are
//                    read once into registers, each row reduction is a
//                    register fold plus a wave butterfly, and the outputs (or
//                    the row's reduction) are written in the same pass;
//   row.partial,     a single fold over few long rows: partials of pieces of
//   row.combine      each row in one kernel, combined per row in a second;
//   row.split        softmax-shaped rows of more than 32768 values: each row
//                    split over workgroups that exchange partial (max, sum)
//                    words, so the row is read once;
//   reduce.column    one lane per output, sequential fold over a non-last
//                    axis with lanes along the contiguous output dimension;
//   reduce.column_softmax  the same layout folding a softmax's max and sum
//                    (relative to a moving anchor) in one read;
//   gemm             LDS-tiled v_mfma_f32_32x32x2f32 with the elementwise
//                    epilogue applied to the accumulators before the store;
//   gemm.rows,       products with a few rows (or columns), streaming the
//   gemm.cols        long operand once;
//   gemm.narrow      7 to 32 columns over many rows: v_mfma_f32_16x16x4f32
//                    blocks fed straight from 128-bit loads of A;
//   gemm.wide        8 to 32 (64) rows over many columns: the same blocks
//                    fed from 128-bit loads of B;
//   gemm.combine     the sum of K-chunk partial products (gemm.rows,
//                    gemm.narrow, gemm.wide, or the MFMA kernel split over
//                    K), with the epilogue.

#include "lower.hpp"

#include <string>
#include <vector>

namespace porch::cg {

    struct kernel_code {
        std::string kind;
        std::string name;
        std::string source;
        unsigned grid_x = 1;
        unsigned grid_y = 1;
        unsigned grid_z = 1;
        unsigned block = 256;
        int n_slots = 0; // kernel takes slot 0..n_slots-1, then `out`
    };

    // Largest element count of any tensor the kernel touches; decides
    // between 32- and 64-bit index arithmetic.
    struct index_width {
        bool wide = false;
        [[nodiscard]] const char* type() const {
            return wide ? "long long" : "int";
        }
    };

    struct pointwise_request {
        const kexpr* expr = nullptr;
        int root = -1;
        std::vector<int64_t> shape; // output shape (kernel coordinates)
        int n_slots = 0;
        std::vector<int64_t> slot_elems; // floats each slot's buffer holds
        index_width width;
        int compute_units = 256;
    };

    kernel_code emit_pointwise(const pointwise_request& request);

    // Row programs: reductions over the last axis of `shape` consumed
    // through broadcasts, then either an elementwise output over `shape`
    // or a final reduction per row.
    struct row_reduction {
        bool is_max = false; // sum otherwise
        int producer = -1;   // kexpr root of the reduced values
    };
    struct row_request {
        const kexpr* expr = nullptr;
        std::vector<int64_t> shape; // row space [rows..., L]
        std::vector<row_reduction> reductions; // in dependency order
        bool reduce_output = false; // output is one value per row
        bool output_is_max = false;
        int output = -1;            // kexpr root of the output values
        int n_slots = 0;
        index_width width;
        int compute_units = 256;
        // Rows split over workgroups (row_split_parts > 0): the slot of a
        // zeroed temporary of rows x parts 64-bit words through which the
        // parts of a row exchange their partial reductions.
        int split_slot = -1;
        int64_t split_parts = 0;
    };

    kernel_code emit_row(const row_request& request);
    // How many workgroups each row is split over (0: not split): rows of
    // more than 32768 values in a softmax-shaped program (a max, then a
    // sum of exp(f - that max), then an elementwise output) over a single
    // leaf, so that each row is read from memory once.
    int64_t row_split_parts(const row_request& request);
    // Floats of the exchange temporary a split row program needs.
    int64_t row_split_temp_floats(const row_request& request);
    // The split form (emit_row_split.cpp); `request.split_slot` and
    // `split_parts` set, the temporary zeroed before the launch.
    kernel_code emit_row_split(const row_request& request);
    // A single fold per row over few, long rows (emit_row_partial.cpp): the
    // number of pieces each row is split into (0: not split), then the two
    // kernels: partials of every (row, piece) into a [rows, parts]
    // temporary (the kernel's `out`), and their combination per row from
    // slot `partial_slot`.
    int64_t row_partial_parts(const row_request& request);
    kernel_code emit_row_partial(const row_request& request);
    kernel_code emit_row_combine(const row_request& request, int partial_slot);

    struct column_reduce_request {
        const kexpr* expr = nullptr;
        int producer = -1;
        std::vector<int64_t> shape; // producer shape
        size_t axis = 0;            // reduced axis (not the last)
        bool is_max = false;
        int n_slots = 0;
        index_width width;
        // > 1: the axis is split into `parts` chunks (grid y); chunk g's
        // fold goes to out[g * outputs + o] for a second pass to combine.
        int64_t parts = 1;
        // Output groups per workgroup at most (a power of two up to 64);
        // the rest of its 256 lanes are strands along the axis.
        int max_cols = 64;
        // Max over the whole axis only: the reduction as the reference
        // states it (`exact_producer` over `exact_shape`, reduced along
        // `exact_axis`; for a second pass, the first pass's), evaluated in
        // the reference's order for outputs whose order-free result may
        // differ from it.  Null for a first pass of a split axis.
        const kexpr* exact_expr = nullptr;
        int exact_producer = -1;
        std::vector<int64_t> exact_shape;
        size_t exact_axis = 0;
    };

    kernel_code emit_column_reduce(const column_reduce_request& request);
    // Softmax statistics along a non-last axis in one read of the producer
    // (emit_reduce.cpp): per output column the max M and S = sum exp(f - M).
    // partial_slot < 0: the pass over `request.producer` (with
    // request.parts > 1: [3][parts][outputs] partial triples to `out`, else
    // M and S as [2][outputs]); partial_slot >= 0: the combination of such
    // partials (request.shape = {parts, outputs}) into [2][outputs].
    kernel_code emit_column_softmax(const column_reduce_request& request, int partial_slot);
    // How many chunks to split the reduced axis into (1: no split): about
    // four workgroups per compute unit, chunks of at least 32, and only for
    // reductions of at least 2^20 values over an axis of at least 256.
    int64_t column_reduce_parts(const column_reduce_request& request, int compute_units);

    // C = epilogue(A @ B) with A [M,K], B [K,N] given by element strides;
    // batched: C[b] = epilogue(A[b] @ B[b]) for b < batch.
    struct gemm_operand {
        int slot = -1;
        int64_t offset = 0;
        int64_t stride_row = 0;   // A: per m, B: per k
        int64_t stride_col = 0;   // A: per k, B: per n
        int64_t stride_batch = 0; // per batch entry (0: shared)
    };
    struct gemm_request {
        const kexpr* expr = nullptr;
        bool batched = false;     // epilogue over (b, m, n), output [batch, m, n]
        int64_t batch = 1;
        int64_t m = 0, n = 0, k = 0;
        gemm_operand a, b;
        int epilogue = -1;        // kexpr over (m, n) or (b, m, n); row_value 0 = acc
        int n_slots = 0;
        index_width width;
        int compute_units = 256;
        // > 1: the MFMA kernel computes K in this many chunks, each
        // workgroup one chunk of one tile, writing partial products to its
        // `out` as [chunks, batch, m, n] for emit_gemm_combine.
        int64_t k_chunks = 1;
    };

    kernel_code emit_gemm(const gemm_request& request);
    // How many chunks of K the MFMA kernel should split a product into (1:
    // none): when its tiles cannot fill the machine and K is long.
    int64_t gemm_k_chunks(const gemm_request& request);
    // Sums `chunks` partial products [chunks, batch, m, n] from slot
    // `partial_slot` per output and applies the epilogue.
    kernel_code emit_gemm_combine(const gemm_request& request, int64_t chunks, int partial_slot);

    // Products with one short side (emit_gemm_skinny.cpp).  A few rows
    // (m <= 16, n >= 256): `gemm_few_rows_partials` floats of partial
    // products over `gemm_few_rows_chunks` chunks of K (0 partials: one
    // chunk, the first kernel writes the result), then emit_gemm_combine.
    bool gemm_few_rows(const gemm_request& request);
    int64_t gemm_few_rows_partials(const gemm_request& request);
    int64_t gemm_few_rows_chunks(const gemm_request& request);
    kernel_code emit_gemm_few_rows(const gemm_request& request);
    // A few columns (n <= 4 over 64 rows or more, n <= 8 over 2048 rows or
    // more): one wave per 1, 2 or 4 output rows.
    bool gemm_few_cols(const gemm_request& request);
    kernel_code emit_gemm_few_cols(const gemm_request& request);
    // 7 to 32 columns over 128 rows or more (A rows contiguous along K):
    // a workgroup of four waves per 32 rows and a chunk of K on 16x16x4
    // MFMA blocks (or, for up to 16 columns over enough rows, one workgroup
    // per 16 rows over all of K), the chunks' partial products summed by
    // emit_gemm_combine.
    bool gemm_narrow(const gemm_request& request);
    int64_t gemm_narrow_chunks(const gemm_request& request);
    kernel_code emit_gemm_narrow(const gemm_request& request);
    // 1 to 32 rows over 256 columns or more (B rows contiguous along N; up
    // to 64 where the workgroups fill every compute unit): a workgroup of
    // four waves per 64 columns and a chunk of K on 16x16x4 MFMA blocks, the
    // chunks' partial products summed by emit_gemm_combine.
    bool gemm_wide(const gemm_request& request);
    int64_t gemm_wide_chunks(const gemm_request& request);
    kernel_code emit_gemm_wide(const gemm_request& request);

    // A short K (8 to 64, a multiple of 8) over 256 columns or more, A's
    // rows contiguous along K and B's rows along N or its columns along K
    // (B stored transposed), with two workgroups per
    // compute unit (emit_gemm_band.cpp): one workgroup per band of 128 rows
    // and run of at least two column tiles, its A held in registers.
    bool gemm_band(const gemm_request& request);
    kernel_code emit_gemm_band(const gemm_request& request);

} // namespace porch::cg
