// Matmuls with one short side, bound by reading the long operand once.
//
// The one-output-per-lane K loop (gemm.scalar) gives a vector-matrix
// product [1, 4096] @ [4096, 4096] 16 workgroups and 182 us; the MFMA tiles
// of 128 x 128 spend most of their work on padding when one side is a few
// rows or columns.  Two forms instead:
//
//   gemm.rows     few rows (m <= 16, n >= 256): one wave per 256 columns
//                 of B and a chunk of K, each lane holding m x 4
//                 accumulators for its four columns, A's values read as
//                 wave-uniform scalars; the chunks' partial products go to a
//                 temporary [chunks, batch, m, n] that gemm.combine sums
//                 per output, applying the epilogue.  With one chunk
//                 the first kernel applies the epilogue itself.
//   gemm.cols     few columns (n <= 4 over 64 rows or more, n <= 8 over 2048
//                 or more): one wave per 1, 2 or 4 output rows (which share
//                 each load of B), lanes along K reading A with 128-bit
//                 loads, n accumulators per row and lane and a butterfly
//                 per output.
//
// Sums run in other orders than the reference's sequential K loop, within
// the matmul's tolerance (an accumulation-bound per element).

#include "emit_gemm.hpp"

#include <algorithm>
#include <stdexcept>

namespace porch::cg {
    namespace {

        // Up to 16 rows: from 24 on, the MFMA kernel split over K is faster
        // (measured at K, N in {1024, 4096}: 43-44 against 47-57 us at 24
        // and 32 rows of 4096 x 4096, 17-20 against 28-40 us at 1024).
        constexpr int64_t max_rows = 16;
        constexpr int64_t max_cols = 4;
        constexpr int64_t max_cols_many_rows = 8;
        constexpr int64_t block_cols = 256; // columns per wave in gemm.rows

        bool big_enough(const gemm_request& r) { return r.batch * r.m * r.n * r.k >= (int64_t{1} << 18); }

        bool b_vector(const gemm_request& r) {
            return r.b.stride_col == 1 && r.n % 4 == 0 && r.b.offset % 4 == 0 && r.b.stride_row % 4 == 0 &&
                   r.b.stride_batch % 4 == 0;
        }

        bool a_vector(const gemm_request& r) {
            return r.a.stride_col == 1 && r.k % 4 == 0 && r.a.offset % 4 == 0 && r.a.stride_row % 4 == 0 &&
                   r.a.stride_batch % 4 == 0;
        }

        struct rows_shape {
            int64_t blocks = 0; // 256-column blocks
            int64_t chunks = 0; // K chunks
            int64_t chunk = 0;  // rows of K per chunk
        };

        rows_shape rows_plan(const gemm_request& r) {
            rows_shape sh;
            if (r.m > max_rows || r.n < block_cols || !big_enough(r)) return sh;
            sh.blocks = (r.n + block_cols - 1) / block_cols;
            // About eight waves per compute unit in all, and a chunk long
            // enough that the partials (m x 256 floats per wave) stay below
            // the B rows it reads (chunk x 256 floats).  (A chunk of at
            // least 8 m rows, fewer waves, was 16-30% slower at 16 rows.)
            const int64_t target = std::max<int64_t>(1, 8 * std::max(r.compute_units, 8) / (r.batch * sh.blocks));
            int64_t chunk = std::max<int64_t>(std::max<int64_t>(64, 2 * r.m), (r.k + target - 1) / target);
            chunk = std::min(chunk, r.k);
            sh.chunks = (r.k + chunk - 1) / chunk;
            sh.chunk = chunk;
            return sh;
        }

        std::vector<std::string> names_of(const gemm_request& r) {
            return r.batched ? std::vector<std::string>{"qb", "q0", "q1"} : std::vector<std::string>{"q0", "q1"};
        }

        // The epilogue of output (qb, q0, q1) with the product in `acc`,
        // stored to out[o].
        std::string epilogue_store(const gemm_request& r, const std::string& acc, const std::string& o,
                                   const std::string& indent) {
            std::string body;
            emitter em(*r.expr, body, 1);
            em.indent = indent;
            em.declare_roots({r.epilogue});
            epilogue_emitter(em, r, names_of(r), acc);
            const std::string v = em.emit(r.epilogue)[0];
            return body + indent + "out[" + o + "] = " + v + ";\n";
        }

    } // namespace

    bool gemm_few_rows(const gemm_request& r) { return rows_plan(r).blocks > 0; }

    int64_t gemm_few_rows_partials(const gemm_request& r) {
        const rows_shape sh = rows_plan(r);
        return sh.chunks > 1 ? sh.chunks * r.batch * r.m * r.n : 0;
    }

    kernel_code emit_gemm_few_rows(const gemm_request& r) {
        const rows_shape sh = rows_plan(r);
        if (sh.blocks == 0) throw std::logic_error("emit_gemm_few_rows: not a few-row product");
        const bool final = sh.chunks == 1;
        const bool vec = b_vector(r);
        const char* T = r.width.type();
        const std::string batch = r.batched ? "qb" : "";
        const std::string M = std::to_string(r.m);
        const std::string N = std::to_string(r.n);

        kernel_code kc;
        kc.kind = "gemm.rows";
        kc.name = "porch_gemm";
        kc.n_slots = r.n_slots;
        kc.block = 64;
        kc.grid_x = static_cast<unsigned>(r.batch * sh.blocks * sh.chunks);

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(64) porch_gemm(" + kernel_params(r.n_slots) + ") {\n";
        s += "    const int lane = threadIdx.x;\n";
        s += "    const idx_t ks = (idx_t)blockIdx.x % " + std::to_string(sh.chunks) + ";\n";
        s += "    const idx_t blk = ((idx_t)blockIdx.x / " + std::to_string(sh.chunks) + ") % " +
             std::to_string(sh.blocks) + ";\n";
        if (r.batched) s += "    const idx_t qb = (idx_t)blockIdx.x / " + std::to_string(sh.chunks * sh.blocks) + ";\n";
        s += "    const idx_t k0 = ks * " + std::to_string(sh.chunk) + ";\n";
        s += "    const idx_t k1 = k0 + " + std::to_string(sh.chunk) + " < " + std::to_string(r.k) + " ? k0 + " +
             std::to_string(sh.chunk) + " : (idx_t)" + std::to_string(r.k) + ";\n";
        s += "    float acc[" + M + "][4];\n";
        s += "    #pragma unroll\n    for (int i = 0; i < " + M + "; ++i)\n";
        s += "        #pragma unroll\n        for (int e = 0; e < 4; ++e) acc[i][e] = 0.0f;\n";
        // column of value e of this lane
        const std::string col0 = vec ? "blk * 256 + lane * 4" : "blk * 256 + lane";
        const std::string col_step = vec ? "1" : "64";
        s += "    const idx_t c0 = " + col0 + ";\n";
        // B rows in flight per lane: 8 for up to 8 rows of A (measured
        // [1 and 4, 4096] @ [4096, 4096]: 15.5 -> 13.2 and 18.2 -> 15.5 us
        // against 4; 16 gave no more, and at 16 rows 8 gave no gain).
        s += std::string("    #pragma unroll ") + (r.m <= 8 ? "8" : "4") + "\n    for (idx_t kk = k0; kk < k1; ++kk) {\n";
        s += "        float bv[4];\n";
        if (vec) {
            s += "        if (c0 < " + N + ") {\n";
            s += "            const porch_v4f w = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(a" +
                 std::to_string(r.b.slot) + " + " + operand_index(r.b, "kk", "c0", batch) + "));\n";
            s += "            bv[0] = w.x; bv[1] = w.y; bv[2] = w.z; bv[3] = w.w;\n";
            s += "        }\n        else {\n            bv[0] = bv[1] = bv[2] = bv[3] = 0.0f;\n        }\n";
        }
        else {
            s += "        #pragma unroll\n        for (int e = 0; e < 4; ++e) {\n";
            s += "            const idx_t c = c0 + e * " + col_step + ";\n";
            s += "            bv[e] = c < " + N + " ? a" + std::to_string(r.b.slot) + "[" +
                 operand_index(r.b, "kk", "c", batch) + "] : 0.0f;\n";
            s += "        }\n";
        }
        s += "        #pragma unroll\n        for (int i = 0; i < " + M + "; ++i) {\n";
        s += "            const float av = a" + std::to_string(r.a.slot) + "[" + operand_index(r.a, "i", "kk", batch) +
             "];\n";
        s += "            #pragma unroll\n            for (int e = 0; e < 4; ++e) acc[i][e] = __builtin_fmaf(av, bv[e], acc[i][e]);\n";
        s += "        }\n    }\n";
        s += "    #pragma unroll\n    for (int i = 0; i < " + M + "; ++i) {\n";
        s += "        #pragma unroll\n        for (int e = 0; e < 4; ++e) {\n";
        s += "            const idx_t q1 = c0 + e * " + col_step + ";\n";
        s += "            if (q1 < " + N + ") {\n";
        const std::string o = std::string(r.batched ? "(qb * " + M + " + i)" : "(idx_t)i") + " * " + N + " + q1";
        if (final) {
            s += "                const idx_t q0 = i;\n";
            s += "                const float acc_v = acc[i][e];\n";
            s += epilogue_store(r, "acc_v", o, "                ");
        }
        else {
            s += "                out[ks * " + std::to_string(r.batch * r.m * r.n) + " + " + o + "] = acc[i][e];\n";
        }
        s += "            }\n        }\n    }\n}\n";
        return kc;
    }

    int64_t gemm_few_rows_chunks(const gemm_request& r) { return rows_plan(r).chunks; }

    kernel_code emit_gemm_combine(const gemm_request& r, int64_t chunks, int partial_slot) {
        if (chunks < 2) throw std::logic_error("emit_gemm_combine: one chunk");
        const char* T = r.width.type();
        const int64_t outputs = r.batch * r.m * r.n;
        const std::string O = std::to_string(outputs);

        kernel_code kc;
        kc.kind = "gemm.combine";
        kc.name = "porch_gemm";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>((outputs + 255) / 256);

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(256) porch_gemm(" + kernel_params(r.n_slots) + ") {\n";
        s += "    const idx_t o = (idx_t)blockIdx.x * 256 + threadIdx.x;\n";
        s += "    if (o >= " + O + ") return;\n";
        s += "    const float* __restrict__ xp = a" + std::to_string(partial_slot) + " + o;\n";
        s += "    float acc = 0.0f;\n";
        s += "    #pragma unroll 8\n";
        s += "    for (int c = 0; c < " + std::to_string(chunks) + "; ++c) acc += xp[(idx_t)c * " + O + "];\n";
        if (r.batched) s += "    const idx_t qb = o / " + std::to_string(r.m * r.n) + ";\n";
        s += "    const idx_t q0 = (o / " + std::to_string(r.n) + ") % " + std::to_string(r.m) + ";\n";
        s += "    const idx_t q1 = o % " + std::to_string(r.n) + ";\n";
        s += epilogue_store(r, "acc", "o", "    ");
        s += "}\n";
        return kc;
    }

    bool gemm_few_cols(const gemm_request& r) {
        // 5 to 8 columns only over many rows (measured at 4096 rows: 23 us
        // at 8 columns against 31 us for the split MFMA kernel)
        return ((r.n <= max_cols && r.m >= 64) || (r.n <= max_cols_many_rows && r.batch * r.m >= 2048)) &&
               big_enough(r);
    }

    kernel_code emit_gemm_few_cols(const gemm_request& r) {
        if (!gemm_few_cols(r)) throw std::logic_error("emit_gemm_few_cols: not a few-column product");
        const bool vec = a_vector(r);
        const char* T = r.width.type();
        const std::string batch = r.batched ? "qb" : "";
        const std::string N = std::to_string(r.n);
        const std::string M = std::to_string(r.m);
        // Rows per wave: B is read once per wave, so the wave's rows share
        // each load of it (with one row per wave, every wave reread all of
        // B from the L2: n x 64 MB over [4096, 4096] @ [4096, n]), against
        // fewer waves to hide the loads' latency.  Measured on
        // [4096, 4096] @ [4096, n] (1, 2, 4 or 8 rows a wave): n = 1, 2
        // fastest with 1 (12.8, 13.2 us), n = 4 with 2 (15.3 against 19.6
        // us with 1), n = 8 with 4 (23.2 against 33.8 with 2).
        const int64_t R = r.n <= 2 ? 1 : (r.n <= 4 ? 2 : 4);
        const std::string RS = std::to_string(R);
        const int64_t row_groups = (r.m + R - 1) / R; // per batch entry
        const int64_t groups = r.batch * row_groups;

        kernel_code kc;
        kc.kind = "gemm.cols";
        kc.name = "porch_gemm";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>(std::min<int64_t>((groups + 3) / 4, 16 * std::max(r.compute_units, 8)));

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(256) porch_gemm(" + kernel_params(r.n_slots) + ") {\n";
        s += "    const int lane = threadIdx.x & 63;\n";
        s += "    for (idx_t grp = (idx_t)blockIdx.x * 4 + (threadIdx.x >> 6); grp < " + std::to_string(groups) +
             "; grp += (idx_t)gridDim.x * 4) {\n";
        s += "        const idx_t qb = grp / " + std::to_string(row_groups) + ";\n";
        if (!r.batched) s += "        (void)qb;\n";
        s += "        const idx_t q00 = (grp % " + std::to_string(row_groups) + ") * " + RS + ";\n";
        s += "        float acc[" + RS + "][" + N + "];\n";
        s += "        #pragma unroll\n        for (int r = 0; r < " + RS + "; ++r)\n";
        s += "            #pragma unroll\n            for (int j = 0; j < " + N + "; ++j) acc[r][j] = 0.0f;\n";
        const std::string bslot = "a" + std::to_string(r.b.slot);
        if (vec) {
            // one column: four A loads in flight per lane (12.9 -> 11.6 us
            // on [4096, 4096] @ [4096, 1]; no gain from 2 columns on)
            if (r.n == 1) s += "        #pragma unroll 4\n";
            s += "        for (idx_t kq = lane * 4; kq < " + std::to_string(r.k) + "; kq += 256) {\n";
            s += "            float av[" + RS + "][4];\n";
            s += "            #pragma unroll\n            for (int r = 0; r < " + RS + "; ++r) {\n";
            s += "                const idx_t q0 = q00 + r;\n";
            s += "                porch_v4f w = {0.0f, 0.0f, 0.0f, 0.0f};\n";
            s += "                if (q0 < " + M + ") w = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(a" +
                 std::to_string(r.a.slot) + " + " + operand_index(r.a, "q0", "kq", batch) + "));\n";
            s += "                av[r][0] = w.x; av[r][1] = w.y; av[r][2] = w.z; av[r][3] = w.w;\n";
            s += "            }\n";
            s += "            #pragma unroll\n            for (int e = 0; e < 4; ++e)\n";
            s += "                #pragma unroll\n                for (int j = 0; j < " + N + "; ++j) {\n";
            s += "                    const float b = " + bslot + "[" + operand_index(r.b, "kq + e", "j", batch) + "];\n";
            s += "                    #pragma unroll\n                    for (int r = 0; r < " + RS + "; ++r)\n";
            s += "                        acc[r][j] = __builtin_fmaf(av[r][e], b, acc[r][j]);\n";
            s += "                }\n";
            s += "        }\n";
        }
        else {
            s += "        for (idx_t kk = lane; kk < " + std::to_string(r.k) + "; kk += 64) {\n";
            s += "            #pragma unroll\n            for (int j = 0; j < " + N + "; ++j) {\n";
            s += "                const float b = " + bslot + "[" + operand_index(r.b, "kk", "j", batch) + "];\n";
            s += "                #pragma unroll\n                for (int r = 0; r < " + RS + "; ++r) {\n";
            s += "                    const idx_t q0 = q00 + r;\n";
            s += "                    const float av = q0 < " + M + " ? a" + std::to_string(r.a.slot) + "[" +
                 operand_index(r.a, "q0", "kk", batch) + "] : 0.0f;\n";
            s += "                    acc[r][j] = __builtin_fmaf(av, b, acc[r][j]);\n";
            s += "                }\n";
            s += "            }\n";
            s += "        }\n";
        }
        s += "        #pragma unroll\n        for (int r = 0; r < " + RS + "; ++r)\n";
        s += "            #pragma unroll\n            for (int j = 0; j < " + N + "; ++j)\n";
        s += "                for (int d = 32; d >= 1; d >>= 1) acc[r][j] += __shfl_xor(acc[r][j], d, 64);\n";
        s += "        if (lane == 0) {\n";
        s += "            #pragma unroll\n            for (int r = 0; r < " + RS + "; ++r) {\n";
        s += "                const idx_t q0 = q00 + r;\n";
        s += "                if (q0 < " + M + ") {\n";
        s += "                    const idx_t row = qb * " + M + " + q0;\n";
        s += "                    #pragma unroll\n                    for (int j = 0; j < " + N + "; ++j) {\n";
        s += "                        const idx_t q1 = j;\n";
        s += "                        const float acc_v = acc[r][j];\n";
        s += epilogue_store(r, "acc_v", "row * " + N + " + q1", "                        ");
        s += "                    }\n";
        s += "                }\n";
        s += "            }\n        }\n    }\n}\n";
        return kc;
    }

} // namespace porch::cg
