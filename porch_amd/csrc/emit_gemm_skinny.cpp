// Matmuls with one short side, bound by reading the long operand once.
//
// The one-output-per-lane K loop (gemm.scalar) gives a vector-matrix
// product [1, 4096] @ [4096, 4096] 16 workgroups and 182 us; the MFMA tiles
// of 128 x 128 spend most of their work on padding when one side is a few
// rows or columns.  Instead:
//
//   gemm.rows     few rows (m <= 16, n >= 256) where gemm.wide cannot read
//                 B's rows as float4s: one wave per 256 columns
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
//   gemm.narrow   7 to 32 columns over 128 rows or more: a workgroup of
//                 four waves per 32 rows and a chunk of K, the waves taking
//                 its groups of 16 values in turn; v_mfma_f32_16x16x4f32
//                 blocks fed straight from 128-bit loads of A (lane l reads
//                 row l % 16, k in 4 (l / 16) .. +3, one MFMA per k of the
//                 four), B read per lane from the L2; the waves' sums added
//                 through LDS, the chunks' partial products summed by
//                 gemm.combine.
//   gemm.narrow_rows  7 to 16 columns over 4096 rows or more: a workgroup
//                 per 16 rows over all of K, the rows' values staged
//                 through LDS into the MFMA layout, no partial products
//                 (its constants below say more).
//   gemm.wide     the same blocks the other way round, few rows (up to 64)
//                 over many columns: a workgroup of four waves per 64
//                 columns and a chunk of K, the waves taking its groups of
//                 16 values in turn; lane l reads B's rows at
//                 columns 4 (l % 16) .. + 3 with 128-bit loads, so that MFMA
//                 e covers the 16 columns 4 (l % 16) + e, and A's row l % 16
//                 from the L2; the waves' sums are added through LDS.  Where
//                 B is stored transposed (x @ W^T with a weight W [n, K]),
//                 lane l reads column 16 e + l % 16 at its four k with one
//                 128-bit load (a wave taking 32 values of K a group, two
//                 such loads a column), so that MFMA e covers 16 adjacent
//                 columns
//                 (x [32, 4096] @ W^T: 20.1 + 4.0 us, against 42.5 + 4.8
//                 for the split MFMA kernel that took it before; x @ W
//                 with W stored [K, n]: 15.0 + 4.0).  gemm.narrow_rows reads
//                 such a B's four values of a group as one 128-bit load too
//                 ([4096, 4096] @ w^T, w [16, 4096]: 19.3 against 38.6 us).
//
// Sums run in other orders than the reference's sequential K loop, within
// the matmul's tolerance (an accumulation-bound per element).

#include "emit_gemm.hpp"

#include <algorithm>
#include <functional>
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
        // gemm.cols is faster up to 6 columns (17.6 and 18.2 against 19.4
        // and 19.2 us at 5 and 6 over 4096 rows; at 8 20.4 against 23.1)
        constexpr int64_t narrow_min_cols = 7;
        constexpr int64_t narrow_max_cols = 32;
        // rows of A over all batch entries (at 128 rows of 4096 x 4096 with
        // 32 columns: 8.7 us against 12.6 for the split MFMA kernel)
        constexpr int64_t narrow_min_rows = 128;
        // gemm.wide from 1 row (kernel + combine, against gemm.rows: 17.0
        // against 18.5 us at 1 row of [4096, 4096], 17.2 against 19.6 at 4,
        // 12.3 against 19.8 at [4, 1024] @ [1024, 16384]) to 64 (27.3 us;
        // the split MFMA kernel took 47.6, and the MFMAs, 4 per row block
        // and 128-bit load of B, take over from there); gemm.rows keeps the
        // products whose B rows are not read as float4s
        constexpr int64_t wide_min_rows = 1;
        constexpr int64_t wide_max_rows = 64;
        // gemm.wide and gemm.narrow: four waves a workgroup share one tile
        // and one chunk of K, taking its groups of 16 values in turn
        constexpr int64_t group_waves = 4;
        constexpr int64_t group_size = 16;
        constexpr int group_depth = 2; // groups in flight per wave

        bool big_enough(const gemm_request& r) { return r.batch * r.m * r.n * r.k >= (int64_t{1} << 18); }

        // B's columns contiguous along K in aligned quads (B stored
        // transposed, as in x @ w^T with a weight w [n, K])
        bool b_column_runs(const gemm_request& r) {
            return r.b.stride_row == 1 && r.b.stride_col % 4 == 0 && r.b.offset % 4 == 0 &&
                   r.b.stride_batch % 4 == 0 && r.k % 4 == 0;
        }

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

        struct narrow_shape {
            int64_t rb = 0;     // 16-row MFMA blocks per wave
            int64_t nb = 0;     // 16-column MFMA blocks
            int64_t tiles = 0;  // row tiles of 16 rb rows per batch entry
            int64_t chunks = 0; // K chunks
            int64_t chunk = 0;  // K per chunk, a multiple of 16
        };

        // gemm.narrow_rows: 7 to 16 columns, one workgroup of 8 (or 4)
        // waves per 16 rows of A over all of K (no partial products, no
        // combine).  Each wave takes K / 8 values in rounds of 256 (64
        // lanes x a float4): the 16 rows' values are read as one 1 KB run
        // per row, written to the wave's own area of LDS and read back in
        // the MFMA layout; the next round's rows are loaded during this
        // round.  At least one workgroup per compute unit, and K long
        // enough for a full round per wave (measured on [4096, 4096] @
        // [4096, 16]: 16.0 us, against 16.7 + 4.5 us for gemm.narrow and its
        // combine).  The rounds are written out: past two rounds a wave of
        // eight no longer fits the register budget of two waves per SIMD
        // (spills: 42.6 us at [4096, 8192] @ [8192, 16]), so longer K takes
        // four waves a workgroup (28.3 us there; at K = 4096 four waves are
        // 3-7 % slower than eight), up to 16 rounds a wave.
        constexpr int64_t rows_round = 256;
        constexpr int64_t rows_stride = rows_round + 4; // LDS row, floats
        constexpr int64_t rows_max_rounds = 16;

        int64_t rows_waves(const gemm_request& r) { return r.k <= 8 * 2 * rows_round ? 8 : 4; }

        bool narrow_rows(const gemm_request& r) {
            return r.n >= narrow_min_cols && r.n <= 16 && a_vector(r) && big_enough(r) &&
                   r.batch * ((r.m + 15) / 16) >= std::max(r.compute_units, 8) && r.k >= 8 * rows_round &&
                   r.k <= 4 * rows_max_rounds * rows_round;
        }

        narrow_shape narrow_plan(const gemm_request& r) {
            narrow_shape sh;
            if (r.n < narrow_min_cols || r.n > narrow_max_cols || r.batch * r.m < narrow_min_rows || !a_vector(r) ||
                !big_enough(r))
                return sh;
            if (narrow_rows(r)) {
                sh.rb = 1;
                sh.nb = 1;
                sh.tiles = (r.m + 15) / 16;
                sh.chunks = 1;
                sh.chunk = r.k;
                return sh;
            }
            sh.rb = 2;
            sh.nb = (r.n + 15) / 16;
            sh.tiles = (r.m + 16 * sh.rb - 1) / (16 * sh.rb);
            // One workgroup (four waves) per 32-row tile and chunk of K, about
            // one workgroup per compute unit; the partial products (chunks x
            // m x n) at most 1/4 of A (m x K) and at most 32 chunks (64
            // chunks made the combine dear, 4.9 us at [512, 4096] @ [4096,
            // 16]); chunks a multiple of the waves' 64 values of K.
            const int64_t cus = std::max(r.compute_units, 8);
            const int64_t batch_k = group_waves * group_size;
            int64_t chunks = (cus + r.batch * sh.tiles - 1) / (r.batch * sh.tiles);
            chunks = std::min(chunks, std::max<int64_t>(1, r.k / (4 * r.n)));
            chunks = std::min(chunks, std::max<int64_t>(1, r.k / batch_k));
            chunks = std::min<int64_t>(chunks, 32);
            int64_t chunk = (r.k + chunks - 1) / chunks;
            chunk = (chunk + batch_k - 1) / batch_k * batch_k;
            sh.chunks = (r.k + chunk - 1) / chunk;
            sh.chunk = chunk;
            return sh;
        }

        struct wide_shape {
            int64_t rb = 0;     // 16-row MFMA blocks
            int64_t tiles = 0;  // 64-column tiles per batch entry
            int64_t chunks = 0; // K chunks
            int64_t chunk = 0;  // K per chunk, a multiple of 64 (a group per wave)
        };

        // Values of K a wave of gemm.wide takes per group: 16, or 32 where
        // B is stored transposed (a lane then reads 128 B of each of its
        // columns in two loads; x [32, 4096] @ W^T: 18.7 against 23.3 us
        // with 16 in a standalone copy timed back to back, 20.1 against
        // 21.1 us as emitted, under the kernel tracer)
        int64_t wide_group(const gemm_request& r) { return b_vector(r) ? group_size : 2 * group_size; }

        wide_shape wide_plan(const gemm_request& r) {
            wide_shape sh;
            // B's rows read along N, or its columns along K where B is
            // stored transposed (then in whole groups of 32 values of K)
            const bool b_ok = b_vector(r) || (b_column_runs(r) && r.k % (2 * group_size) == 0);
            if (r.m < wide_min_rows || r.m > wide_max_rows || r.n < 256 || !b_ok || !big_enough(r)) return sh;
            sh.rb = (r.m + 15) / 16;
            sh.tiles = (r.n + 63) / 64;
            // About one workgroup (four waves) per compute unit, partials
            // (chunks x m x n) at most 1/4 of B (K x n), at most 32 chunks.
            const int64_t cus = std::max(r.compute_units, 8);
            const int64_t batch_k = group_waves * wide_group(r);
            int64_t chunks = (cus + r.batch * sh.tiles - 1) / (r.batch * sh.tiles);
            chunks = std::min(chunks, std::max<int64_t>(1, r.k / (4 * r.m)));
            chunks = std::min(chunks, std::max<int64_t>(1, r.k / batch_k));
            chunks = std::min<int64_t>(chunks, 32);
            int64_t chunk = (r.k + chunks - 1) / chunks;
            chunk = (chunk + batch_k - 1) / batch_k * batch_k;
            sh.chunks = (r.k + chunk - 1) / chunk;
            sh.chunk = chunk;
            // Over 32 rows a wave's 3 or 4 row blocks of MFMAs are long: only
            // with a workgroup on every CU ([48, 2048] @ [2048, 2048] in
            // 320 single waves: 28.9 us against 19.9 for the split MFMA
            // kernel).
            if (r.m > 32 && r.batch * sh.tiles * sh.chunks < cus) return wide_shape{};
            return sh;
        }

        // Emitted code, at indent `ind`, for operand register set `set` of
        // one group ...
        using group_text = std::function<std::string(const std::string& set, const std::string& ind)>;
        // ... loading the group of 16 values of K from `kq` into it.
        using group_load_text =
            std::function<std::string(const std::string& set, const std::string& kq, const std::string& ind)>;

        // The K loop of gemm.wide and gemm.narrow over a workgroup's chunk
        // [k0, k1) (names k0, k1 and the uniform wave index w in scope): the
        // chunk's full groups go to the waves in turn (wave w: groups w,
        // w + 4, ...), so the four waves read 64 adjacent values of K at a
        // time.  Each wave keeps two groups' loads in flight: the next
        // group's loads are issued before this group's MFMAs.  Where every
        // chunk is whole (`per_wave` groups for every wave, > 0) the loop is
        // written out: rolled, the compiler's register assignment copied the
        // accumulators at every turn.  Otherwise the loop takes the groups in
        // pairs with no exit in between (with a break after the first half
        // the compiler sank the second set's loads below the first set's
        // MFMAs), the last prefetch of a wave with an even count reloading
        // its own last group (in bounds, no branch around the loads), and
        // declares `full`, the chunk's count of full groups, for a partial
        // last group that the caller handles.  (Measured for gemm.wide on
        // [32, 4096] @ [4096, 4096], 4 chunks of 1024: 14.4 us, against 22.7
        // us for one wave per tile and chunk with 16 chunks; eight or sixteen
        // waves a workgroup 17.5 and 21.7 us, three groups in flight 15.6.)
        std::string group_loop(int64_t per_wave, const group_text& declare, const group_load_text& loads,
                               const group_text& mfmas, int64_t width = group_size) {
            const std::string GW = std::to_string(width);
            std::string s;
            if (per_wave > 0 && per_wave <= 32) {
                auto set_of = [](int64_t t) { return "S" + std::to_string(t % group_depth); };
                auto load_group = [&](int64_t t) {
                    return "    {\n        const idx_t kq = k0 + " + GW + " * w + " +
                           std::to_string(t * group_waves * width) + ";\n" + loads(set_of(t), "kq", "        ") +
                           "    }\n";
                };
                for (int d = 0; d < group_depth; ++d) s += declare(set_of(d), "    ");
                for (int64_t t = 0; t + 1 < group_depth && t < per_wave; ++t) s += load_group(t);
                for (int64_t t = 0; t < per_wave; ++t) {
                    if (t + group_depth - 1 < per_wave) s += load_group(t + group_depth - 1);
                    s += "    __builtin_amdgcn_sched_barrier(0);\n" + mfmas(set_of(t), "    ") +
                         "    __builtin_amdgcn_sched_barrier(0);\n";
                }
                return s;
            }
            s += declare("P", "    ") + declare("Q", "    ");
            s += "    const idx_t full = (k1 - k0) / " + GW + ";\n";
            s += "    const idx_t nf = full > w ? (full - w + 3) / 4 : 0;\n";
            s += "    if (nf > 0) {\n        const idx_t kq = k0 + " + GW + " * w;\n" + loads("P", "kq", "        ") + "    }\n";
            s += "    idx_t t = 0;\n";
            s += "    for (; t + 2 <= nf; t += 2) {\n";
            s += "        {\n            const idx_t kq = k0 + " + GW + " * (w + 4 * (t + 1));\n" +
                 loads("Q", "kq", "            ") + "        }\n";
            s += "        __builtin_amdgcn_sched_barrier(0);\n" + mfmas("P", "        ") +
                 "        __builtin_amdgcn_sched_barrier(0);\n";
            s += "        {\n            const idx_t kq = k0 + " + GW + " * (w + 4 * (t + 2 < nf ? t + 2 : t + 1));\n" +
                 loads("P", "kq", "            ") + "        }\n";
            s += "        __builtin_amdgcn_sched_barrier(0);\n" + mfmas("Q", "        ") +
                 "        __builtin_amdgcn_sched_barrier(0);\n";
            s += "    }\n";
            s += "    if (t < nf) {\n" + mfmas("P", "        ") + "    }\n";
            return s;
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
        // value e of this lane is column c0 + 64 e: B's rows are not read as
        // float4s here (gemm.wide takes the products where they can be)
        const std::string col_step = "64";
        s += "    const idx_t c0 = blk * 256 + lane;\n";
        // B rows in flight per lane: 8 for up to 8 rows of A (measured when
        // this kernel also read float4s of B, [1 and 4, 4096] @ [4096, 4096]:
        // 15.5 -> 13.2 and 18.2 -> 15.5 us against 4; 16 gave no more, and at
        // 16 rows 8 gave no gain).
        s += std::string("    #pragma unroll ") + (r.m <= 8 ? "8" : "4") + "\n    for (idx_t kk = k0; kk < k1; ++kk) {\n";
        s += "        float bv[4];\n";
        s += "        #pragma unroll\n        for (int e = 0; e < 4; ++e) {\n";
        s += "            const idx_t c = c0 + e * " + col_step + ";\n";
        s += "            bv[e] = c < " + N + " ? a" + std::to_string(r.b.slot) + "[" +
             operand_index(r.b, "kk", "c", batch) + "] : 0.0f;\n";
        s += "        }\n";
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
        // at 8 columns against 31 us for the split MFMA kernel); the
        // planner takes gemm.narrow first where A allows it
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

    bool gemm_narrow(const gemm_request& r) { return narrow_plan(r).rb > 0; }

    int64_t gemm_narrow_chunks(const gemm_request& r) { return narrow_plan(r).chunks; }

    namespace {

        kernel_code emit_gemm_narrow_rows(const gemm_request& r) {
            const char* T = r.width.type();
            const std::string batch = r.batched ? "qb" : "";
            const std::string M = std::to_string(r.m);
            const std::string N = std::to_string(r.n);
            const std::string K = std::to_string(r.k);
            const int64_t row_tiles = (r.m + 15) / 16;
            // K per wave: a multiple of 4, so a float4 never straddles a
            // wave's end
            const int64_t waves = rows_waves(r);
            const int64_t kw = (r.k + 4 * waves - 1) / (4 * waves) * 4;
            const int64_t rounds = (kw + rows_round - 1) / rows_round;
            const std::string KW = std::to_string(kw);
            const std::string RS = std::to_string(rows_stride);

            kernel_code kc;
            kc.kind = "gemm.narrow_rows";
            kc.name = "porch_gemm";
            kc.n_slots = r.n_slots;
            kc.block = static_cast<unsigned>(64 * waves);
            kc.grid_x = static_cast<unsigned>(r.batch * row_tiles);

            const std::string aslot = "a" + std::to_string(r.a.slot);
            const std::string bslot = "a" + std::to_string(r.b.slot);
            std::string& s = kc.source;
            s = kernel_prologue(r.n_slots, T);
            s += "extern \"C\" __global__ void __launch_bounds__(" + std::to_string(kc.block) + ") porch_gemm(" +
                 kernel_params(r.n_slots) + ") {\n";
            // each wave's own area: 16 rows of a round, rows padded by 16 bytes
            s += "    __shared__ __attribute__((aligned(16))) float stage[" + std::to_string(waves) + "][16 * " + RS +
                 "];\n";
            s += "    const int lane = threadIdx.x & 63;\n";
            s += "    const int li = lane & 15;\n    const int lg = lane >> 4;\n";
            s += "    const int w = threadIdx.x >> 6;\n";
            s += "    const idx_t tile = blockIdx.x;\n";
            s += "    const idx_t qb = tile / " + std::to_string(row_tiles) + ";\n";
            if (!r.batched) s += "    (void)qb;\n";
            s += "    const idx_t r0 = (tile % " + std::to_string(row_tiles) + ") * 16;\n";
            s += "    const idx_t kbeg = (idx_t)w * " + KW + ";\n";
            s += "    const idx_t kend = kbeg + " + KW + " < " + K + " ? kbeg + " + KW + " : (idx_t)" + K + ";\n";
            // Rows past m are read at m - 1 and columns past n at n - 1: they
            // feed only outputs that are not stored.  Values of K past the
            // wave's end are read at column 0 and zeroed in both operands
            // (zeroing one would turn an infinity in the other into NaN).
            s += "    const idx_t qc = li < " + N + " ? (idx_t)li : (idx_t)" + std::to_string(r.n - 1) + ";\n";
            s += "    porch_v4f acc = porch_v4f{0.0f, 0.0f, 0.0f, 0.0f};\n";
            s += "    float* const my = &stage[w][0];\n";
            s += "    porch_v4f x0[16], x1[16];\n";
            // The zeroing happens where a value is used (the LDS write,
            // the MFMA), not after its load: a select right after a load
            // made the compiler wait for each load before issuing the next.
            // (A round inside the wave's range, the same for all its lanes,
            // takes the loads without clamping: constant offsets from one
            // address.)
            auto load_rows = [&](const std::string& set, int64_t round) {
                std::string t;
                auto body = [&](bool clamp) {
                    std::string b;
                    b += "        const idx_t k = kbeg + " + std::to_string(round * rows_round) + " + 4 * lane;\n";
                    b += std::string("        const idx_t kr = ") + (clamp ? "k < kend ? k : (idx_t)0" : "k") + ";\n";
                    b += "        #pragma unroll\n        for (int rr = 0; rr < 16; ++rr) {\n";
                    b += "            const idx_t q0 = r0 + rr < " + M + " ? r0 + rr : (idx_t)" + std::to_string(r.m - 1) +
                         ";\n";
                    b += "            " + set + "[rr] = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" +
                         aslot + " + " + operand_index(r.a, "q0", "kr", batch) + "));\n";
                    b += "        }\n";
                    return b;
                };
                t += "    if (kbeg + " + std::to_string((round + 1) * rows_round) + " <= kend) {\n" + body(false) +
                     "    }\n    else {\n" + body(true) + "    }\n";
                return t;
            };
            // Every wave's range whole rounds (K = waves x a multiple of
            // 256): no clamps and no zeroing, and each later round's values
            // of B are loaded during the round before it, group q's right
            // after that round's MFMAs of group q have used the registers
            // (the loads' latency then overlaps the rest of the round:
            // 18.4-18.6 against 18.8-19.1 us at [4096, 4096] @ [4096, 16],
            // timed back to back; the same with the ragged rounds' clamps
            // and branches kept was slower, 19.7-19.8 us).
            const bool whole = kw * waves == r.k && kw % rows_round == 0;
            auto b_group = [&](int64_t n, const std::string& q, const std::string& ind) {
                std::string t;
                if (b_column_runs(r)) {
                    t += ind + "{\n";
                    t += ind + "    const porch_v4f bq = *reinterpret_cast<const porch_v4f*>(" + bslot + " + " +
                         operand_index(r.b, "(kbeg + " + std::to_string(n * rows_round) + " + " + q + " * 16 + lg * 4)", "qc",
                                       batch) + ");\n";
                    t += ind + "    #pragma unroll\n" + ind + "    for (int e = 0; e < 4; ++e) bv[" + q + "][e] = bq[e];\n";
                    t += ind + "}\n";
                    return t;
                }
                t += ind + "#pragma unroll\n" + ind + "for (int e = 0; e < 4; ++e)\n";
                t += ind + "    bv[" + q + "][e] = " + bslot + "[" +
                     operand_index(r.b, "(kbeg + " + std::to_string(n * rows_round) + " + " + q + " * 16 + lg * 4 + e)", "qc",
                                   batch) + "];\n";
                return t;
            };
            auto whole_rows = [&](const std::string& set, int64_t round) {
                std::string t;
                t += "    #pragma unroll\n    for (int rr = 0; rr < 16; ++rr) {\n";
                t += "        const idx_t q0 = r0 + rr < " + M + " ? r0 + rr : (idx_t)" + std::to_string(r.m - 1) + ";\n";
                t += "        " + set + "[rr] = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" + aslot + " + " +
                     operand_index(r.a, "q0", "(kbeg + " + std::to_string(round * rows_round) + " + 4 * lane)", batch) +
                     "));\n";
                t += "    }\n";
                return t;
            };
            if (whole) {
                s += "    float bv[16][4];\n";
                s += whole_rows("x0", 0);
                s += "    #pragma unroll\n    for (int q = 0; q < 16; ++q) {\n" + b_group(0, "q", "        ") + "    }\n";
                for (int64_t n = 0; n < rounds; ++n) {
                    const std::string cur = n % 2 == 0 ? "x0" : "x1";
                    const std::string nxt = n % 2 == 0 ? "x1" : "x0";
                    const bool more = n + 1 < rounds;
                    if (more) s += whole_rows(nxt, n + 1);
                    s += "    __builtin_amdgcn_sched_barrier(0);\n";
                    s += "    #pragma unroll\n    for (int rr = 0; rr < 16; ++rr)\n";
                    s += "        *reinterpret_cast<porch_v4f*>(my + rr * " + RS + " + 4 * lane) = " + cur + "[rr];\n";
                    // the wave's lanes read each other's values (see below)
                    s += "    __builtin_amdgcn_wave_barrier();\n";
                    s += "    __builtin_amdgcn_sched_barrier(0);\n";
                    s += "    #pragma unroll\n    for (int q = 0; q < 16; ++q) {\n";
                    s += "        const porch_v4f av = *reinterpret_cast<const porch_v4f*>(my + li * " + RS +
                         " + q * 16 + lg * 4);\n";
                    s += "        #pragma unroll\n        for (int e = 0; e < 4; ++e)\n";
                    s += "            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], bv[q][e], acc, 0, 0, 0);\n";
                    if (more) {
                        s += "        __builtin_amdgcn_sched_barrier(0);\n";
                        s += b_group(n + 1, "q", "        ");
                        s += "        __builtin_amdgcn_sched_barrier(0);\n";
                    }
                    s += "    }\n";
                    s += "    __builtin_amdgcn_wave_barrier();\n";
                    s += "    __builtin_amdgcn_sched_barrier(0);\n";
                }
            }
            else {
                s += load_rows("x0", 0);
                for (int64_t n = 0; n < rounds; ++n) {
                    const std::string cur = n % 2 == 0 ? "x0" : "x1";
                    const std::string nxt = n % 2 == 0 ? "x1" : "x0";
                    s += "    {\n";
                    // this round's values of B first: lane (li, lg) needs column
                    // li at k = base + 16 q + 4 lg + e for its 4 steps of group q.
                    // (Loads complete in issue order: B before the next round's
                    // rows, so waiting for B does not wait for them.)
                    s += "        float bv[16][4];\n";
                    s += "        const bool full = kbeg + " + std::to_string((n + 1) * rows_round) + " <= kend;\n";
                    auto b_loads = [&](bool clamp) {
                        std::string t;
                        if (b_column_runs(r)) {
                            // B stored transposed (w^T of a weight w [n, K]):
                            // the lane's four values of group q are one float4
                            // of column li (a quad past the wave's range reads
                            // k = 0 and is masked in the MFMAs)
                            t += "            #pragma unroll\n            for (int q = 0; q < 16; ++q) {\n";
                            t += "                const idx_t k = kbeg + " + std::to_string(n * rows_round) +
                                 " + q * 16 + lg * 4;\n";
                            t += std::string("                const idx_t kr = ") +
                                 (clamp ? "k < kend ? k : (idx_t)0" : "k") + ";\n";
                            t += "                const porch_v4f bq = *reinterpret_cast<const porch_v4f*>(" + bslot + " + " +
                                 operand_index(r.b, "kr", "qc", batch) + ");\n";
                            t += "                #pragma unroll\n                for (int e = 0; e < 4; ++e) bv[q][e] = bq[e];\n";
                            t += "            }\n";
                            return t;
                        }
                        t += "            #pragma unroll\n            for (int q = 0; q < 16; ++q)\n";
                        t += "                #pragma unroll\n                for (int e = 0; e < 4; ++e) {\n";
                        t += "                    const idx_t k = kbeg + " + std::to_string(n * rows_round) +
                             " + q * 16 + lg * 4 + e;\n";
                        t += std::string("                    const idx_t kr = ") + (clamp ? "k < kend ? k : (idx_t)0" : "k") +
                             ";\n";
                        t += "                    bv[q][e] = " + bslot + "[" + operand_index(r.b, "kr", "qc", batch) + "];\n";
                        t += "                }\n";
                        return t;
                    };
                    s += "        if (full) {\n" + b_loads(false) + "        }\n        else {\n" + b_loads(true) + "        }\n";
                    if (n + 1 < rounds) s += load_rows(nxt, n + 1);
                    s += "        __builtin_amdgcn_sched_barrier(0);\n";
                    // lane l holds k = base + 4 l .. + 3 of each of the 16 rows
                    // a round inside the wave's range needs no zeroing
                    s += "        if (full) {\n";
                    s += "            #pragma unroll\n            for (int rr = 0; rr < 16; ++rr)\n";
                    s += "                *reinterpret_cast<porch_v4f*>(my + rr * " + RS + " + 4 * lane) = " + cur + "[rr];\n";
                    s += "        }\n        else {\n";
                    s += "            const bool kin = kbeg + " + std::to_string(n * rows_round) + " + 4 * lane < kend;\n";
                    s += "            #pragma unroll\n            for (int rr = 0; rr < 16; ++rr)\n";
                    s += "                *reinterpret_cast<porch_v4f*>(my + rr * " + RS + " + 4 * lane) = kin ? " + cur +
                         "[rr] : porch_v4f{0.0f, 0.0f, 0.0f, 0.0f};\n";
                    s += "        }\n";
                    // the wave's lanes read each other's values: LDS operations
                    // of one wave complete in order, and the wave barrier keeps
                    // the compiler from moving the reads above the writes
                    s += "        __builtin_amdgcn_wave_barrier();\n";
                    s += "        __builtin_amdgcn_sched_barrier(0);\n";
                    // MFMA step e of group q: lane (li, lg) gives row li at
                    // k = base + 16 q + 4 lg + e (a float4 of the row per group)
                    auto mfma_loop = [&](bool guarded) {
                        std::string t;
                        t += "            #pragma unroll\n            for (int q = 0; q < 16; ++q) {\n";
                        t += "                const porch_v4f av = *reinterpret_cast<const porch_v4f*>(my + li * " + RS +
                             " + q * 16 + lg * 4);\n";
                        t += "                #pragma unroll\n                for (int e = 0; e < 4; ++e) {\n";
                        if (guarded) {
                            t += "                    const bool kin = kbeg + " + std::to_string(n * rows_round) +
                                 " + q * 16 + lg * 4 + e < kend;\n";
                            t += "                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], kin ? bv[q][e] : 0.0f, acc, "
                                 "0, 0, 0);\n";
                        }
                        else {
                            t += "                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], bv[q][e], acc, 0, 0, 0);\n";
                        }
                        t += "                }\n            }\n";
                        return t;
                    };
                    s += "        if (full) {\n" + mfma_loop(false) + "        }\n        else {\n" + mfma_loop(true) +
                         "        }\n";
                    s += "        __builtin_amdgcn_wave_barrier();\n";
                    s += "        __builtin_amdgcn_sched_barrier(0);\n";
                    s += "    }\n";
                }
            }
            // the waves' sums added in wave order
            s += "    __syncthreads();\n";
            s += "    porch_v4f* const red = reinterpret_cast<porch_v4f*>(&stage[0][0]);\n";
            s += "    red[w * 64 + lane] = acc;\n";
            s += "    __syncthreads();\n";
            s += "    if (w != 0) return;\n";
            s += "    #pragma unroll\n    for (int q = 1; q < " + std::to_string(waves) + "; ++q) acc += red[q * 64 + lane];\n";
            // accumulator value v of lane l: row 4 (l / 16) + v, column l % 16
            s += "    #pragma unroll\n    for (int v = 0; v < 4; ++v) {\n";
            s += "        const idx_t q0 = r0 + lg * 4 + v;\n";
            s += "        const idx_t q1 = li;\n";
            s += "        if (q0 < " + M + " && q1 < " + N + ") {\n";
            const std::string o = std::string(r.batched ? "(qb * " + M + " + q0)" : "q0") + " * " + N + " + q1";
            s += "            const float acc_v = acc[v];\n";
            s += epilogue_store(r, "acc_v", o, "            ");
            s += "        }\n    }\n}\n";
            return kc;
        }

    } // namespace

    kernel_code emit_gemm_narrow(const gemm_request& r) {
        const narrow_shape sh = narrow_plan(r);
        if (sh.rb == 0) throw std::logic_error("emit_gemm_narrow: not a narrow product");
        if (narrow_rows(r)) return emit_gemm_narrow_rows(r);
        const bool final = sh.chunks == 1;
        const char* T = r.width.type();
        const std::string batch = r.batched ? "qb" : "";
        const std::string M = std::to_string(r.m);
        const std::string N = std::to_string(r.n);
        const std::string K = std::to_string(r.k);
        const std::string RB = std::to_string(sh.rb);
        const std::string NB = std::to_string(sh.nb);
        const std::string CH = std::to_string(sh.chunks);
        const std::string CK = std::to_string(sh.chunk);
        const std::string G16 = std::to_string(group_size);

        kernel_code kc;
        kc.kind = "gemm.narrow";
        kc.name = "porch_gemm";
        kc.n_slots = r.n_slots;
        kc.block = 64 * group_waves;
        kc.grid_x = static_cast<unsigned>(r.batch * sh.tiles * sh.chunks);

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(256) porch_gemm(" + kernel_params(r.n_slots) + ") {\n";
        s += "    const int lane = threadIdx.x & 63;\n";
        s += "    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);\n";
        s += "    const int li = lane & 15;\n    const int lg = lane >> 4;\n";
        // the chunks of a tile are adjacent workgroups: the workgroups of one
        // chunk (which share its rows of B) land on the same XCDs
        s += "    const idx_t ks = (idx_t)blockIdx.x % " + CH + ";\n";
        s += "    const idx_t tile = (idx_t)blockIdx.x / " + CH + ";\n";
        s += "    const idx_t qb = tile / " + std::to_string(sh.tiles) + ";\n";
        if (!r.batched) s += "    (void)qb;\n";
        s += "    const idx_t r0 = (tile % " + std::to_string(sh.tiles) + ") * " + std::to_string(16 * sh.rb) + ";\n";
        s += "    const idx_t k0 = ks * " + CK + ";\n";
        s += "    const idx_t k1 = k0 + " + CK + " < " + K + " ? k0 + " + CK + " : (idx_t)" + K + ";\n";
        s += "    porch_v4f acc[" + RB + "][" + NB + "];\n";
        s += "    #pragma unroll\n    for (int i = 0; i < " + RB + "; ++i)\n";
        s += "        #pragma unroll\n        for (int j = 0; j < " + NB + "; ++j) acc[i][j] = porch_v4f{0.0f, 0.0f, 0.0f, 0.0f};\n";
        // Rows past m and columns past n are read at m - 1 and n - 1: they
        // feed only outputs that are not stored, so the loads need no
        // guard (guarded loads became one branch each, with every step
        // waiting for all of its loads).
        s += "    idx_t qa[" + RB + "];\n";
        s += "    #pragma unroll\n    for (int i = 0; i < " + RB + "; ++i) {\n";
        s += "        const idx_t q0 = r0 + i * 16 + li;\n";
        s += "        qa[i] = q0 < " + M + " ? q0 : (idx_t)" + std::to_string(r.m - 1) + ";\n";
        s += "    }\n";
        s += "    idx_t qc[" + NB + "];\n";
        s += "    #pragma unroll\n    for (int j = 0; j < " + NB + "; ++j) {\n";
        s += "        const idx_t q1 = j * 16 + li;\n";
        s += "        qc[j] = q1 < " + N + " ? q1 : (idx_t)" + std::to_string(r.n - 1) + ";\n";
        s += "    }\n";
        // A group: 16 values of K from kq.  Lane l holds k = kq + 4 (l / 16)
        // + e of its A row (one 128-bit non-temporal load a row block: 16
        // rows x 64 B an instruction) and of its B column (scalar loads from
        // the L2); MFMA e takes value e of every lane.
        const std::string aslot = "a" + std::to_string(r.a.slot);
        const std::string bslot = "a" + std::to_string(r.b.slot);
        auto declare = [&](const std::string& set, const std::string& ind) {
            return ind + "porch_v4f av" + set + "[" + RB + "];\n" + ind + "float bv" + set + "[" + NB + "][4];\n";
        };
        auto loads = [&](const std::string& set, const std::string& kq, const std::string& ind) {
            std::string t;
            t += ind + "#pragma unroll\n" + ind + "for (int i = 0; i < " + RB + "; ++i)\n";
            t += ind + "    av" + set + "[i] = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" + aslot +
                 " + " + operand_index(r.a, "qa[i]", "(" + kq + " + lg * 4)", batch) + "));\n";
            t += ind + "#pragma unroll\n" + ind + "for (int j = 0; j < " + NB + "; ++j) {\n";
            if (b_column_runs(r)) {
                // B stored transposed: the lane's four values of column
                // qc[j] are one 128-bit load
                t += ind + "    const porch_v4f bq = *reinterpret_cast<const porch_v4f*>(" + bslot + " + " +
                     operand_index(r.b, "(" + kq + " + lg * 4)", "qc[j]", batch) + ");\n";
                t += ind + "    #pragma unroll\n" + ind + "    for (int e = 0; e < 4; ++e) bv" + set + "[j][e] = bq[e];\n";
            } else {
                t += ind + "    #pragma unroll\n" + ind + "    for (int e = 0; e < 4; ++e)\n";
                t += ind + "        bv" + set + "[j][e] = " + bslot + "[" +
                     operand_index(r.b, "(" + kq + " + lg * 4 + e)", "qc[j]", batch) + "];\n";
            }
            t += ind + "}\n";
            return t;
        };
        auto mfmas = [&](const std::string& set, const std::string& ind) {
            std::string t;
            t += ind + "#pragma unroll\n" + ind + "for (int e = 0; e < 4; ++e)\n";
            t += ind + "    #pragma unroll\n" + ind + "    for (int i = 0; i < " + RB + "; ++i)\n";
            t += ind + "        #pragma unroll\n" + ind + "        for (int j = 0; j < " + NB + "; ++j)\n";
            t += ind + "            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av" + set + "[i][e], bv" + set +
                 "[j][e], acc[i][j], 0, 0, 0);\n";
            return t;
        };
        s += group_loop(r.k % sh.chunk == 0 ? sh.chunk / (group_waves * group_size) : 0, declare, loads, mfmas);
        // The partial last group (a chunk not a multiple of 16 values), in
        // the wave whose turn it is.  K and the chunks are multiples of 4,
        // so a lane's four values lie all inside or all past the chunk:
        // past it they are read at its last four values and both operands
        // are zeroed (zeroing one would turn an infinity in the other into
        // NaN).
        if (sh.chunk % group_size != 0 || r.k % group_size != 0) {
            s += "    if (full * " + G16 + " < k1 - k0 && full % 4 == w) {\n";
            s += "        const idx_t kb = k0 + full * " + G16 + " + lg * 4;\n";
            s += "        const bool kin = kb < k1;\n";
            s += "        const idx_t kr = kin ? kb : k1 - 4;\n";
            s += declare("R", "        ");
            s += "        #pragma unroll\n        for (int i = 0; i < " + RB + "; ++i) {\n";
            s += "            avR[i] = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" + aslot + " + " +
                 operand_index(r.a, "qa[i]", "kr", batch) + "));\n";
            s += "            if (!kin) avR[i] = porch_v4f{0.0f, 0.0f, 0.0f, 0.0f};\n";
            s += "        }\n";
            s += "        #pragma unroll\n        for (int j = 0; j < " + NB + "; ++j)\n";
            s += "            #pragma unroll\n            for (int e = 0; e < 4; ++e) {\n";
            s += "                const float x = " + bslot + "[" + operand_index(r.b, "(kr + e)", "qc[j]", batch) + "];\n";
            s += "                bvR[j][e] = kin ? x : 0.0f;\n";
            s += "            }\n";
            s += mfmas("R", "        ");
            s += "    }\n";
        }
        // The waves' sums, added in wave order through LDS.  Accumulator
        // value v of lane l: row 16 i + 4 (l / 16) + v, column 16 j + l % 16.
        const int64_t blocks = sh.rb * sh.nb;
        s += "    __shared__ porch_v4f red[4][" + std::to_string(blocks) + "][64];\n";
        s += "    #pragma unroll\n    for (int i = 0; i < " + RB + "; ++i)\n";
        s += "        #pragma unroll\n        for (int j = 0; j < " + NB + "; ++j) red[w][i * " + NB +
             " + j][lane] = acc[i][j];\n";
        s += "    __syncthreads();\n";
        s += "    for (int t = threadIdx.x; t < " + std::to_string(64 * blocks) + "; t += 256) {\n";
        s += "        const int b = t >> 6, l = t & 63;\n";
        s += "        const int i = b / " + NB + ", j = b % " + NB + ";\n";
        s += "        porch_v4f sum = red[0][b][l];\n";
        s += "        #pragma unroll\n        for (int u = 1; u < 4; ++u) sum += red[u][b][l];\n";
        s += "        const idx_t q1 = j * 16 + (l & 15);\n";
        s += "        #pragma unroll\n        for (int v = 0; v < 4; ++v) {\n";
        s += "            const idx_t q0 = r0 + i * 16 + (l >> 4) * 4 + v;\n";
        s += "            if (q0 < " + M + " && q1 < " + N + ") {\n";
        const std::string o = std::string(r.batched ? "(qb * " + M + " + q0)" : "q0") + " * " + N + " + q1";
        if (final) {
            s += "                const float acc_v = sum[v];\n";
            s += epilogue_store(r, "acc_v", o, "                ");
        }
        else {
            s += "                out[ks * " + std::to_string(r.batch * r.m * r.n) + " + " + o + "] = sum[v];\n";
        }
        s += "            }\n        }\n    }\n}\n";
        return kc;
    }

    bool gemm_wide(const gemm_request& r) { return wide_plan(r).rb > 0; }

    int64_t gemm_wide_chunks(const gemm_request& r) { return wide_plan(r).chunks; }

    kernel_code emit_gemm_wide(const gemm_request& r) {
        const wide_shape sh = wide_plan(r);
        if (sh.rb == 0) throw std::logic_error("emit_gemm_wide: not a wide product");
        const bool final = sh.chunks == 1;
        const bool avec = a_vector(r);
        // B stored transposed: its columns read along K, lane l taking the
        // columns c0 + 16 e + l % 16
        const bool bt = !b_vector(r);
        const char* T = r.width.type();
        const std::string batch = r.batched ? "qb" : "";
        const std::string M = std::to_string(r.m);
        const std::string N = std::to_string(r.n);
        const std::string K = std::to_string(r.k);
        const std::string RB = std::to_string(sh.rb);
        const std::string CH = std::to_string(sh.chunks);
        const std::string CK = std::to_string(sh.chunk);

        kernel_code kc;
        kc.kind = "gemm.wide";
        kc.name = "porch_gemm";
        kc.n_slots = r.n_slots;
        kc.block = 64 * group_waves;
        kc.grid_x = static_cast<unsigned>(r.batch * sh.tiles * sh.chunks);

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "extern \"C\" __global__ void __launch_bounds__(256) porch_gemm(" + kernel_params(r.n_slots) + ") {\n";
        s += "    const int lane = threadIdx.x & 63;\n";
        // the wave's index, known to the compiler as uniform: the loop over
        // the wave's groups branches on scalars (as a vector value the loop
        // was masked per lane and every wait drained all loads)
        s += "    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);\n";
        s += "    const int li = lane & 15;\n    const int lg = lane >> 4;\n";
        // the chunks of a tile are adjacent workgroups: the workgroups of one
        // chunk (which share its columns of A) land on the same XCDs
        s += "    const idx_t ks = (idx_t)blockIdx.x % " + CH + ";\n";
        s += "    const idx_t tile = (idx_t)blockIdx.x / " + CH + ";\n";
        s += "    const idx_t qb = tile / " + std::to_string(sh.tiles) + ";\n";
        if (!r.batched) s += "    (void)qb;\n";
        s += "    const idx_t c0 = (tile % " + std::to_string(sh.tiles) + ") * 64;\n";
        s += "    const idx_t k0 = ks * " + CK + ";\n";
        s += "    const idx_t k1 = k0 + " + CK + " < " + K + " ? k0 + " + CK + " : (idx_t)" + K + ";\n";
        // acc[i][e]: rows 16 i + 4 (l / 16) + v, column c0 + 4 (l % 16) + e
        s += "    porch_v4f acc[" + RB + "][4];\n";
        s += "    #pragma unroll\n    for (int i = 0; i < " + RB + "; ++i)\n";
        s += "        #pragma unroll\n        for (int e = 0; e < 4; ++e) acc[i][e] = porch_v4f{0.0f, 0.0f, 0.0f, 0.0f};\n";
        // Rows past m are read at m - 1 and columns past n at n - 4: they
        // feed only outputs that are not stored.
        s += "    idx_t qa[" + RB + "];\n";
        s += "    #pragma unroll\n    for (int i = 0; i < " + RB + "; ++i) {\n";
        s += "        const idx_t q0 = i * 16 + li;\n";
        s += "        qa[i] = q0 < " + M + " ? q0 : (idx_t)" + std::to_string(r.m - 1) + ";\n";
        s += "    }\n";
        if (bt) {
            s += "    idx_t qc[4];\n";
            s += "    #pragma unroll\n    for (int e = 0; e < 4; ++e) {\n";
            s += "        const idx_t c = c0 + 16 * e + li;\n";
            s += "        qc[e] = c < " + N + " ? c : (idx_t)" + std::to_string(r.n - 1) + ";\n";
            s += "    }\n";
        } else {
            s += "    const idx_t qc = c0 + li * 4 < " + N + " ? c0 + li * 4 : (idx_t)" + std::to_string(r.n - 4) + ";\n";
        }
        // A group: 16 values of K from kq.  MFMA j of the group gives lane l
        // k = kq + 4 (l / 16) + j: B's row there at columns qc .. qc + 3 (one
        // 128-bit load a j: 4 rows x 256 B an instruction; MFMA e takes
        // value e, the 16 columns 4 (l % 16) + e), and A's row qa[i] at the
        // four k of the lane (one 128-bit load where A's rows run along K).
        const std::string aslot = "a" + std::to_string(r.a.slot);
        const std::string bslot = "a" + std::to_string(r.b.slot);
        auto declare = [&](const std::string& set, const std::string& ind) {
            if (bt)
                return ind + "porch_v4f bv" + set + "[4][2];\n" + ind + "porch_v4f av" + set + "[" + RB + "][2];\n";
            return ind + "porch_v4f bv" + set + "[4];\n" + ind + "porch_v4f av" + set + "[" + RB + "];\n";
        };
        auto loads = [&](const std::string& set, const std::string& kq, const std::string& ind) {
            std::string t;
            if (bt) {
                // a group of 32 values of K in two halves s: column qc[e]
                // at the lane's four k of half s, one 128-bit load each
                // (16 columns x 64 B an instruction, the two halves of a
                // column's 128 B in two)
                t += ind + "#pragma unroll\n" + ind + "for (int e = 0; e < 4; ++e)\n";
                t += ind + "    #pragma unroll\n" + ind + "    for (int h = 0; h < 2; ++h)\n";
                t += ind + "        bv" + set + "[e][h] = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" +
                     bslot + " + " + operand_index(r.b, "(" + kq + " + 16 * h + lg * 4)", "qc[e]", batch) + "));\n";
                t += ind + "#pragma unroll\n" + ind + "for (int i = 0; i < " + RB + "; ++i)\n";
                t += ind + "    #pragma unroll\n" + ind + "    for (int h = 0; h < 2; ++h) {\n";
                if (avec) {
                    t += ind + "        av" + set + "[i][h] = *reinterpret_cast<const porch_v4f*>(" + aslot + " + " +
                         operand_index(r.a, "qa[i]", "(" + kq + " + 16 * h + lg * 4)", batch) + ");\n";
                } else {
                    t += ind + "        #pragma unroll\n" + ind + "        for (int j = 0; j < 4; ++j)\n";
                    t += ind + "            av" + set + "[i][h][j] = " + aslot + "[" +
                         operand_index(r.a, "qa[i]", "(" + kq + " + 16 * h + lg * 4 + j)", batch) + "];\n";
                }
                t += ind + "    }\n";
                return t;
            } else {
                t += ind + "#pragma unroll\n" + ind + "for (int j = 0; j < 4; ++j)\n";
                t += ind + "    bv" + set + "[j] = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" + bslot +
                     " + " + operand_index(r.b, "(" + kq + " + lg * 4 + j)", "qc", batch) + "));\n";
            }
            t += ind + "#pragma unroll\n" + ind + "for (int i = 0; i < " + RB + "; ++i) {\n";
            if (avec) {
                t += ind + "    av" + set + "[i] = *reinterpret_cast<const porch_v4f*>(" + aslot + " + " +
                     operand_index(r.a, "qa[i]", "(" + kq + " + lg * 4)", batch) + ");\n";
            }
            else {
                t += ind + "    #pragma unroll\n" + ind + "    for (int j = 0; j < 4; ++j)\n";
                t += ind + "        av" + set + "[i][j] = " + aslot + "[" +
                     operand_index(r.a, "qa[i]", "(" + kq + " + lg * 4 + j)", batch) + "];\n";
            }
            t += ind + "}\n";
            return t;
        };
        auto mfmas = [&](const std::string& set, const std::string& ind) {
            std::string t;
            if (bt) {
                t += ind + "#pragma unroll\n" + ind + "for (int h = 0; h < 2; ++h)\n";
                t += ind + "#pragma unroll\n" + ind + "for (int j = 0; j < 4; ++j)\n";
                t += ind + "    #pragma unroll\n" + ind + "    for (int e = 0; e < 4; ++e)\n";
                t += ind + "        #pragma unroll\n" + ind + "        for (int i = 0; i < " + RB + "; ++i)\n";
                t += ind + "            acc[i][e] = __builtin_amdgcn_mfma_f32_16x16x4f32(av" + set + "[i][h][j], bv" + set +
                     "[e][h][j], acc[i][e], 0, 0, 0);\n";
                return t;
            }
            t += ind + "#pragma unroll\n" + ind + "for (int j = 0; j < 4; ++j)\n";
            t += ind + "    #pragma unroll\n" + ind + "    for (int e = 0; e < 4; ++e)\n";
            t += ind + "        #pragma unroll\n" + ind + "        for (int i = 0; i < " + RB + "; ++i)\n";
            t += ind + "            acc[i][e] = __builtin_amdgcn_mfma_f32_16x16x4f32(av" + set + "[i][j], bv" + set +
                 "[j][e], acc[i][e], 0, 0, 0);\n";
            return t;
        };
        const int64_t width = wide_group(r);
        s += group_loop(r.k % sh.chunk == 0 ? sh.chunk / (group_waves * width) : 0, declare, loads, mfmas, width);
        const std::string G16 = std::to_string(group_size);
        // The partial last group (a chunk not a multiple of 16 values), in
        // the wave whose turn it is: lanes past the chunk read its last
        // value and zero both operands.
        if (sh.chunk % group_size != 0 || r.k % group_size != 0) {
            if (bt) throw std::logic_error("emit_gemm_wide: B read along K needs whole groups");
            s += "    if (full * " + G16 + " < k1 - k0 && full % 4 == w) {\n";
            s += "        const idx_t kq = k0 + full * " + G16 + ";\n";
            s += declare("R", "        ");
            s += "        #pragma unroll\n        for (int j = 0; j < 4; ++j) {\n";
            s += "            const idx_t kb = kq + lg * 4 + j;\n";
            s += "            const bool kin = kb < k1;\n";
            s += "            const idx_t kr = kin ? kb : k1 - 1;\n";
            s += "            bvR[j] = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" + bslot + " + " +
                 operand_index(r.b, "kr", "qc", batch) + "));\n";
            s += "            if (!kin) bvR[j] = porch_v4f{0.0f, 0.0f, 0.0f, 0.0f};\n";
            s += "            #pragma unroll\n            for (int i = 0; i < " + RB + "; ++i) {\n";
            s += "                const float x = " + aslot + "[" + operand_index(r.a, "qa[i]", "kr", batch) + "];\n";
            s += "                avR[i][j] = kin ? x : 0.0f;\n";
            s += "            }\n        }\n";
            s += mfmas("R", "        ");
            s += "    }\n";
        }
        // The waves' sums, added in wave order through LDS; each thread
        // then holds four adjacent columns of one row (B read along K: the
        // columns c0 + 16 e + l % 16).
        s += "    __shared__ porch_v4f red[4][" + std::to_string(4 * sh.rb) + "][64];\n";
        s += "    #pragma unroll\n    for (int i = 0; i < " + RB + "; ++i)\n";
        s += "        #pragma unroll\n        for (int e = 0; e < 4; ++e) red[w][i * 4 + e][lane] = acc[i][e];\n";
        s += "    __syncthreads();\n";
        s += "    for (int t = threadIdx.x; t < " + std::to_string(256 * sh.rb) + "; t += 256) {\n";
        s += "        const int i = t >> 8, v = (t >> 6) & 3, l = t & 63;\n";
        s += "        const idx_t q0 = i * 16 + (l >> 4) * 4 + v;\n";
        s += std::string("        const idx_t qc4 = c0 + (l & 15) * ") + (bt ? "1" : "4") + ";\n";
        s += "        if (q0 < " + M + " && qc4 < " + N + ") {\n";
        s += "            porch_v4f sum;\n";
        s += "            #pragma unroll\n            for (int e = 0; e < 4; ++e) {\n";
        s += "                float x = red[0][i * 4 + e][l][v];\n";
        s += "                #pragma unroll\n                for (int u = 1; u < 4; ++u) x += red[u][i * 4 + e][l][v];\n";
        s += "                sum[e] = x;\n            }\n";
        const std::string row = r.batched ? "(qb * " + M + " + q0)" : "q0";
        if (bt) {
            s += "            #pragma unroll\n            for (int e = 0; e < 4; ++e) {\n";
            s += "                const idx_t q1 = qc4 + 16 * e;\n";
            s += "                if (q1 < " + N + ") {\n";
            if (final) {
                s += "                    const float acc_v = sum[e];\n";
                s += epilogue_store(r, "acc_v", row + " * " + N + " + q1", "                    ");
            } else {
                s += "                    out[ks * " + std::to_string(r.batch * r.m * r.n) + " + " + row + " * " + N +
                     " + q1] = sum[e];\n";
            }
            s += "                }\n            }\n";
        }
        else if (final) {
            s += "            #pragma unroll\n            for (int e = 0; e < 4; ++e) {\n";
            s += "                const idx_t q1 = qc4 + e;\n";
            s += "                const float acc_v = sum[e];\n";
            s += epilogue_store(r, "acc_v", row + " * " + N + " + q1", "                ");
            s += "            }\n";
        }
        else {
            s += "            *reinterpret_cast<porch_v4f*>(out + ks * " + std::to_string(r.batch * r.m * r.n) + " + " + row +
                 " * " + N + " + qc4) = sum;\n";
        }
        s += "        }\n    }\n}\n";
        return kc;
    }

} // namespace porch::cg
