// Products with a short K (8 to 64, a multiple of 8) over many rows and
// columns, such as attention scores q @ k^T per head: each output costs only
// K multiply-adds, so the kernel is bound by its MFMAs and its output
// stores together, and what a 128 x 128 tile spends besides its MFMAs
// decides the rate.
//
//   gemm.band   one workgroup (four waves, two per compute unit) per batch
//               entry and band of 128 rows, walking the band's column tiles
//               (or a run of them, where there are fewer bands than two per
//               compute unit).
//               Each wave keeps its 64 rows x K of A in registers as
//               v_mfma_f32_32x32x2f32 operands for the whole band, with K
//               permuted so that lane half h takes k = hK/2 + s at step s
//               (a lane's K/2 values are one run, read as float4s); only
//               the K x 128 tile of B goes through LDS, double-buffered,
//               the next tile's loads one tile ahead in registers (B's
//               rows read along N, or, where B is stored transposed as in
//               q @ k^T with k [n, K], its columns read along K and
//               written to LDS transposed).  A
//               wave's 64 x 64 of a tile is two halves of 64 x 32: the
//               MFMAs of one half run while the other half's results (of
//               this tile or the previous one), with the epilogue applied,
//               go out through LDS 16 rows at a time as float4 rows (8 rows
//               x 128 B a store instruction; the MFMA layout would take 64
//               stores of 2 rows x 128 B a lane per tile), spread over the
//               MFMA steps.
//
// Measured against the persistent gemm.mfma on the attention product
// [16, 4096, 64] @ [16, 64, 4096]: in the benchmark, two runs of each on one
// box, 328.9 and 333.7 us against 370.9 and 370.0 us; launches alternating
// in one process, 338.0 against 377.3 us (a form storing straight from the
// MFMA layout 357.4 against 384.9 us).  The persistent kernel's
// texture-address FIFOs were full for about as many cycles as the shader
// engines were busy; this kernel's never are.  B's tiles are read with
// plain loads: every band of a batch entry reads them (with non-temporal
// loads the kernel was no faster than the persistent one, 376.7 us).  With
// the bands split into runs, against the persistent kernel on one box:
// [2, 8192, 64] @ [2, 64, 8192] 213.0 against 243.9 us, [4096, 64] @ [64,
// 4096] 28.8 against 31.6, [6016, 8] @ [8, 3968] 17.5 against 23.0.  With
// the staging of one half spread over the other half's MFMAs (against the
// results staged after all of a tile's MFMAs), under the kernel tracer on one
// box: attention 375.7 against 392.3 us, [2, 8192, 64] @ [2, 64, 8192] 198.6
// against 215.5, [64, 1024, 64] @ [64, 64, 1024] 94.2 against 107.0, [16,
// 4096, 32] @ [16, 32, 4096] 261.9 against 266.5; at K of 8 and 16 within
// 1-2 %.  In the benchmark, alternating runs on one box: attention 309.4
// against 324.3-325.2 us (70.6 % against 67.3 % of the fp32 MFMA peak).
// With k^T a view (B's columns along K), the attention product under the
// tracer on one (slow) box: 383.0 us, against 371.2 for k^T stored and
// 436.1 for the persistent kernel that took the view before.
//
// Sums: each output's K products in the MFMA's order, within the matmul's
// accumulation bound.

#include "emit_gemm.hpp"

#include <algorithm>
#include <stdexcept>

namespace porch::cg {
    namespace {

        constexpr int64_t band_rows = 128;
        constexpr int64_t tile_cols = 128;
        constexpr int64_t max_k = 64;
        constexpr int64_t b_pitch = tile_cols + 4; // LDS row of B, floats
        // LDS row of B read from columns along K: 129 = 1 mod 64, so the
        // scalar writes of a wave (16 k-quads x 4 columns) and the MFMA-side
        // reads (32 columns of two rows K/2 apart) meet 64 different banks
        constexpr int64_t b_pitch_cols = tile_cols + 1;
        constexpr int64_t w_pitch = 32 + 4;        // LDS row of a wave's staged results, floats

        struct band_shape {
            int64_t per_entry = 0; // bands of 128 rows per batch entry
            int64_t tiles = 0;     // column tiles of 128
            int64_t chunks = 0;    // runs of column tiles a band is split into
            int64_t per_chunk = 0; // column tiles a run
            int64_t groups = 0;    // workgroups
        };

        // Two workgroups for every compute unit: the bands, each split into
        // runs of its column tiles where there are fewer bands than that,
        // every run at least two tiles (a workgroup loads its rows of A once
        // for all of its tiles).
        band_shape band_plan(const gemm_request& r) {
            band_shape sh;
            sh.per_entry = (r.m + band_rows - 1) / band_rows;
            sh.tiles = (r.n + tile_cols - 1) / tile_cols;
            const int64_t want = 2 * static_cast<int64_t>(std::max(r.compute_units, 8));
            const int64_t bands = r.batch * sh.per_entry;
            int64_t chunks = std::max<int64_t>(1, (want + bands - 1) / bands);
            chunks = std::min(chunks, std::max<int64_t>(1, sh.tiles / 2));
            sh.per_chunk = (sh.tiles + chunks - 1) / chunks;
            sh.chunks = (sh.tiles + sh.per_chunk - 1) / sh.per_chunk;
            sh.groups = bands * sh.chunks;
            return sh;
        }

        // B's rows contiguous along N (read as float4 rows of a tile)
        bool b_rows(const gemm_request& r) {
            return r.b.stride_col == 1 && r.b.offset % 4 == 0 && r.b.stride_row % 4 == 0 && r.b.stride_batch % 4 == 0;
        }

        // B's columns contiguous along K, as in q @ k^T with k stored [n, K]
        // (read as float4 runs of a column, written to LDS transposed)
        bool b_cols(const gemm_request& r) {
            return r.b.stride_row == 1 && r.b.offset % 4 == 0 && r.b.stride_col % 4 == 0 && r.b.stride_batch % 4 == 0;
        }

    } // namespace

    bool gemm_band(const gemm_request& r) {
        const bool a_runs = r.a.stride_col == 1 && r.a.offset % 4 == 0 && r.a.stride_row % 4 == 0 &&
                            r.a.stride_batch % 4 == 0;
        if (r.k_chunks != 1 || r.k < 8 || r.k > max_k || r.k % 8 != 0 || !a_runs || r.n % 4 != 0 ||
            !(b_rows(r) || b_cols(r)) || r.n < 2 * tile_cols)
            return false;
        return band_plan(r).groups >= 2 * static_cast<int64_t>(std::max(r.compute_units, 8));
    }

    kernel_code emit_gemm_band(const gemm_request& r) {
        if (!gemm_band(r)) throw std::logic_error("emit_gemm_band: not a short-K band product");
        const char* T = r.width.type();
        const band_shape sh = band_plan(r);
        const int64_t total = sh.groups;
        const int64_t hk = r.k / 2;                        // MFMA steps a half (and values a lane holds a row)
        const int64_t b_loads = r.k * tile_cols / 4 / 256; // float4s of B a thread per tile
        const int64_t span = hk / 4;                        // steps a staging pass spans
        const bool ragged = r.m % band_rows != 0 || r.n % tile_cols != 0;
        // Non-temporal stores where the MFMAs dominate (K past 32: 375.7
        // against 392.4 us on the attention product, 198.6 against 211.1 at
        // [2, 8192, 64] @ [2, 64, 8192]); where the stores dominate they
        // were slower ([16, 4096, 8] @ [16, 8, 4096] 226.3 against 203.2 us,
        // [4, 4096, 32] @ [4, 32, 4096] 78.9 against 59.6).  In between, at
        // [16, 4096, K] @ [16, K, 4096] timed back to back: K = 40 216.4
        // against 214.3 us, 48 214.9 against 241.5, 56 242.8 against 269.3.
        const bool nt_store = r.k > 32;
        const std::string M = std::to_string(r.m);
        const std::string N = std::to_string(r.n);
        const std::string HK = std::to_string(hk);
        const std::string BL = std::to_string(b_loads);
        const std::string TC = std::to_string(tile_cols);
        const bool transposed = !b_rows(r); // B's columns contiguous along K
        const std::string BP = std::to_string(transposed ? b_pitch_cols : b_pitch);
        const std::string WP = std::to_string(w_pitch);
        const std::string batch = r.batched ? "qb" : "";
        const std::string last = "t0 + count - 1";

        kernel_code kc;
        kc.kind = "gemm.band";
        kc.name = "porch_gemm";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>(total);

        const std::string aslot = "a" + std::to_string(r.a.slot);
        const std::string bslot = "a" + std::to_string(r.b.slot);
        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "typedef float floatx16 __attribute__((ext_vector_type(16)));\n";
        // two workgroups per compute unit: the register budget of two waves
        // per SIMD
        s += "extern \"C\" __global__ void __launch_bounds__(256, 2) porch_gemm(" + kernel_params(r.n_slots) + ") {\n";
        s += "    __shared__ __attribute__((aligned(16))) float Bs[2][" + std::to_string(r.k) + "][" + BP + "];\n";
        s += "    __shared__ __attribute__((aligned(16))) float Ws[4][16][" + WP + "];\n";
        s += "    const int tid = threadIdx.x;\n";
        s += "    const int lane = tid & 63;\n";
        s += "    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);\n";
        s += "    const int wm = wave >> 1, wn = wave & 1;\n";
        s += "    const int h = lane >> 5, li = lane & 31;\n";
        // Workgroups are dispatched round-robin over the 8 XCDs: adjacent
        // bands of one run of tiles (which read the same B) go to one XCD
        // where the grid allows.  Workgroup (batch entry, run, band), the
        // band fastest.
        if (total % 8 == 0)
            s += "    const idx_t lin = (idx_t)(blockIdx.x % 8) * " + std::to_string(total / 8) + " + blockIdx.x / 8;\n";
        else
            s += "    const idx_t lin = blockIdx.x;\n";
        s += "    const idx_t m0 = (lin % " + std::to_string(sh.per_entry) + ") * " + std::to_string(band_rows) + ";\n";
        s += "    const idx_t run = (lin / " + std::to_string(sh.per_entry) + ") % " + std::to_string(sh.chunks) + ";\n";
        s += "    const idx_t qb = lin / " + std::to_string(sh.per_entry * sh.chunks) + ";\n";
        if (!r.batched) s += "    (void)qb;\n";
        // this workgroup's column tiles: t0 .. t0 + count - 1
        s += "    const int t0 = (int)run * " + std::to_string(sh.per_chunk) + ";\n";
        s += "    const int count = " + std::to_string(sh.tiles) + " - t0 < " + std::to_string(sh.per_chunk) + " ? " +
             std::to_string(sh.tiles) + " - t0 : " + std::to_string(sh.per_chunk) + ";\n";
        // A as MFMA operands: af[bi][j] holds row 64 wm + 32 bi + li of the
        // band at k = h K/2 + 4 j .. + 3 (rows past m read at m - 1: they
        // feed only outputs that are not stored)
        s += "    porch_v4f af[2][" + std::to_string(hk / 4) + "];\n";
        s += "    #pragma unroll\n    for (int bi = 0; bi < 2; ++bi) {\n";
        s += "        const idx_t q0 = m0 + 64 * wm + 32 * bi + li;\n";
        s += "        const idx_t qa = q0 < " + M + " ? q0 : (idx_t)" + std::to_string(r.m - 1) + ";\n";
        s += "        #pragma unroll\n        for (int j = 0; j < " + std::to_string(hk / 4) + "; ++j)\n";
        s += "            af[bi][j] = *reinterpret_cast<const porch_v4f*>(" + aslot + " + " +
             operand_index(r.a, "qa", HK + " * h + 4 * j", batch) + ");\n";
        s += "    }\n";
        // B's tile nt, rows along N: thread tid takes float4 f = tid + 256 u,
        // row f / 32, columns 4 (f % 32) .. + 3 (columns past n read at
        // n - 4).  Columns along K: float4 f holds k = 4 (f % (K / 4)) .. + 3
        // of column f / (K / 4) (columns past n read at n - 1), written to
        // LDS as four rows of one column.
        const std::string KQ = std::to_string(r.k / 4);
        s += "    porch_v4f rb[" + BL + "];\n";
        auto load_b = [&](const std::string& nt) {
            std::string t;
            t += "    {\n        const int nt = " + nt + ";\n";
            t += "        #pragma unroll\n        for (int u = 0; u < " + BL + "; ++u) {\n";
            t += "            const int f = tid + 256 * u;\n";
            if (transposed) {
                t += "            const idx_t c = (idx_t)nt * " + TC + " + f / " + KQ + ";\n";
                t += "            const idx_t cc = c < " + N + " ? c : (idx_t)" + std::to_string(r.n - 1) + ";\n";
                t += "            rb[u] = *reinterpret_cast<const porch_v4f*>(" + bslot + " + " +
                     operand_index(r.b, "4 * (f % " + KQ + ")", "cc", batch) + ");\n";
            } else {
                t += "            const idx_t c = (idx_t)nt * " + TC + " + 4 * (f & 31);\n";
                t += "            const idx_t cc = c < " + N + " ? c : (idx_t)" + std::to_string(r.n - 4) + ";\n";
                // plain loads: every band of a batch entry reads the same tiles
                t += "            rb[u] = *reinterpret_cast<const porch_v4f*>(" + bslot + " + " +
                     operand_index(r.b, "(f >> 5)", "cc", batch) + ");\n";
            }
            t += "        }\n    }\n";
            return t;
        };
        auto write_b = [&](const std::string& buf) {
            std::string t;
            t += "    #pragma unroll\n    for (int u = 0; u < " + BL + "; ++u) {\n";
            t += "        const int f = tid + 256 * u;\n";
            if (transposed) {
                t += "        #pragma unroll\n        for (int e = 0; e < 4; ++e)\n";
                t += "            Bs[" + buf + "][4 * (f % " + KQ + ") + e][f / " + KQ + "] = rb[u][e];\n";
            } else {
                t += "        *reinterpret_cast<porch_v4f*>(&Bs[" + buf + "][f >> 5][4 * (f & 31)]) = rb[u];\n";
            }
            t += "    }\n";
            return t;
        };
        // the run's tile `x` tiles on, clamped to its last: loads past the
        // run repeat the last tile and go into a buffer no tile reads
        auto clamped = [&](const std::string& x) { return "(t0 + " + x + " < t0 + count ? t0 + " + x + " : " + last + ")"; };

        // The epilogue of one value: acc_v at output (q0, q1), its inputs
        // read at coordinates clamped into the output (values past it are
        // not stored).
        std::string epi_body, epi_value;
        {
            emitter em(*r.expr, epi_body, 1);
            em.indent = "            ";
            em.declare_roots({r.epilogue});
            const std::vector<std::string> names =
                r.batched ? std::vector<std::string>{"qb", "e0", "e1"} : std::vector<std::string>{"e0", "e1"};
            epilogue_emitter(em, r, names, "acc_v");
            epi_value = em.emit(r.epilogue)[0];
        }
        const std::string row = r.batched ? "(qb * " + M + " + q0)" : "q0";
        // Staging pass p (0..3) of half bj of the tile at column tile `tile`:
        // rows 32 (p / 2) + 16 (p % 2) .. + 15 of the wave's 64, its 32
        // columns.  Part 0 applies the epilogue and writes the 8 values a
        // lane holds there into the wave's 16 x 32 area (register v of
        // block bi is row 8 (v / 4) + 4 h + v % 4, column li); part 1 reads
        // it back as float4 rows; part 2 stores them, 8 rows x 128 B a store
        // instruction.
        auto stage_part = [&](int bj, int p, int part, const std::string& tile) {
            const int bi = p >> 1, vh = (p & 1) * 2;
            const std::string acc = "c" + std::to_string(bi) + std::to_string(bj);
            std::string t;
            if (part == 0) {
                t += "        #pragma unroll\n        for (int vv = 0; vv < 2; ++vv)\n";
                t += "        #pragma unroll\n        for (int q = 0; q < 4; ++q) {\n";
                t += "            const idx_t q0 = m0 + 64 * wm + " + std::to_string(32 * bi + 16 * (p & 1)) +
                     " + 8 * vv + 4 * h + q;\n";
                t += "            const idx_t q1 = (idx_t)(" + tile + ") * " + TC + " + 64 * wn + " +
                     std::to_string(32 * bj) + " + li;\n";
                t += "            const idx_t e0 = q0 < " + M + " ? q0 : (idx_t)" + std::to_string(r.m - 1) + ";\n";
                t += "            const idx_t e1 = q1 < " + N + " ? q1 : (idx_t)" + std::to_string(r.n - 1) + ";\n";
                t += "            (void)e0; (void)e1;\n";
                t += "            const float acc_v = " + acc + "[" + std::to_string(4 * vh) + " + 4 * vv + q];\n";
                t += epi_body;
                t += "            Ws[wave][8 * vv + 4 * h + q][li] = " + epi_value + ";\n";
                t += "        }\n";
                // the wave reads other lanes' writes: its LDS operations
                // complete in order, and the wave barrier keeps the compiler
                // from moving the reads above the writes (or the next pass's
                // writes above these reads)
                t += "        __builtin_amdgcn_wave_barrier();\n";
            } else if (part == 1) {
                t += "        #pragma unroll\n        for (int u = 0; u < 2; ++u)\n";
                t += "            sx[u] = *reinterpret_cast<const porch_v4f*>(&Ws[wave][(lane >> 3) + 8 * u][4 * (lane & 7)]);\n";
                t += "        __builtin_amdgcn_wave_barrier();\n";
            } else {
                t += "        #pragma unroll\n        for (int u = 0; u < 2; ++u) {\n";
                t += "            const idx_t q0 = m0 + 64 * wm + " + std::to_string(32 * bi + 16 * (p & 1)) +
                     " + 8 * u + (lane >> 3);\n";
                t += "            const idx_t q1 = (idx_t)(" + tile + ") * " + TC + " + 64 * wn + " +
                     std::to_string(32 * bj) + " + 4 * (lane & 7);\n";
                if (ragged) t += "            if (q0 < " + M + " && q1 < " + N + ")\n";
                if (nt_store)
                    t += "            __builtin_nontemporal_store(sx[u], reinterpret_cast<porch_v4f*>(out + " + row + " * " +
                         N + " + q1));\n";
                else
                    t += "            *reinterpret_cast<porch_v4f*>(out + " + row + " * " + N + " + q1) = sx[u];\n";
                t += "        }\n";
            }
            return t;
        };
        // One half's MFMAs (columns 32 bj .. + 31 of the wave's 64) over the
        // tile in buffer `buf`, two blocks of 32 x 32 (bi = 0, 1) sharing
        // each value of B, read from LDS two steps ahead; the other half's
        // staging (half sbj of tile `stile`, if any) spread over the steps:
        // pass p's parts at steps p span, p span + span / 4, p span + span / 2.
        auto phase = [&](int bj, const std::string& buf, int sbj, const std::string& stile) {
            const std::string c0 = "c0" + std::to_string(bj), c1 = "c1" + std::to_string(bj);
            const std::string col = "64 * wn + " + std::to_string(32 * bj) + " + li";
            std::string t;
            t += "    {\n";
            t += "        float bq[" + HK + "];\n";
            t += "        porch_v4f sx[2];\n";
            t += "        (void)sx;\n";
            const int64_t ahead = std::min<int64_t>(2, hk);
            for (int64_t st = 0; st < ahead; ++st)
                t += "        bq[" + std::to_string(st) + "] = Bs[" + buf + "][" + HK + " * h + " + std::to_string(st) +
                     "][" + col + "];\n";
            for (int64_t st = 0; st < hk; ++st) {
                if (st + ahead < hk)
                    t += "        bq[" + std::to_string(st + ahead) + "] = Bs[" + buf + "][" + HK + " * h + " +
                         std::to_string(st + ahead) + "][" + col + "];\n";
                t += "        __builtin_amdgcn_sched_barrier(0);\n";
                if (sbj >= 0)
                    for (int p = 0; p < 4; ++p)
                        for (int part = 0; part < 3; ++part) {
                            const int64_t at = p * span + (part == 0 ? 0 : part == 1 ? span / 4 : span / 2);
                            if (at == st) t += stage_part(sbj, p, part, stile);
                        }
                t += "        __builtin_amdgcn_sched_barrier(0);\n";
                const std::string j = std::to_string(st >> 2), e = std::to_string(st & 3);
                const std::string b = "bq[" + std::to_string(st) + "]";
                t += "        " + c0 + " = __builtin_amdgcn_mfma_f32_32x32x2f32(af[0][" + j + "][" + e + "], " + b +
                     ", " + (st == 0 ? std::string("zero") : c0) + ", 0, 0, 0);\n";
                t += "        " + c1 + " = __builtin_amdgcn_mfma_f32_32x32x2f32(af[1][" + j + "][" + e + "], " + b +
                     ", " + (st == 0 ? std::string("zero") : c1) + ", 0, 0, 0);\n";
                t += "        __builtin_amdgcn_sched_barrier(0);\n";
            }
            t += "    }\n";
            return t;
        };
        auto stage_all = [&](int bj, const std::string& tile) {
            std::string t = "    {\n        porch_v4f sx[2];\n";
            for (int p = 0; p < 4; ++p)
                for (int part = 0; part < 3; ++part) t += stage_part(bj, p, part, tile);
            return t + "    }\n";
        };

        // Each tile: its two halves' MFMAs, half 0 while half 1 of the
        // previous tile goes out, half 1 while half 0 of this tile goes out;
        // the next tile's LDS writes and the loads of the one after (both
        // clamped to the run, so every tile issues the same loads, LDS
        // writes and stores) ahead of them.
        s += "    const floatx16 zero = {};\n";
        s += "    floatx16 c00, c10, c01, c11;\n";
        s += load_b("t0") + write_b("0");
        s += "    __syncthreads();\n";
        s += load_b(clamped("1"));
        s += write_b("1");
        s += load_b(clamped("2"));
        s += "    __builtin_amdgcn_sched_barrier(0);\n";
        s += phase(0, "0", -1, "");
        s += phase(1, "0", 0, "t0");
        s += "    __syncthreads();\n";
        s += "    for (int t = 1; t < count; ++t) {\n";
        s += "    const int buf = t & 1;\n";
        s += write_b("buf ^ 1");
        s += load_b(clamped("t + 2"));
        s += "    __builtin_amdgcn_sched_barrier(0);\n";
        s += phase(0, "buf", 1, "t0 + t - 1");
        s += phase(1, "buf", 0, "t0 + t");
        s += "    __syncthreads();\n";
        s += "    }\n";
        s += stage_all(1, last);
        s += "}\n";
        return kc;
    }

} // namespace porch::cg
