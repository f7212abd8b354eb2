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
//               the next tile's loads one tile ahead in registers.  A
//               tile's results, with the epilogue applied, go out through
//               LDS 8 rows at a time as float4 rows (4 rows x 256 B a store
//               instruction; the MFMA layout would take 64 stores of 2 rows
//               x 128 B a lane per tile).
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
// 4096] 28.8 against 31.6, [6016, 8] @ [8, 3968] 17.5 against 23.0.
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
        constexpr int64_t w_pitch = 64 + 4;        // LDS row of a wave's results, floats

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

    } // namespace

    bool gemm_band(const gemm_request& r) {
        const bool a_runs = r.a.stride_col == 1 && r.a.offset % 4 == 0 && r.a.stride_row % 4 == 0 &&
                            r.a.stride_batch % 4 == 0;
        const bool b_rows = r.b.stride_col == 1 && r.n % 4 == 0 && r.b.offset % 4 == 0 && r.b.stride_row % 4 == 0 &&
                            r.b.stride_batch % 4 == 0;
        if (r.k_chunks != 1 || r.k < 8 || r.k > max_k || r.k % 8 != 0 || !a_runs || !b_rows || r.n < 2 * tile_cols)
            return false;
        return band_plan(r).groups >= 2 * static_cast<int64_t>(std::max(r.compute_units, 8));
    }

    kernel_code emit_gemm_band(const gemm_request& r) {
        if (!gemm_band(r)) throw std::logic_error("emit_gemm_band: not a short-K band product");
        const char* T = r.width.type();
        const band_shape sh = band_plan(r);
        const int64_t per_entry = sh.per_entry;
        const int64_t total = sh.groups;
        const int64_t tiles = sh.tiles;
        const int64_t hk = r.k / 2;                      // MFMA steps (and values a lane holds a row)
        const int64_t b_loads = r.k * tile_cols / 4 / 256; // float4s of B a thread per tile
        const std::string M = std::to_string(r.m);
        const std::string N = std::to_string(r.n);
        const std::string K = std::to_string(r.k);
        const std::string HK = std::to_string(hk);
        const std::string BL = std::to_string(b_loads);
        const std::string batch = r.batched ? "qb" : "";

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
        s += "    __shared__ __attribute__((aligned(16))) float Bs[2][" + K + "][" + std::to_string(b_pitch) + "];\n";
        s += "    __shared__ __attribute__((aligned(16))) float Ws[4][8][" + std::to_string(w_pitch) + "];\n";
        s += "    const int tid = threadIdx.x;\n";
        s += "    const int lane = tid & 63;\n";
        s += "    const int wave = tid >> 6;\n";
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
        s += "    const idx_t m0 = (lin % " + std::to_string(per_entry) + ") * " + std::to_string(band_rows) + ";\n";
        s += "    const idx_t run = (lin / " + std::to_string(per_entry) + ") % " + std::to_string(sh.chunks) + ";\n";
        s += "    const idx_t qb = lin / " + std::to_string(per_entry * sh.chunks) + ";\n";
        if (!r.batched) s += "    (void)qb;\n";
        // this workgroup's column tiles: t0 .. t0 + count - 1
        s += "    const int t0 = (int)run * " + std::to_string(sh.per_chunk) + ";\n";
        s += "    const int count = " + std::to_string(tiles) + " - t0 < " + std::to_string(sh.per_chunk) + " ? " +
             std::to_string(tiles) + " - t0 : " + std::to_string(sh.per_chunk) + ";\n";
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
        // B's tile nt: thread tid takes float4 f = tid + 256 u, row f / 32,
        // columns 4 (f % 32) .. + 3 (columns past n read at n - 4)
        s += "    porch_v4f rb[" + BL + "];\n";
        auto load_b = [&](const std::string& nt) {
            std::string t;
            t += "    #pragma unroll\n    for (int u = 0; u < " + BL + "; ++u) {\n";
            t += "        const int f = tid + 256 * u;\n";
            t += "        const idx_t c = (idx_t)(" + nt + ") * " + std::to_string(tile_cols) + " + 4 * (f & 31);\n";
            t += "        const idx_t cc = c < " + N + " ? c : (idx_t)" + std::to_string(r.n - 4) + ";\n";
            // plain loads: every band of a batch entry reads the same tiles
            t += "        rb[u] = *reinterpret_cast<const porch_v4f*>(" + bslot + " + " +
                 operand_index(r.b, "(f >> 5)", "cc", batch) + ");\n";
            t += "    }\n";
            return t;
        };
        auto write_b = [&](const std::string& buf) {
            std::string t;
            t += "    #pragma unroll\n    for (int u = 0; u < " + BL + "; ++u) {\n";
            t += "        const int f = tid + 256 * u;\n";
            t += "        *reinterpret_cast<porch_v4f*>(&Bs[" + buf + "][f >> 5][4 * (f & 31)]) = rb[u];\n";
            t += "    }\n";
            return t;
        };
        // (a run's second tile is loaded ahead even where the run has one:
        // the columns are clamped into B and the values never used)
        s += load_b("t0") + write_b("0");
        s += "    __syncthreads();\n";
        s += load_b("t0 + 1");
        s += "    for (int t = 0; t < count; ++t) {\n";
        s += "        const int buf = t & 1;\n";
        s += "        floatx16 acc[2][2];\n";
        s += "        #pragma unroll\n        for (int i = 0; i < 2; ++i)\n";
        s += "            #pragma unroll\n            for (int j = 0; j < 2; ++j)\n";
        s += "                #pragma unroll\n                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;\n";
        // the next tile into the other buffer (its last readers finished
        // before the previous barrier) and the one after into registers,
        // issued ahead of this tile's MFMAs
        s += "        if (t + 1 < count) {\n" + write_b("buf ^ 1") + "        }\n";
        s += "        if (t + 2 < count) {\n" + load_b("t0 + t + 2") + "        }\n";
        s += "        __builtin_amdgcn_sched_barrier(0);\n";
        s += "        #pragma unroll\n        for (int st = 0; st < " + HK + "; ++st) {\n";
        s += "            const float b0 = Bs[buf][" + HK + " * h + st][64 * wn + li];\n";
        s += "            const float b1 = Bs[buf][" + HK + " * h + st][64 * wn + 32 + li];\n";
        s += "            const float x0 = af[0][st >> 2][st & 3];\n";
        s += "            const float x1 = af[1][st >> 2][st & 3];\n";
        s += "            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(x0, b0, acc[0][0], 0, 0, 0);\n";
        s += "            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(x0, b1, acc[0][1], 0, 0, 0);\n";
        s += "            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(x1, b0, acc[1][0], 0, 0, 0);\n";
        s += "            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(x1, b1, acc[1][1], 0, 0, 0);\n";
        s += "        }\n";
        // The results, 8 rows at a time: register v of block (bi, bj) is row
        // 8 (v / 4) + 4 h + v % 4 of the block, column li; pass g takes
        // block row bi = g / 4 and registers 4 (g % 4) .. + 3.  The epilogue
        // reads its inputs at coordinates clamped into the output (values
        // past it are not stored).
        s += "        #pragma unroll\n        for (int g = 0; g < 8; ++g) {\n";
        s += "            const int bi = g >> 2, vb = (g & 3) * 4;\n";
        s += "            #pragma unroll\n            for (int bj = 0; bj < 2; ++bj)\n";
        s += "                #pragma unroll\n                for (int q = 0; q < 4; ++q) {\n";
        s += "                    const idx_t q0 = m0 + 64 * wm + 32 * bi + 8 * (g & 3) + 4 * h + q;\n";
        s += "                    const idx_t q1 = (idx_t)(t0 + t) * " + std::to_string(tile_cols) + " + 64 * wn + 32 * bj + li;\n";
        s += "                    const idx_t e0 = q0 < " + M + " ? q0 : (idx_t)" + std::to_string(r.m - 1) + ";\n";
        s += "                    const idx_t e1 = q1 < " + N + " ? q1 : (idx_t)" + std::to_string(r.n - 1) + ";\n";
        s += "                    (void)e0; (void)e1;\n";
        s += "                    const float acc_v = acc[bi][bj][vb + q];\n";
        {
            std::string body;
            emitter em(*r.expr, body, 1);
            em.indent = "                    ";
            em.declare_roots({r.epilogue});
            const std::vector<std::string> names =
                r.batched ? std::vector<std::string>{"qb", "e0", "e1"} : std::vector<std::string>{"e0", "e1"};
            epilogue_emitter(em, r, names, "acc_v");
            const std::string v = em.emit(r.epilogue)[0];
            s += body;
            s += "                    Ws[wave][4 * h + q][32 * bj + li] = " + v + ";\n";
        }
        s += "                }\n";
        // the wave reads its own writes: its LDS operations complete in
        // order, and the wave barrier keeps the compiler from moving the
        // reads above the writes
        s += "            __builtin_amdgcn_wave_barrier();\n";
        s += "            #pragma unroll\n            for (int u = 0; u < 2; ++u) {\n";
        s += "                const int f = lane + 64 * u;\n";
        s += "                const int rr = f >> 4, c4 = f & 15;\n";
        s += "                const idx_t q0 = m0 + 64 * wm + 32 * bi + 8 * (g & 3) + rr;\n";
        s += "                const idx_t q1 = (idx_t)(t0 + t) * " + std::to_string(tile_cols) + " + 64 * wn + 4 * c4;\n";
        s += "                const porch_v4f x = *reinterpret_cast<const porch_v4f*>(&Ws[wave][rr][4 * c4]);\n";
        const std::string row = r.batched ? "(qb * " + M + " + q0)" : "q0";
        s += "                if (q0 < " + M + " && q1 < " + N + ")\n";
        s += "                    *reinterpret_cast<porch_v4f*>(out + " + row + " * " + N + " + q1) = x;\n";
        s += "            }\n";
        s += "            __builtin_amdgcn_wave_barrier();\n";
        s += "        }\n";
        s += "        __syncthreads();\n";
        s += "    }\n}\n";
        return kc;
    }

} // namespace porch::cg
