// Rank-2 (and batched) matmul with a fused elementwise epilogue.
//
// The reference emits a per-output K loop inside the elementwise kernel
// (reference src/tensor.cpp:684-721).  Here small products use the same
// one-output-per-lane K loop (sequential fp32 sum, exactly the reference's
// order), and large ones use LDS-tiled fp32 MFMA.  A batched product runs
// the same kernels over (batch entry, tile) pairs, each entry's operands
// offset by their batch strides.

#include "emit_gemm.hpp"

#include <algorithm>
#include <stdexcept>

namespace porch::cg {

    std::string operand_index(const gemm_operand& op, const std::string& row, const std::string& col,
                              const std::string& batch) {
        std::string s = std::to_string(op.offset);
        if (!batch.empty() && op.stride_batch != 0)
            s += " + (idx_t)(" + batch + ") * " + std::to_string(op.stride_batch);
        s += " + (idx_t)(" + row + ") * " + std::to_string(op.stride_row);
        s += " + (idx_t)(" + col + ") * " + std::to_string(op.stride_col);
        return s;
    }

    void epilogue_emitter(emitter& em, const gemm_request& r, const std::vector<std::string>& names,
                          const std::string& acc) {
        const kexpr& k = *r.expr;
        // the names by value: callers may pass a temporary
        em.load = [&k, names](int id) {
            const knode& n = k.at(id);
            return std::vector<std::string>{"a" + std::to_string(n.slot) + "[" + index_text(n.index, names) + "]"};
        };
        em.condition = [names](const kcond& c) { return index_text(c.lhs, names) + " < " + std::to_string(c.bound); };
        em.row_value = [acc](int) { return acc; };
    }

    namespace {

        kernel_code emit_gemm_scalar(const gemm_request& r) {
            kernel_code kc;
            kc.kind = "gemm.scalar";
            kc.name = "porch_gemm";
            kc.n_slots = r.n_slots;
            kc.block = 256;
            const int64_t outputs = r.batch * r.m * r.n;
            kc.grid_x = static_cast<unsigned>(
                std::clamp<int64_t>((outputs + 255) / 256, 1, int64_t{1} << 22)
            );
            const char* T = r.width.type();
            const std::vector<std::string> names =
                r.batched ? std::vector<std::string>{"qb", "q0", "q1"}
                          : std::vector<std::string>{"q0", "q1"};
            std::string& s = kc.source;
            s = kernel_prologue(r.n_slots, T);
            s += "extern \"C\" __global__ void __launch_bounds__(256) porch_gemm(" +
                 kernel_params(r.n_slots) + ") {\n";
            s += "    for (idx_t o = (idx_t)blockIdx.x * 256 + threadIdx.x; o < " +
                 std::to_string(outputs) + "; o += (idx_t)gridDim.x * 256) {\n";
            if (r.batched) {
                s += "        const idx_t qb = o / " + std::to_string(r.m * r.n) + ";\n";
                s += "        const idx_t q0 = (o / " + std::to_string(r.n) + ") % " +
                     std::to_string(r.m) + ";\n";
            }
            else {
                s += "        const idx_t q0 = o / " + std::to_string(r.n) + ";\n";
            }
            s += "        const idx_t q1 = o % " + std::to_string(r.n) + ";\n";
            const std::string batch = r.batched ? "qb" : "";
            s += "        float acc = 0.0f;\n";
            s += "        for (idx_t kk = 0; kk < " + std::to_string(r.k) + "; ++kk) {\n";
            s += "            acc += a" + std::to_string(r.a.slot) + "[" +
                 operand_index(r.a, "q0", "kk", batch) + "] * a" + std::to_string(r.b.slot) + "[" +
                 operand_index(r.b, "kk", "q1", batch) + "];\n";
            s += "        }\n";
            std::string body;
            emitter em(*r.expr, body, 1);
            em.indent = "        ";
            em.declare_roots({r.epilogue});
            epilogue_emitter(em, r, names, "acc");
            const std::string v = em.emit(r.epilogue)[0];
            s += body;
            s += "        out[o] = " + v + ";\n";
            s += "    }\n}\n";
            return kc;
        }

        // ----------------------------------------------------------------
        // LDS-tiled fp32 MFMA: 128x128 tile per 256-thread workgroup, each
        // wave a 64x64 quadrant as 2x2 v_mfma_f32_32x32x2f32 blocks, K in
        // steps of 16 through double-buffered LDS (one barrier per step).
        // Operand lane layout (checked on gfx950): A[i = l%32][k = l/32],
        // B[k = l/32][j = l%32]; accumulator register v of lane l holds
        // C[8*(v/4) + 4*(l/32) + v%4][l%32].
        //
        // LDS holds each operand tile as X[k % 2][i][k / 2] (i = m for A, n
        // for B; row pitch 12 floats): lane l of the MFMAs of one K step
        // needs k = 2s + l/32 for s = 0..7, which is one contiguous row of
        // eight floats, read with two 128-bit LDS loads instead of eight
        // 32-bit ones.  With the 12-float pitch, eight consecutive rows
        // cover all 32 banks exactly once per 128-bit access.
        // ----------------------------------------------------------------
        constexpr int BM = 128;
        constexpr int BN = 128;
        constexpr int BK = 16;
        constexpr int PITCH = 12;

        struct operand_layout {
            bool k_major;      // contiguous along k (A row-major, B col-major)
            bool vector;       // 128-bit global loads are aligned and in bounds
        };

        // "a && b" of the bounds tests that can fail (a tile dimension that
        // divides its extent needs none); "true" when none can.
        std::string in_bounds(const std::string& i_test, bool i_exact, const std::string& k_test,
                              bool k_exact) {
            std::string t;
            if (!i_exact) t = i_test;
            if (!k_exact) t += (t.empty() ? "" : " && ") + k_test;
            return t.empty() ? "true" : t;
        }

        // Loads of one operand tile into registers r{X}[8] and their stores
        // to LDS in the X[k % 2][i][k / 2] layout.
        void operand_code(std::string& load, std::string& store, const char* X,
                          const gemm_operand& op, bool is_a, int64_t rows_ext,
                          int64_t k_ext, const operand_layout& lay, int tile_rows) {
            const bool i_exact = rows_ext % tile_rows == 0;
            // float4 chunks per thread: tile_rows x 16 floats over 256 threads
            const std::string chunks = std::to_string(tile_rows / 64);
            const bool k_exact = k_ext % BK == 0;
            // i: the m (A) or n (B) coordinate; stride_i / stride_k in memory
            const int64_t stride_i = is_a ? op.stride_row : op.stride_col;
            const int64_t stride_k = is_a ? op.stride_col : op.stride_row;
            const std::string base = std::string(is_a ? "A" : "B");
            const std::string i0 = is_a ? "m0" : "n0";
            const std::string x{X};
            if (lay.k_major) {
                // chunk c: i = c >> 2, k = (c & 3) * 4 .. +3
                load += "    #pragma unroll\n    for (int i = 0; i < " + chunks + "; ++i) {\n";
                load += "        const int c = tid + i * 256;\n";
                load += "        const int ii = c >> 2;\n        const int kq = (c & 3) * 4;\n";
                load += "        const idx_t gi = " + i0 + " + ii;\n";
                load += "        const idx_t gk = k0 + kq;\n";
                if (lay.vector) {
                    load += "        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);\n";
                    load += "        if (" + in_bounds("gi < " + std::to_string(rows_ext), i_exact,
                                                 "gk < " + std::to_string(k_ext), k_exact) +
                            ") v = *reinterpret_cast<const float4*>(" +
                            base + " + gi * " + std::to_string(stride_i) + " + gk);\n";
                    load += "        r" + x + "[i * 4 + 0] = v.x; r" + x + "[i * 4 + 1] = v.y; r" +
                            x + "[i * 4 + 2] = v.z; r" + x + "[i * 4 + 3] = v.w;\n";
                }
                else {
                    load += "        #pragma unroll\n        for (int e = 0; e < 4; ++e)\n";
                    load += "            r" + x + "[i * 4 + e] = (" +
                            in_bounds("gi < " + std::to_string(rows_ext), i_exact,
                                      "gk + e < " + std::to_string(k_ext), k_exact) +
                            ") ? " + base + "[gi * " + std::to_string(stride_i) + " + (gk + e) * " +
                            std::to_string(stride_k) + "] : 0.0f;\n";
                }
                load += "    }\n";
                // k = kq, kq+2 go to parity 0, k = kq+1, kq+3 to parity 1
                store += "    #pragma unroll\n    for (int i = 0; i < " + chunks + "; ++i) {\n";
                store += "        const int c = tid + i * 256;\n";
                store += "        const int ii = c >> 2;\n        const int kq = (c & 3) * 4;\n";
                store += "        *reinterpret_cast<float2*>(&" + x + "s[nb][0][ii][kq >> 1]) = make_float2(r" +
                         x + "[i * 4 + 0], r" + x + "[i * 4 + 2]);\n";
                store += "        *reinterpret_cast<float2*>(&" + x + "s[nb][1][ii][kq >> 1]) = make_float2(r" +
                         x + "[i * 4 + 1], r" + x + "[i * 4 + 3]);\n";
                store += "    }\n";
            }
            else {
                // contiguous along i: chunk c: k = c & 15, i = (c >> 4) * 4 .. +3
                // (a wave reads 16 rows x 64 bytes; its LDS writes spread
                // over the banks instead of hitting two of them)
                load += "    #pragma unroll\n    for (int i = 0; i < " + chunks + "; ++i) {\n";
                load += "        const int c = tid + i * 256;\n";
                load += "        const int kk = c & 15;\n        const int iq = (c >> 4) * 4;\n";
                load += "        const idx_t gi = " + i0 + " + iq;\n";
                load += "        const idx_t gk = k0 + kk;\n";
                if (lay.vector) {
                    load += "        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);\n";
                    load += "        if (" + in_bounds("gi < " + std::to_string(rows_ext), i_exact,
                                                 "gk < " + std::to_string(k_ext), k_exact) +
                            ") v = *reinterpret_cast<const float4*>(" +
                            base + " + gk * " + std::to_string(stride_k) + " + gi);\n";
                    load += "        r" + x + "[i * 4 + 0] = v.x; r" + x + "[i * 4 + 1] = v.y; r" +
                            x + "[i * 4 + 2] = v.z; r" + x + "[i * 4 + 3] = v.w;\n";
                }
                else {
                    load += "        #pragma unroll\n        for (int e = 0; e < 4; ++e)\n";
                    load += "            r" + x + "[i * 4 + e] = (" +
                            in_bounds("gi + e < " + std::to_string(rows_ext), i_exact,
                                      "gk < " + std::to_string(k_ext), k_exact) +
                            ") ? " + base + "[(gi + e) * " + std::to_string(stride_i) + " + gk * " +
                            std::to_string(stride_k) + "] : 0.0f;\n";
                }
                load += "    }\n";
                store += "    #pragma unroll\n    for (int i = 0; i < " + chunks + "; ++i) {\n";
                store += "        const int c = tid + i * 256;\n";
                store += "        const int kk = c & 15;\n        const int iq = (c >> 4) * 4;\n";
                store += "        #pragma unroll\n        for (int e = 0; e < 4; ++e) " + x +
                         "s[nb][kk & 1][iq + e][kk >> 1] = r" + x + "[i * 4 + e];\n";
                store += "    }\n";
            }
        }

        operand_layout layout_of(const gemm_operand& op, bool is_a, int64_t rows_ext,
                                 int64_t k_ext) {
            const int64_t stride_i = is_a ? op.stride_row : op.stride_col;
            const int64_t stride_k = is_a ? op.stride_col : op.stride_row;
            operand_layout lay;
            lay.k_major = stride_k == 1 && !(stride_i == 1 && stride_k != 1);
            if (stride_k != 1 && stride_i != 1) lay.k_major = true; // strided: scalar path
            if (lay.k_major)
                lay.vector = stride_k == 1 && op.offset % 4 == 0 && stride_i % 4 == 0 &&
                             k_ext % 4 == 0;
            else
                lay.vector = op.offset % 4 == 0 && stride_k % 4 == 0 && rows_ext % 4 == 0;
            // every batch entry's base must keep the 16-byte alignment
            lay.vector = lay.vector && op.stride_batch % 4 == 0;
            return lay;
        }

        kernel_code emit_gemm_mfma(const gemm_request& r) {
            const int64_t tiles_n = (r.n + BN - 1) / BN;
            const int64_t steps = (r.k + BK - 1) / BK;
            const operand_layout la = layout_of(r.a, true, r.m, r.k);
            const operand_layout lb = layout_of(r.b, false, r.n, r.k);
            const bool scheduled = la.vector && lb.vector;
            // LDS stores of the next K-slice per wave, and whether they and
            // the global loads fit between a step's MFMAs
            auto ds_writes_of = [&](int rows) {
                return (la.k_major ? 2 : 4) * (rows / 64) + (lb.k_major ? 2 : 4) * (BN / 64);
            };
            auto interleaves = [&](int rows) {
                return scheduled && 4 * (rows / 64 + BN / 64) + 4 + ds_writes_of(rows) <= (BK / 2) * (rows / 64) * 2;
            };
            // A short K (at most 4 steps, K <= 64) with more tiles than
            // resident workgroups (two per compute unit): the output stores
            // cost about as much as the MFMAs, and a workgroup that computes,
            // then stores, leaves the MFMA units idle while its stores drain.
            // Persistent workgroups walk the tiles instead, keep the previous
            // tile's accumulators and store one slice of them during each
            // K-step of the current tile (the last steps also load the next
            // tile's first K-slices), so the stores overlap the MFMAs
            // (measured 9-20% faster at K = 16 to 64).  From 6 steps on it
            // stops paying (K = 96 and 128: 5-8% slower): the 128-row tiles
            // it needs cost more LDS reads per MFMA, and the stores are a
            // smaller share of the time.  The stores go through a buffer
            // resource whose range check drops out-of-range lanes (offset
            // 2^31), which keeps them branch-free.
            // Two accumulator sets need 128-row tiles (a wave's 64 x 64 block)
            // to stay within the register budget of two workgroups per
            // compute unit.
            const int64_t resident = static_cast<int64_t>(std::max(r.compute_units, 1)) * 2;
            const int64_t out_elems = r.batch * r.m * r.n;
            const bool persistent = r.k_chunks == 1 && interleaves(BM) &&
                                    ((r.m + BM - 1) / BM) * tiles_n * r.batch > resident && steps <= 4 &&
                                    out_elems < (int64_t{1} << 29);
            // Split over K (k_chunks > 1): workgroup w computes chunk
            // w % k_chunks of tile w / k_chunks, steps_c K-steps from kbase,
            // and stores its accumulators unchanged as partial products.
            const int64_t kc_n = r.k_chunks;
            if (kc_n > 1 && steps % kc_n != 0) throw std::logic_error("emit_gemm: K chunks must divide the K-steps");
            const int64_t steps_c = steps / kc_n;
            // Otherwise 256-row tiles (each wave 128 x 64: 4 x 2 MFMA blocks)
            // halve the LDS reads per MFMA and the B re-reads; used while
            // they still give every compute unit a tile (measured 2.7%
            // faster at 4096^3).
            const int bm = persistent ? BM
                           : (r.m >= 256 && ((r.m + 255) / 256) * tiles_n * r.batch >= r.compute_units) ? 256
                                                                                                        : BM;
            const int ib = bm / 64; // 32-row MFMA blocks per wave
            const int64_t tiles_m = (r.m + bm - 1) / bm;
            const int64_t tiles = tiles_m * tiles_n;
            const int64_t total = tiles * r.batch; // (batch entry, tile) pairs
            const std::string IB = std::to_string(ib);
            const std::string HALF = std::to_string(bm / 2);
            const int vmem = bm / 64 + BN / 64;
            const int mfmas = (BK / 2) * ib * 2;
            const int ds_writes = ds_writes_of(bm);
            const bool interleave = interleaves(bm);
            kernel_code kc;
            kc.kind = "gemm.mfma";
            kc.name = "porch_gemm";
            kc.n_slots = r.n_slots;
            kc.block = 256;
            kc.grid_x = static_cast<unsigned>(persistent ? resident : total * kc_n);
            const char* T = r.width.type();
            std::string& s = kc.source;
            s = kernel_prologue(r.n_slots, T);
            s += "typedef float floatx16 __attribute__((ext_vector_type(16)));\n";
            // Two workgroups per compute unit (two waves per SIMD): the
            // register budget within which the accumulators stay in VGPRs.
            s += "extern \"C\" __global__ void __launch_bounds__(256, 2) porch_gemm(" +
                 kernel_params(r.n_slots) + ") {\n";
            s += "    __shared__ __attribute__((aligned(16))) float As[2][2][" + std::to_string(bm) + "][" +
                 std::to_string(PITCH) + "];\n";
            s += "    __shared__ __attribute__((aligned(16))) float Bs[2][2][" + std::to_string(BN) + "][" +
                 std::to_string(PITCH) + "];\n";
            s += "    const int tid = threadIdx.x;\n";
            s += "    const int lane = tid & 63;\n";
            s += "    const int wave = tid >> 6;\n";
            s += "    const int wm = wave >> 1;\n    const int wn = wave & 1;\n";
            // Workgroups are dispatched round-robin over the 8 XCDs; give
            // each XCD a contiguous band of tile rows so its L2 holds them.
            // (For a batched product the bands run over (entry, tile) pairs,
            // entry-major, so an XCD holds whole entries where it can.)
            // Tile `raw` (a workgroup index, or a persistent workgroup's
            // running index) -> m0, n0 (and qb), A, B with name suffix `sx`.
            // With a grid that is a multiple of 8, raw % 8 is the XCD.
            auto decode = [&](const std::string& raw, const std::string& sx, const std::string& ind) {
                std::string d;
                const std::string lin = r.batched ? "lin" + sx : "tile" + sx;
                const std::string cast = raw != "blockIdx.x" ? "(int)" : ""; // an idx_t running index
                if (total % 8 == 0)
                    d += ind + "const int " + lin + " = " + cast + "(" + raw + " % 8) * " +
                         std::to_string(total / 8) + " + " + (cast.empty() ? raw + " / 8" : cast + "(" + raw + " / 8)") +
                         ";\n";
                else
                    d += ind + "const int " + lin + " = " + cast + raw + ";\n";
                if (r.batched) {
                    d += ind + "const idx_t qb" + sx + " = " + lin + " / " + std::to_string(tiles) + ";\n";
                    d += ind + "const int tile" + sx + " = " + lin + " % " + std::to_string(tiles) + ";\n";
                }
                d += ind + "const idx_t m0" + sx + " = (idx_t)(tile" + sx + " / " + std::to_string(tiles_n) +
                     ") * " + std::to_string(bm) + ";\n";
                d += ind + "const idx_t n0" + sx + " = (idx_t)(tile" + sx + " % " + std::to_string(tiles_n) +
                     ") * " + std::to_string(BN) + ";\n";
                auto base = [&](const gemm_operand& op) {
                    std::string b = "a" + std::to_string(op.slot) + " + " + std::to_string(op.offset);
                    if (r.batched && op.stride_batch != 0)
                        b += " + qb" + sx + " * " + std::to_string(op.stride_batch);
                    return b;
                };
                d += ind + "const float* __restrict__ A" + sx + " = " + base(r.a) + ";\n";
                d += ind + "const float* __restrict__ B" + sx + " = " + base(r.b) + ";\n";
                return d;
            };
            if (!persistent && kc_n == 1) s += decode("blockIdx.x", "", "    ");
            if (kc_n > 1) {
                s += "    const idx_t ks = (idx_t)blockIdx.x % " + std::to_string(kc_n) + ";\n";
                s += "    const idx_t kbase = ks * " + std::to_string(steps_c * BK) + ";\n";
                s += "    const idx_t wt = (idx_t)blockIdx.x / " + std::to_string(kc_n) + ";\n";
                s += decode("wt", "", "    ");
            }
            const std::string kb = kc_n > 1 ? "kbase + " : "";
            // Even step counts of a persistent kernel load two K-slices
            // ahead, through two register sets: a slice's LDS store then
            // waits only for loads issued a step earlier, behind the output
            // stores of two steps before, not of the step before.
            const bool ahead2 = persistent && steps % 2 == 0;
            auto in_set = [](std::string code, int set) {
                for (const char* name : {"rA[", "rB["}) {
                    const std::string from{name};
                    const std::string to = from.substr(0, 2) + std::to_string(set) + "[";
                    for (size_t at = code.find(from); at != std::string::npos; at = code.find(from, at + to.size()))
                        code.replace(at, from.size(), to);
                }
                return code;
            };
            if (ahead2)
                for (int set = 0; set < 2; ++set)
                    s += "    float rA" + std::to_string(set) + "[" + std::to_string(4 * (bm / 64)) + "];\n    float rB" +
                         std::to_string(set) + "[8];\n";
            else
                s += "    float rA[" + std::to_string(4 * (bm / 64)) + "];\n    float rB[8];\n";
            s += "    floatx16 acc[" + IB + "][2];\n";
            const std::string zero_acc =
                "    #pragma unroll\n    for (int i = 0; i < " + IB + "; ++i)\n"
                "        #pragma unroll\n        for (int j = 0; j < 2; ++j)\n"
                "            #pragma unroll\n            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;\n";
            std::string load_a, store_a, load_b, store_b;
            operand_code(load_a, store_a, "A", r.a, true, r.m, r.k, la, bm);
            operand_code(load_b, store_b, "B", r.b, false, r.n, r.k, lb, BN);
            if (!persistent) s += zero_acc;
            // prologue: the first K-slice of the (first) tile
            s += "    {\n";
            if (persistent) s += decode("blockIdx.x", "", "        ");
            s += "        const idx_t k0 = " + (kc_n > 1 ? std::string("kbase") : std::string("0")) +
                 ";\n        const int nb = 0;\n";
            if (ahead2) {
                s += in_set(load_a + load_b + store_a + store_b, 0);
                // and its second, held in registers
                s += "        {\n        const idx_t k0 = " + std::to_string(BK) + ";\n";
                s += in_set(load_a + load_b, 1) + "        }\n";
            }
            else {
                s += load_a + load_b + store_a + store_b;
            }
            s += "    }\n    __syncthreads();\n";
            // Epilogue for the accumulator blocks u = 2 bi + bj in [lo, hi)
            // of `accn` at tile origin (m0n, n0n, qbn).  Buffered: branch-free,
            // with clamped coordinates for the epilogue's own loads and the
            // store offset set out of the buffer's range for lanes outside
            // the output.
            auto epilogue = [&](const std::string& accn, const std::string& m0n, const std::string& n0n,
                                const std::string& qbn, int lo, int hi, bool buffered) {
                std::string e;
                if (lo >= hi) return e;
                const std::string M = std::to_string(r.m), N = std::to_string(r.n);
                if (buffered) {
                    e += "    #pragma unroll\n    for (int u = " + std::to_string(lo) + "; u < " + std::to_string(hi) +
                         "; ++u)\n";
                    e += "    #pragma unroll\n    for (int v = 0; v < 16; ++v) {\n";
                    e += "        const int bi = u >> 1;\n        const int bj = u & 1;\n";
                }
                else {
                    e += "    #pragma unroll\n    for (int bi = 0; bi < " + IB + "; ++bi)\n";
                    e += "    #pragma unroll\n    for (int bj = 0; bj < 2; ++bj)\n";
                    e += "    #pragma unroll\n    for (int v = 0; v < 16; ++v) {\n";
                }
                e += "        const idx_t q0 = " + m0n + " + wm * " + HALF +
                     " + bi * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);\n";
                e += "        const idx_t q1 = " + n0n + " + wn * 64 + bj * 32 + (lane & 31);\n";
                std::string body;
                emitter em(*r.expr, body, 1);
                std::vector<std::string> names;
                if (buffered) {
                    e += "        const bool inb = q0 < " + M + " && q1 < " + N + ";\n";
                    e += "        const idx_t e0 = inb ? q0 : (idx_t)0;\n";
                    e += "        const idx_t e1 = inb ? q1 : (idx_t)0;\n";
                    e += "        const float acc_v = " + accn + "[bi][bj][v];\n";
                    em.indent = "        ";
                    names = r.batched ? std::vector<std::string>{qbn, "e0", "e1"}
                                      : std::vector<std::string>{"e0", "e1"};
                }
                else {
                    e += "        if (q0 < " + M + " && q1 < " + N + ") {\n";
                    e += "            const float acc_v = " + accn + "[bi][bj][v];\n";
                    em.indent = "            ";
                    names = r.batched ? std::vector<std::string>{qbn, "q0", "q1"}
                                      : std::vector<std::string>{"q0", "q1"};
                }
                em.declare_roots({r.epilogue});
                epilogue_emitter(em, r, names, "acc_v");
                const std::string v = em.emit(r.epilogue)[0];
                e += body;
                const std::string i0 = buffered ? "e0" : "q0", i1 = buffered ? "e1" : "q1";
                const std::string at = r.batched ? "(" + qbn + " * " + M + " + " + i0 + ") * " + N + " + " + i1
                                                 : i0 + " * " + N + " + " + i1;
                if (buffered) {
                    e += "        const int off = inb ? (int)((" + at + ") * 4) : (int)0x80000000;\n";
                    e += "        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, " + v +
                         "), orsrc, off, 0, 0);\n";
                    e += "    }\n";
                }
                else if (kc_n > 1) {
                    e += "            out[ks * " + std::to_string(out_elems) + " + " + at + "] = acc_v;\n        }\n    }\n";
                }
                else {
                    e += "            out[" + at + "] = " + v + ";\n        }\n    }\n";
                }
                return e;
            };
            if (persistent) {
                s += "    const auto orsrc = __builtin_amdgcn_make_buffer_rsrc(out, 0, " +
                     std::to_string(out_elems * 4) + ", 0x00020000);\n";
                s += "    floatx16 accP[" + IB + "][2];\n";
                s += "    #pragma unroll\n    for (int i = 0; i < " + IB + "; ++i)\n";
                s += "        #pragma unroll\n        for (int j = 0; j < 2; ++j)\n";
                s += "            #pragma unroll\n            for (int v = 0; v < 16; ++v) accP[i][j][v] = 0.0f;\n";
                // the first tile has no predecessor: a row origin past the
                // output masks every lane of its slices
                s += "    idx_t m0p = " + std::to_string(r.m) + ";\n    idx_t n0p = 0;\n";
                if (r.batched) s += "    idx_t qbp = 0;\n";
                if (steps % 2 != 0) s += "    int phase = 0;\n";
                s += "    for (idx_t rr = blockIdx.x; rr < " + std::to_string(total) + "; rr += gridDim.x) {\n";
                s += decode("rr", "c", "    ");
                s += "    const idx_t rn = rr + gridDim.x < " + std::to_string(total) + " ? rr + gridDim.x : rr;\n";
                s += decode("rn", "x", "    ");
            }
            if (persistent) s += zero_acc;
            // With both operands on the 128-bit path the next tile's global
            // loads and LDS stores are issued in the same block as the
            // MFMAs, so the scheduler can interleave both with them (the last
            // step reloads its own tile, in bounds, into the idle buffer, or
            // loads a persistent workgroup's next tile); otherwise they are
            // skipped on the last step.
            std::string head;
            if (persistent) {
                head += steps % 2 != 0 ? "        const int cb = (phase + t) & 1;\n" : "        const int cb = t & 1;\n";
                head += "        const int nb = cb ^ 1;\n";
                head += "        const bool to_next = t + 1 == " + std::to_string(steps) + ";\n";
                head += "        const idx_t k0 = to_next ? (idx_t)0 : (idx_t)(t + 1) * " + std::to_string(BK) + ";\n";
                head += "        {\n";
                head += "        const idx_t m0 = to_next ? m0x : m0c;\n";
                head += "        const idx_t n0 = to_next ? n0x : n0c;\n";
                head += "        const float* __restrict__ A = to_next ? Ax : Ac;\n";
                head += "        const float* __restrict__ B = to_next ? Bx : Bc;\n";
                head += load_a + load_b + "        }\n";
            }
            else {
                head += "        const int cb = t & 1;\n";
                head += "        const int nb = cb ^ 1;\n";
                if (interleave) {
                    head += "        const idx_t k0 = " + kb + "(idx_t)(t + 1 < " + std::to_string(steps_c) +
                            " ? t + 1 : t) * " + std::to_string(BK) + ";\n";
                    head += "        {\n" + load_a + load_b + "        }\n";
                }
                else {
                    head += "        const idx_t k0 = " + kb + "(idx_t)(t + 1) * " + std::to_string(BK) + ";\n";
                    head += "        const bool more = t + 1 < " + std::to_string(steps_c) + ";\n";
                    head += "        if (more) {\n" + load_a + load_b + "        }\n";
                }
            }
            std::string step;
            // this lane's k parity and row inside each 32-row block
            step += "        const int h = lane >> 5;\n";
            step += "        const int li = lane & 31;\n";
            step += "        float av[" + IB + "][8];\n        float bv[2][8];\n";
            step += "        #pragma unroll\n        for (int b = 0; b < " + IB + "; ++b) {\n";
            step += "            const float4 al = *reinterpret_cast<const float4*>(&As[cb][h][wm * " + HALF +
                    " + b * 32 + li][0]);\n";
            step += "            const float4 ah = *reinterpret_cast<const float4*>(&As[cb][h][wm * " + HALF +
                    " + b * 32 + li][4]);\n";
            step += "            av[b][0] = al.x; av[b][1] = al.y; av[b][2] = al.z; av[b][3] = al.w;\n";
            step += "            av[b][4] = ah.x; av[b][5] = ah.y; av[b][6] = ah.z; av[b][7] = ah.w;\n";
            step += "        }\n";
            step += "        #pragma unroll\n        for (int b = 0; b < 2; ++b) {\n";
            step += "            const float4 bl = *reinterpret_cast<const float4*>(&Bs[cb][h][wn * 64 + b * 32 + li][0]);\n";
            step += "            const float4 bh = *reinterpret_cast<const float4*>(&Bs[cb][h][wn * 64 + b * 32 + li][4]);\n";
            step += "            bv[b][0] = bl.x; bv[b][1] = bl.y; bv[b][2] = bl.z; bv[b][3] = bl.w;\n";
            step += "            bv[b][4] = bh.x; bv[b][5] = bh.y; bv[b][6] = bh.z; bv[b][7] = bh.w;\n";
            step += "        }\n";
            step += "        #pragma unroll\n";
            step += "        for (int st = 0; st < " + std::to_string(BK / 2) + "; ++st)\n";
            step += "            #pragma unroll\n            for (int i = 0; i < " + IB + "; ++i)\n";
            step += "                #pragma unroll\n                for (int j = 0; j < 2; ++j)\n";
            step += "                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][st], bv[j][st], acc[i][j], 0, 0, 0);\n";
            // the LDS stores of the next slice, then the schedule; the
            // two-ahead persistent form picks its register set per step
            const std::string step_compute = step;
            step.clear();
            const int stores_per_step = static_cast<int>((2 * ib + steps - 1) / steps) * 16;
            if (scheduled) {
                // Instruction order for the scheduler: the 128-bit LDS reads
                // first, then one of the next tile's global loads after every
                // four MFMAs, so those loads leave early and their latency
                // hides under the remaining MFMAs (measured 7% faster at
                // 4096^3 than the compiler's own order, which issued them
                // after nearly all MFMAs).  Then, after a gap of MFMAs that
                // covers the loads' latency, one LDS store of the next tile
                // after each MFMA, instead of all of them after the last
                // MFMA (another 4% at 4096^3).  With the previous tile's
                // stores in the same block the load groups name reads only
                // (0x040); the stores fill in around them.
                const int ds_reads = 2 * ib + 4;
                const std::string vmem_mask = persistent ? "0x040" : "0x020";
                step += "        __builtin_amdgcn_sched_group_barrier(0x100, " + std::to_string(ds_reads) + ", 0);\n";
                for (int g = 0; g < vmem; ++g) {
                    step += "        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);\n";
                    step += "        __builtin_amdgcn_sched_group_barrier(" + vmem_mask + ", 1, 0);\n";
                }
                // the previous tile's output stores after this step's loads
                if (ahead2)
                    step += "        __builtin_amdgcn_sched_group_barrier(0x080, " + std::to_string(stores_per_step) +
                            ", 0);\n";
                int rest = mfmas - 4 * vmem;
                if (interleave) {
                    const int gap = std::min(16, rest - ds_writes);
                    step += "        __builtin_amdgcn_sched_group_barrier(0x008, " + std::to_string(gap) + ", 0);\n";
                    for (int g = 0; g < ds_writes; ++g) {
                        step += "        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);\n";
                        step += "        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);\n";
                    }
                    rest -= gap + ds_writes;
                }
                if (rest > 0)
                    step += "        __builtin_amdgcn_sched_group_barrier(0x008, " + std::to_string(rest) + ", 0);\n";
            }
            if (!interleave) step += "        if (more) {\n" + store_a + store_b + "        }\n";
            step += "        __syncthreads();\n";
            const std::string step_schedule = step;
            auto step_of = [&](const std::string& lds_stores) {
                return step_compute + (interleave ? "        {\n" + lds_stores + "        }\n" : std::string()) +
                       step_schedule;
            };
            step = step_of(store_a + store_b);
            if (persistent) {
                // steps unrolled, so each stores a fixed slice of the
                // previous tile's accumulator blocks
                for (int64_t t = 0; t < steps; ++t) {
                    const int lo = static_cast<int>(t * 2 * ib / steps);
                    const int hi = static_cast<int>((t + 1) * 2 * ib / steps);
                    s += "    {\n        const int t = " + std::to_string(t) + ";\n";
                    if (ahead2) {
                        // load slice t + 2 (of this tile or the next) into
                        // set t % 2; store slice t + 1 from the other set
                        const bool next = t + 2 >= steps;
                        const std::string sx = next ? "x" : "c";
                        s += "        const int cb = t & 1;\n        const int nb = cb ^ 1;\n        {\n";
                        s += "        const idx_t k0 = " + std::to_string(((t + 2) % steps) * BK) + ";\n";
                        s += "        const idx_t m0 = m0" + sx + ";\n        const idx_t n0 = n0" + sx + ";\n";
                        s += "        const float* __restrict__ A = A" + sx + ";\n";
                        s += "        const float* __restrict__ B = B" + sx + ";\n";
                        s += in_set(load_a + load_b, static_cast<int>(t % 2)) + "        }\n";
                        s += epilogue("accP", "m0p", "n0p", "qbp", lo, hi, true);
                        s += step_of(in_set(store_a + store_b, static_cast<int>((t + 1) % 2))) + "    }\n";
                    }
                    else {
                        s += head;
                        s += epilogue("accP", "m0p", "n0p", "qbp", lo, hi, true);
                        s += step + "    }\n";
                    }
                }
                if (steps % 2 != 0) s += "    phase += " + std::to_string(steps) + ";\n";
                s += "    #pragma unroll\n    for (int i = 0; i < " + IB + "; ++i)\n";
                s += "        #pragma unroll\n        for (int j = 0; j < 2; ++j) accP[i][j] = acc[i][j];\n";
                s += "    m0p = m0c;\n    n0p = n0c;\n";
                if (r.batched) s += "    qbp = qbc;\n";
                s += "    }\n";
                // the last tile's accumulators
                s += epilogue("accP", "m0p", "n0p", "qbp", 0, 2 * ib, true);
            }
            else {
                s += "    for (int t = 0; t < " + std::to_string(steps_c) + "; ++t) {\n" + head + step + "    }\n";
                s += epilogue("acc", "m0", "n0", "qb", 0, 2 * ib, false);
            }
            s += "}\n";
            return kc;
        }

    } // namespace

    namespace {
        // Small products keep the reference's sequential K loop (their
        // launch is latency-bound anyway); large ones use MFMA, whatever
        // their shape: a tile that covers only a few rows or columns still
        // beats one thread per output running down a long K (the products
        // with one short side that a skinny kernel serves better do not
        // get here).
        bool uses_mfma(const gemm_request& r) { return r.batch * r.m * r.n * r.k >= (int64_t{1} << 18); }
    } // namespace

    kernel_code emit_gemm(const gemm_request& r) {
        return uses_mfma(r) ? emit_gemm_mfma(r) : emit_gemm_scalar(r);
    }

    int64_t gemm_k_chunks(const gemm_request& r) {
        if (!uses_mfma(r)) return 1;
        // 128 x 128 tiles (the tile size of a product too small for 256-row
        // tiles); split K when they leave over half the compute units idle
        // and K is long (1024 or more: a shorter loop finishes within the
        // time of the extra combine launch), into the fewest chunks
        // (dividing the K-steps, each at least 8 of them) that give two
        // workgroups per compute unit.
        const int64_t cus = std::max(r.compute_units, 8);
        const int64_t tiles = ((r.m + BM - 1) / BM) * ((r.n + BN - 1) / BN) * r.batch;
        const int64_t steps = (r.k + BK - 1) / BK;
        if (2 * tiles >= cus || steps < 64) return 1;
        int64_t best = 1;
        for (int64_t d = 2; d * 8 <= steps; ++d) {
            if (steps % d != 0) continue;
            best = d;
            if (tiles * d >= 2 * cus) break;
        }
        return best;
    }

} // namespace porch::cg
