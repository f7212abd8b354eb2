// Softmax-shaped row programs over long rows (more than 32768 values), read
// from memory once.  The row program row_request describes (a max of f, a
// sum of exp(f - that max), an elementwise output) runs with each row split
// into parts of at most 16384 values (as even as whole float4s allow),
// one part per 256-lane workgroup held in registers (up to 64
// values per lane).  Each part publishes its partial (max m, sum s of
// exp(f - m)) as one 64-bit word; every part of a row then combines the
// row's words, M = max of the m and S = sum of s exp(m - M), and writes its
// outputs from registers.  The one-workgroup form (emit_row) reads rows
// past its register cache twice.
//
// Exchange: the partials go to a temporary zeroed before the launch (a
// published word is never zero: its sum is at least 1, or NaN, or its max
// is -FLT_MAX) with relaxed agent-scope 64-bit stores, and wave 0 polls a
// row's words with one lane per part.  No L2 write-back or invalidate is
// issued: the parts of a row run on one XCD (workgroups are dispatched
// round-robin over the 8 XCDs, and a row's parts take workgroup indices
// congruent modulo 8), so they share its L2.  (Release/acquire fences at
// agent scope measured 2-3x slower: they write back and invalidate the
// whole L2 at every exchange.)
//
// Residency: the grid is at most two workgroups per compute unit, which
// the register budget keeps resident together.  Each workgroup holds two
// parts at once and waits for a part's partners only after loading and
// publishing its next part, so a row's parts rarely wait.  Every wait is
// bounded: a workgroup whose partners do not all publish in time (say, the
// GPU is shared and some are not yet resident) computes the row's max and
// sum itself from memory, so the kernel always finishes.
//
// The max stays the reference's: where the order-free maximum may differ
// from the reference's block order (NaN, or a +0 maximum), it is recomputed
// in that order from memory, as in emit_row.
//
// Measured on [512, 262144] (MI355X): the kernel takes the time of a plain
// non-temporal copy of the same 512 MiB each way (about 190 us), and neither
// the exchange (no waits at all), the arithmetic (no exp or division), a
// third register set in flight, four workgroups per compute unit, nor other
// chunk orders change that.

#include "codegen.hpp"
#include "emit_expr.hpp"

#include <algorithm>
#include <functional>
#include <memory>
#include <set>
#include <stdexcept>

namespace porch::cg {
    namespace {

        // At most 16 chunks of 1024 values per part (64 values per lane).
        constexpr int64_t max_chunks = 16;
        // Workgroups resident per compute unit (the register budget allows
        // two at 225 VGPRs).
        constexpr int groups_per_cu = 2;
        // Parts a workgroup holds in registers at once: one being written
        // out, one published, and (with three) one still loading.
        constexpr int register_sets = 2;
        // Polls of a row's partials before a workgroup computes the row
        // itself (each poll is a memory round trip plus a short sleep).
        constexpr int spin_limit = 16384;

        struct split_shape {
            int64_t parts = 0;
            int64_t chunks = 0; // chunks of 1024 values (4 per lane) per part
            int64_t span = 0;   // values per part (a multiple of 4; the last part may hold fewer)
            int64_t groups = 0; // row groups per XCD per round
            int64_t grid = 0;
            int64_t rounds = 0;
            int leaf = -1;
            // The output is exp(f - rv0) / rv1 itself (softmax): the parts
            // whose values all lie within 60 of the row max take the short
            // exp and the reciprocal-based division.
            bool fast_output = false;
        };

        split_shape analyze(const row_request& r) {
            split_shape sh;
            const kexpr& k = *r.expr;
            if (r.reduce_output || r.output < 0 || r.reductions.size() != 2) return sh;
            if (!r.reductions[0].is_max || r.reductions[1].is_max) return sh;
            const size_t rank = r.shape.size();
            const size_t col = rank - 1;
            const int64_t length = r.shape[col];
            // Rows of up to 32768 values are at least as fast in one
            // workgroup (emit_row); beyond, the split form is faster
            // (softmax over 1 GiB of rows of 32772 / 40964 / 49156 / 65536
            // values: 225 / 226 / 231 / 215 -> 206 / 211 / 222 / 194 us).
            if (length <= 32768 || length % 4 != 0) return sh;
            // the online pair: sum of exp(f - rv0) with f the max's producer
            const knode& g = k.at(r.reductions[1].producer);
            if (g.op != kop::exp) return sh;
            const knode& d = k.at(g.a);
            if (d.op != kop::subtract || d.a != r.reductions[0].producer) return sh;
            const knode& rv = k.at(d.b);
            if (rv.op != kop::row_value || rv.row != 0) return sh;
            // one leaf, read with aligned 128-bit loads; no selects
            std::set<int> loads;
            for (const int root : {r.reductions[0].producer, r.reductions[1].producer, r.output}) {
                for (const int id : k.postorder(root)) {
                    const knode& n = k.at(id);
                    if (n.op == kop::select) return sh;
                    if (n.op == kop::load) loads.insert(id);
                }
            }
            if (loads.size() != 1) return sh;
            const knode& leaf = k.at(*loads.begin());
            if (!leaf.index.is_affine || leaf.index.w[col] != 1 || leaf.index.c0 % 4 != 0) return sh;
            for (size_t dd = 0; dd + 1 < rank; ++dd)
                if (leaf.index.w[dd] % 4 != 0) return sh;
            const int64_t parts = (length + max_chunks * 1024 - 1) / (max_chunks * 1024);
            // Parts as even as whole float4s allow, their last chunk partly
            // used: with parts of whole chunks, 49156 values gave parts of
            // 13, 13, 13 and 9 chunks, and every round waited on a 13.
            const int64_t span = (length + 4 * parts - 1) / (4 * parts) * 4;
            const int64_t chunks = (span + 1023) / 1024;
            const int64_t resident = groups_per_cu * static_cast<int64_t>(std::max(r.compute_units, 8));
            const int64_t groups = resident / (8 * parts);
            if (groups < 1) return sh;
            int64_t rows = 1;
            for (size_t dd = 0; dd + 1 < rank; ++dd) rows *= r.shape[dd];
            sh.parts = parts;
            sh.chunks = chunks;
            sh.span = span;
            sh.groups = groups;
            sh.grid = 8 * parts * groups;
            sh.rounds = (rows + 8 * groups - 1) / (8 * groups);
            sh.leaf = *loads.begin();
            const knode& o = k.at(r.output);
            if (o.op == kop::divide && k.at(o.b).op == kop::row_value && k.at(o.b).row == 1) {
                const knode& e = k.at(o.a);
                if (e.op == kop::exp) {
                    const knode& s = k.at(e.a);
                    sh.fast_output = s.op == kop::subtract && s.a == r.reductions[0].producer &&
                                     k.at(s.b).op == kop::row_value && k.at(s.b).row == 0;
                }
            }
            return sh;
        }

    } // namespace

    int64_t row_split_parts(const row_request& r) { return analyze(r).parts; }

    int64_t row_split_temp_floats(const row_request& r) {
        int64_t rows = 1;
        for (size_t d = 0; d + 1 < r.shape.size(); ++d) rows *= r.shape[d];
        return rows * analyze(r).parts * 2;
    }

    kernel_code emit_row_split(const row_request& r) {
        const split_shape sh = analyze(r);
        if (sh.parts == 0 || sh.parts != r.split_parts || r.split_slot < 0)
            throw std::logic_error("emit_row_split: the row program is not a split softmax");
        const kexpr& k = *r.expr;
        const size_t rank = r.shape.size();
        const size_t col = rank - 1;
        const int64_t length = r.shape[col];
        const std::vector<int64_t> row_shape(r.shape.begin(), r.shape.end() - 1);
        int64_t rows = 1;
        for (const int64_t e : row_shape) rows *= e;
        const char* T = r.width.type();
        std::vector<std::string> names;
        for (size_t d = 0; d < rank; ++d) names.push_back("q" + std::to_string(d));
        const std::string qc = names[col];
        const std::string P = std::to_string(sh.parts);
        const std::string L = std::to_string(length);
        const int f = r.reductions[0].producer;
        const knode& leaf = k.at(sh.leaf);
        const std::string leaf_base = "a" + std::to_string(leaf.slot);

        kernel_code kc;
        kc.kind = "row.split";
        kc.name = "porch_row";
        kc.n_slots = r.n_slots;
        kc.block = 256;
        kc.grid_x = static_cast<unsigned>(sh.grid);

        // Values of `root` for chunk j of register set X (the leaf read
        // from X), with row values rv0, rv1 as named in scope.
        auto values = [&](std::string& body, const std::string& X, int root, const std::string& indent,
                          int lanes = 4) {
            auto em = std::make_unique<emitter>(k, body, lanes);
            em->indent = indent;
            em->declare_roots({f, r.reductions[1].producer, r.output});
            em->override_node = [&, X, lanes](int id) -> std::vector<std::string> {
                if (id != sh.leaf) return {};
                std::vector<std::string> v;
                for (int e = 0; e < lanes; ++e) v.push_back(X + "[j][" + std::to_string(e) + "]");
                return v;
            };
            em->load = [](int) -> std::vector<std::string> {
                throw std::logic_error("emit_row_split: a load besides the leaf");
            };
            em->row_value = [](int row) { return "rv" + std::to_string(row); };
            em->condition = [](const kcond&) -> std::string {
                throw std::logic_error("emit_row_split: a select");
            };
            return em->emit(root);
        };
        auto chunk_loop = [&](const std::string& indent, const std::string& body) {
            std::string c = indent + "#pragma unroll\n";
            c += indent + "for (int j = 0; j < " + std::to_string(sh.chunks) + "; ++j) {\n";
            c += indent + "    const " + T + " " + qc + " = (" + T + ")part * " + std::to_string(sh.span) +
                 " + j * 1024 + tl * 4;\n";
            // inside the part (where its span is not whole chunks) and the row
            std::string inside;
            if (sh.span != sh.chunks * 1024) inside = "j * 1024 + tl * 4 < " + std::to_string(sh.span);
            if (sh.parts * sh.span != length)
                inside += std::string(inside.empty() ? "" : " && ") + qc + " < " + L;
            if (inside.empty()) inside = "true";
            c += indent + "    if (" + inside + ") {\n" + body + indent + "    }\n";
            c += indent + "}\n";
            return c;
        };
        auto row_scope = [&](const std::string& round, const std::string& indent) {
            std::string c = indent + "const idx_t row = (idx_t)(" + round + ") * " + std::to_string(8 * sh.groups) +
                            " + xcd * " + std::to_string(sh.groups) + " + group;\n";
            c += indent + "if (row < " + std::to_string(rows) + ") {\n";
            std::vector<bool> needed(row_shape.size(), true);
            c += decompose("row", row_shape, needed, T, indent + "    ");
            return c;
        };
        // The workgroup's value of a lane-level partial: wave butterfly,
        // then the four waves through LDS slot `slot` (each slot is reused
        // only after at least one barrier more).
        auto block_reduce = [&](const std::string& acc, bool is_max, int slot, const std::string& in) {
            const std::string S = std::to_string(slot);
            std::string c = in + acc + " = " + (is_max ? "porch_wave_fmax(" : "porch_wave_sum(") + acc + ");\n";
            c += in + "if (lane == 0) xred[" + S + "][wave] = " + acc + ";\n";
            c += in + "__syncthreads();\n";
            c += in + acc + " = " +
                 (is_max ? "porch_fmax(porch_fmax(xred[" + S + "][0], xred[" + S + "][1]), porch_fmax(xred[" + S +
                               "][2], xred[" + S + "][3]));\n"
                         : "(xred[" + S + "][0] + xred[" + S + "][1]) + (xred[" + S + "][2] + xred[" + S + "][3]);\n");
            return c;
        };

        auto load_item = [&](const std::string& X, const std::string& round) {
            const std::string in = "        ";
            std::string c = "    {\n" + row_scope(round, in);
            std::string body;
            body += in + "        const porch_v4f w = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(" +
                    leaf_base + " + " + index_text(leaf.index, names) + "));\n";
            body += in + "        " + X + "[j][0] = w.x; " + X + "[j][1] = w.y; " + X + "[j][2] = w.z; " + X +
                    "[j][3] = w.w;\n";
            c += chunk_loop(in + "    ", body);
            c += in + "}\n    }\n";
            return c;
        };
        // The part's max (and, for the fast output, its min) over the
        // workgroup, then its sum of exp(f - max).  LDS slots `slot`,
        // slot + 1, slot + 2 (one set per register set).  Every term of
        // that sum is at most 1 and the part's max contributes exactly 1, so
        // terms below the normal range (flushed to zero by
        // porch_exp_flush) change it by less than 2^-110 relative.
        auto publish = [&](const std::string& X, const std::string& round, int slot) {
            const std::string in = "        ";
            std::string c = "    {\n" + row_scope(round, in);
            const std::string i2 = in + "    ";
            const std::string S0 = std::to_string(slot);
            const std::string S1 = std::to_string(slot + 1);
            c += i2 + "float xm = -PORCH_FLT_MAX;\n";
            if (sh.fast_output) c += i2 + "float xn = PORCH_FLT_MAX;\n";
            {
                std::string body;
                const std::vector<std::string> v = values(body, X, f, i2 + "        ");
                for (int e = 0; e < 4; ++e) body += i2 + "        xm = porch_fmax(xm, " + v[e] + ");\n";
                if (sh.fast_output)
                    for (int e = 0; e < 4; ++e) body += i2 + "        xn = porch_fmin(xn, " + v[e] + ");\n";
                c += chunk_loop(i2, body);
            }
            c += i2 + "xm = porch_wave_fmax(xm);\n";
            if (sh.fast_output) c += i2 + "xn = porch_wave_fmin(xn);\n";
            c += i2 + "if (lane == 0) {\n" + i2 + "    xred[" + S0 + "][wave] = xm;\n";
            if (sh.fast_output) c += i2 + "    xred[" + S1 + "][wave] = xn;\n";
            c += i2 + "}\n" + i2 + "__syncthreads();\n";
            c += i2 + "xm = porch_fmax(porch_fmax(xred[" + S0 + "][0], xred[" + S0 + "][1]), porch_fmax(xred[" + S0 +
                 "][2], xred[" + S0 + "][3]));\n";
            if (sh.fast_output)
                c += i2 + "xn" + X + " = porch_fmin(porch_fmin(xred[" + S1 + "][0], xred[" + S1 +
                     "][1]), porch_fmin(xred[" + S1 + "][2], xred[" + S1 + "][3]));\n";
            c += i2 + "float xs = 0.0f;\n";
            {
                std::string body;
                const std::vector<std::string> v = values(body, X, f, i2 + "        ");
                for (int e = 0; e < 4; ++e) body += i2 + "        xs += porch_exp_flush(" + v[e] + " - xm);\n";
                c += chunk_loop(i2, body);
            }
            c += block_reduce("xs", false, slot + 2, i2);
            c += i2 + "if (tl == 0) {\n";
            c += i2 + "    const unsigned long long word = (unsigned long long)__builtin_bit_cast(unsigned, xm) |\n";
            c += i2 + "        ((unsigned long long)__builtin_bit_cast(unsigned, xs) << 32);\n";
            c += i2 + "    __hip_atomic_store(xw + row * " + P + " + part, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n";
            c += i2 + "}\n";
            c += in + "}\n    }\n";
            return c;
        };
        // The row's max and sum from memory over the whole row (a
        // workgroup whose partners did not arrive): one pass, each lane
        // keeping the exact running max and a sum against an anchor moved
        // (with the sum rescaled) only by more than 64, as in emit_row.  A
        // lane adds L / 256 terms one after another, so it sums in double.
        // LDS slots of its own (after the register sets').
        const int fallback_slot = 3 * register_sets;
        auto whole_row = [&](const std::string& in) {
            std::string c;
            c += in + "float acc_m = -PORCH_FLT_MAX;\n" + in + "float acc_a = -PORCH_FLT_MAX;\n" + in + "double acc_s = 0.0;\n";
            c += in + "#pragma unroll 4\n";
            c += in + "for (" + std::string(T) + " xj = 0; xj < " + std::to_string((length + 1023) / 1024) + "; ++xj) {\n";
            c += in + "    const " + T + " " + qc + " = xj * 1024 + tl * 4;\n";
            c += in + "    if (" + qc + " < " + L + ") {\n";
            c += in + "        const float4 xv = *reinterpret_cast<const float4*>(" + leaf_base + " + " +
                 index_text(leaf.index, names) + ");\n";
            c += in + "        float xq[1][4] = {{xv.x, xv.y, xv.z, xv.w}};\n";
            c += in + "        const int j = 0;\n";
            std::string body;
            const std::vector<std::string> v = values(body, "xq", f, in + "        ");
            c += body;
            c += in + "        const float cm = porch_fmax(porch_fmax(" + v[0] + ", " + v[1] + "), porch_fmax(" + v[2] + ", " +
                 v[3] + "));\n";
            c += in + "        acc_m = porch_fmax(acc_m, cm);\n";
            c += in + "        if (cm > acc_a + 64.0f) {\n" + in +
                 "            acc_s = acc_s * (double)porch_exp(acc_a - cm);\n" + in + "            acc_a = cm;\n" + in +
                 "        }\n";
            for (int e = 0; e < 4; ++e) c += in + "        acc_s += (double)porch_exp(" + v[e] + " - acc_a);\n";
            c += in + "    }\n" + in + "}\n";
            c += block_reduce("acc_m", true, fallback_slot, in);
            c += in + "float acc_l = (float)(acc_s * (double)porch_exp(acc_a - acc_m));\n";
            c += block_reduce("acc_l", false, fallback_slot + 1, in);
            return c;
        };
        // The reference's block order for a max whose order-free value may
        // differ from it (NaN, or +0): 256 virtual lanes over the whole
        // row, then the stride tree.
        auto exact_max = [&](const std::string& acc, const std::string& in) {
            std::string c = in + "if (porch_max_order_matters(" + acc + ")) {\n";
            c += in + "    float xf = -PORCH_FLT_MAX;\n";
            c += in + "    for (" + std::string(T) + " " + qc + " = tl; " + qc + " < " + L + "; " + qc + " += 256) {\n";
            c += in + "        const float xq[1][1] = {{" + leaf_base + "[" + index_text(leaf.index, names) + "]}};\n";
            c += in + "        const int j = 0;\n";
            std::string body;
            const std::vector<std::string> v = values(body, "xq", f, in + "        ", 1);
            c += body + in + "        xf = porch_refmax(xf, " + v[0] + ");\n" + in + "    }\n";
            c += in + "    ex[tl] = xf;\n" + in + "    __syncthreads();\n";
            c += in + "    if (wave == 0) {\n";
            c += in + "        float xh = porch_refmax(porch_refmax(ex[lane], ex[lane + 128]), porch_refmax(ex[lane + 64], ex[lane + 192]));\n";
            for (int m = 32; m >= 1; m /= 2)
                c += in + "        xh = porch_refmax(xh, __shfl_xor(xh, " + std::to_string(m) + ", 64));\n";
            c += in + "        if (lane == 0) ex[256] = xh;\n" + in + "    }\n";
            c += in + "    __syncthreads();\n" + in + "    " + acc + " = ex[256];\n" + in + "}\n";
            return c;
        };
        auto finish = [&](const std::string& X, const std::string& round, int stat) {
            const std::string in = "        ";
            const std::string S = std::to_string(stat);
            std::string c = "    {\n" + row_scope(round, in);
            const std::string i2 = in + "    ";
            c += i2 + "if (wave == 0) {\n";
            c += i2 + "    unsigned long long word = 0ull;\n";
            c += i2 + "    bool ready = false;\n";
            c += i2 + "    for (int spin = 0; spin < porch_spin_limit; ++spin) {\n";
            c += i2 + "        if (lane < " + P + ") word = __hip_atomic_load(xw + row * " + P +
                 " + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n";
            c += i2 + "        ready = __ballot(lane >= " + P + " || word != 0ull) == ~0ull;\n";
            c += i2 + "        if (ready) break;\n";
            c += i2 + "        __builtin_amdgcn_s_sleep(1);\n";
            c += i2 + "    }\n";
            c += i2 + "    const float pm = __builtin_bit_cast(float, (unsigned)word);\n";
            c += i2 + "    const float ps = __builtin_bit_cast(float, (unsigned)(word >> 32));\n";
            c += i2 + "    const float m = porch_wave_fmax(lane < " + P + " ? pm : -PORCH_FLT_MAX);\n";
            c += i2 + "    if (lane == 0) {\n" + i2 + "        xstat[" + S + "][0] = m;\n" + i2 + "        xstat[" + S +
                 "][2] = ready ? 0.0f : 1.0f;\n" + i2 + "    }\n";
            c += i2 + "    xpm = pm;\n" + i2 + "    xps = ps;\n";
            c += i2 + "}\n";
            c += i2 + "__syncthreads();\n";
            c += i2 + "float rv0 = xstat[" + S + "][0];\n";
            c += i2 + "float rv1;\n";
            c += i2 + "if (xstat[" + S + "][2] != 0.0f) {\n";
            c += whole_row(i2 + "    ");
            c += exact_max("acc_m", i2 + "    ");
            c += i2 + "    rv0 = acc_m;\n" + i2 + "    rv1 = acc_l;\n";
            c += i2 + "}\n" + i2 + "else {\n";
            c += exact_max("rv0", i2 + "    ");
            c += i2 + "    if (wave == 0) {\n";
            c += i2 + "        const float t = porch_wave_sum(lane < " + P + " ? xps * porch_exp(xpm - rv0) : 0.0f);\n";
            c += i2 + "        if (lane == 0) xstat[" + S + "][1] = t;\n";
            c += i2 + "    }\n";
            c += i2 + "    __syncthreads();\n";
            c += i2 + "    rv1 = xstat[" + S + "][1];\n";
            c += i2 + "}\n";
            // written once and not read again here: past the caches
            auto store = [&](const std::vector<std::string>& v) {
                return i2 + "        __builtin_nontemporal_store((porch_v4f){" + v[0] + ", " + v[1] + ", " + v[2] + ", " +
                       v[3] + "}, reinterpret_cast<porch_v4f*>(out + row * " + L + " + " + qc + "));\n";
            };
            std::string general;
            {
                std::string body;
                const std::vector<std::string> v = values(body, X, r.output, i2 + "        ");
                general = chunk_loop(i2, body + store(v));
            }
            if (sh.fast_output) {
                // Every f - M in [-60, 0] (the part's min within 60 of the row
                // max; false for NaN): exp(f - M) is normal, where
                // porch_exp_flush is within 1 ulp; S = rv1 is in [1, 2^31]
                // (the row max's own term is 1), so each quotient is normal and
                // porch_div gives the IEEE quotient.
                c += i2 + "if (xn" + X + " - rv0 >= -60.0f) {\n";
                c += i2 + "    const float xr = porch_rcp(rv1);\n";
                std::string body;
                const std::vector<std::string> v = values(body, X, f, i2 + "        ");
                std::vector<std::string> q;
                for (int e = 0; e < 4; ++e) {
                    const std::string E = std::to_string(e);
                    body += i2 + "        const float xe" + E + " = porch_exp_flush_finite(" + v[e] + " - rv0);\n";
                    q.push_back("porch_div(xe" + E + ", xr, rv1)");
                }
                c += chunk_loop(i2 + "    ", body + store(q));
                c += i2 + "}\n" + i2 + "else {\n" + general + i2 + "}\n";
            }
            else {
                c += general;
            }
            c += in + "}\n    }\n";
            return c;
        };

        std::string params;
        for (int s = 0; s < r.n_slots; ++s)
            params += std::string(s == r.split_slot ? "float* __restrict__ a" : "const float* __restrict__ a") +
                      std::to_string(s) + ", ";
        params += "float* __restrict__ out";

        std::string& s = kc.source;
        s = kernel_prologue(r.n_slots, T);
        s += "__device__ __forceinline__ float porch_wave_fmax(float v) {\n"
             "    for (int d = 32; d >= 1; d >>= 1) v = porch_fmax(v, __shfl_xor(v, d, 64));\n    return v;\n}\n";
        s += "__device__ __forceinline__ float porch_wave_sum(float v) {\n"
             "    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);\n    return v;\n}\n";
        if (sh.fast_output) {
            s += "__device__ __forceinline__ float porch_fmin(float a, float b) { return __builtin_elementwise_minimum(a, b); }\n";
            s += "__device__ __forceinline__ float porch_wave_fmin(float v) {\n"
                 "    for (int d = 32; d >= 1; d >>= 1) v = porch_fmin(v, __shfl_xor(v, d, 64));\n    return v;\n}\n";
            // a / b from r = porch_rcp(b), the correctly rounded 1/b, for a
            // normal quotient: q = RN(a r) is within one ulp of a / b, the
            // remainder a - b q is exact in one fma, and RN(q + (a - b q) r)
            // is the correctly rounded quotient (P. Markstein, IBM J. Res.
            // Dev. 34(1), 1990).
            s += "__device__ __forceinline__ float porch_div(float a, float r, float b) {\n"
                 "    const float q = a * r;\n"
                 "    return __builtin_fmaf(__builtin_fmaf(-b, q, a), r, q);\n}\n";
        }
        s += "#define porch_spin_limit " + std::to_string(spin_limit) + "\n";
        s += "extern \"C\" __global__ void __launch_bounds__(256, " + std::to_string(groups_per_cu) + ") porch_row(" + params +
             ") {\n";
        s += "    const int tl = threadIdx.x;\n    const int lane = tl & 63;\n    const int wave = tl >> 6;\n";
        s += "    __shared__ float xred[" + std::to_string(3 * register_sets + 2) + "][4];\n";
        s += "    __shared__ float xstat[" + std::to_string(register_sets) + "][3];\n    __shared__ float ex[257];\n";
        s += "    const int xcd = (int)(blockIdx.x % 8);\n    const int xslot = (int)(blockIdx.x / 8);\n";
        s += "    const int group = xslot / " + P + ";\n    const int part = xslot % " + P + ";\n";
        s += "    unsigned long long* __restrict__ xw = reinterpret_cast<unsigned long long*>(a" +
             std::to_string(r.split_slot) + ");\n";
        // Register set i holds items i, i + n, i + 2n, ... (n sets).  Step
        // for item t: load item t + n - 1 (into the set item t - 1 left),
        // publish item t + 1, write item t out.  A part thus waits for its
        // partners' words of item t a whole step after publishing its own,
        // and with three sets its loads stay in flight across a step.
        const int n_sets = register_sets;
        std::vector<std::string> X;
        for (int i = 0; i < n_sets; ++i) {
            X.push_back("x" + std::string(1, static_cast<char>('a' + i)));
            s += "    float " + X.back() + "[" + std::to_string(sh.chunks) + "][4];\n";
            if (sh.fast_output) s += "    float xn" + X.back() + " = 0.0f;\n";
        }
        s += "    float xpm = 0.0f;\n    float xps = 0.0f;\n";
        const std::string R = std::to_string(sh.rounds);
        auto guarded = [&](const std::string& cond, const std::string& code) {
            return "    if (" + cond + ") {\n" + code + "    }\n";
        };
        for (int i = 0; i + 1 < n_sets; ++i)
            s += guarded(std::to_string(i) + " < " + R, load_item(X[i], std::to_string(i)));
        s += publish(X[0], "0", 0);
        s += "    for (int k = 0; k < " + R + "; k += " + std::to_string(n_sets) + ") {\n";
        for (int t = 0; t < n_sets; ++t) {
            const auto item = [&](int d) { return "k + " + std::to_string(t + d); };
            std::string step;
            const int load_set = (t + n_sets - 1) % n_sets;
            const int pub_set = (t + 1) % n_sets;
            step += guarded(item(n_sets - 1) + " < " + R, load_item(X[load_set], item(n_sets - 1)));
            step += guarded(item(1) + " < " + R, publish(X[pub_set], item(1), 3 * pub_set));
            step += finish(X[t], item(0), t);
            s += t == 0 ? step : guarded(item(0) + " < " + R, step);
        }
        s += "    }\n}\n";
        return kc;
    }

} // namespace porch::cg
