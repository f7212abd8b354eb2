#include "emit_expr.hpp"

#include <cmath>
#include <stdexcept>

namespace porch::cg {

    emitter::emitter(const kexpr& expr, std::string& target, int lanes)
        : k(expr), code(target), width(lanes) {
        frames_.emplace_back();
    }

    const vrange& emitter::range_of(int id) {
        if (ranges_.size() != k.nodes.size()) ranges_ = value_ranges(k, row_value_range, refine_range);
        return ranges_[static_cast<size_t>(id)];
    }

    void emitter::declare_roots(std::vector<int> ids) {
        roots_ = std::move(ids);
        roots_declared_ = true;
    }

    bool emitter::denormals_absorbed(int id) {
        return only_added_to_constants(id, std::ldexp(1.0F, -100));
    }

    bool emitter::only_added_to_constants(int id, float least) {
        if (!roots_declared_) return false;
        for (const int r : roots_) {
            if (r == id) return false;
        }
        auto big_constant = [&](int c) {
            const knode& n = k.at(c);
            return n.op == kop::constant && std::fabs(n.value) >= least;
        };
        int users = 0;
        for (size_t u = 0; u < k.nodes.size(); ++u) {
            const knode& n = k.nodes[u];
            if (n.a != id && n.b != id) continue;
            ++users;
            const bool absorbs = (n.op == kop::add || n.op == kop::subtract) &&
                                 ((n.a == id && n.b != id && big_constant(n.b)) ||
                                  (n.b == id && n.a != id && big_constant(n.a)));
            if (!absorbs) return false;
        }
        return users > 0;
    }

    int emitter::fusable_product(int id) {
        if (!relaxed || !relaxed(id)) return -1;
        const knode& n = k.at(id);
        for (const int side : {n.a, n.b}) {
            if (side < 0 || side == (side == n.a ? n.b : n.a)) continue;
            const knode& m = k.at(side);
            if (m.op != kop::multiply || !relaxed(side) || find(side) != nullptr) continue;
            int users = 0;
            for (const knode& u : k.nodes) users += (u.a == side) + (u.b == side);
            if (users == 1) return side;
        }
        return -1;
    }

    std::string emitter::fresh(const char* prefix) {
        return std::string{prefix} + std::to_string(counter_++);
    }

    void emitter::line(const std::string& text) {
        code += indent;
        code += text;
        code += '\n';
    }

    const std::vector<std::string>* emitter::find(int id) const {
        for (auto frame = frames_.rbegin(); frame != frames_.rend(); ++frame) {
            auto found = frame->find(id);
            if (found != frame->end()) return &found->second;
        }
        return nullptr;
    }

    std::vector<std::string> emitter::emit(int id) {
        if (const auto* known = find(id)) return *known;
        if (override_node) {
            std::vector<std::string> v = override_node(id);
            if (!v.empty()) {
                frames_.back()[id] = v;
                return v;
            }
        }
        const knode& n = k.at(id);
        std::vector<std::string> result(static_cast<size_t>(width));
        auto binary = [&](const char* symbol) {
            const std::vector<std::string> a = emit(n.a);
            const std::vector<std::string> b = emit(n.b);
            for (int e = 0; e < width; ++e) {
                const std::string name = fresh("v");
                line("const float " + name + " = " + a[e] + " " + symbol +
                     " " + b[e] + ";");
                result[e] = name;
            }
        };
        switch (n.op) {
            case kop::constant: {
                const std::string text = float_literal(n.value);
                for (int e = 0; e < width; ++e) result[e] = text;
                break;
            }
            case kop::load:
                result = load(id);
                break;
            case kop::row_value: {
                const std::string text = row_value(n.row);
                for (int e = 0; e < width; ++e) result[e] = text;
                break;
            }
            case kop::add:
            case kop::subtract: {
                // In a relaxed context a product used only here fuses into
                // one fma (one rounding instead of two).
                const int product = fusable_product(id);
                if (product < 0) {
                    binary(n.op == kop::add ? "+" : "-");
                    break;
                }
                const knode& m = k.at(product);
                const std::vector<std::string> x = emit(m.a);
                const std::vector<std::string> y = emit(m.b);
                const std::vector<std::string> c = emit(product == n.a ? n.b : n.a);
                // a*b + c, c + a*b, a*b - c = fma(a, b, -c), c - a*b = fma(-a, b, c)
                const bool negate_c = n.op == kop::subtract && product == n.a;
                const bool negate_p = n.op == kop::subtract && product == n.b;
                for (int e = 0; e < width; ++e) {
                    const std::string name = fresh("v");
                    line("const float " + name + " = __builtin_fmaf(" + (negate_p ? "-" : "") + x[e] + ", " + y[e] +
                         ", " + (negate_c ? "-" : "") + c[e] + ");");
                    result[e] = name;
                }
                break;
            }
            case kop::multiply: binary("*"); break;
            case kop::divide: binary("/"); break;
            case kop::maximum:
            case kop::minimum: {
                const std::vector<std::string> a = emit(n.a);
                const std::vector<std::string> b = emit(n.b);
                const bool is_max = n.op == kop::maximum;
                // Against a constant right operand c, v_max_f32(a, c) (and
                // v_min_f32) give the ternary's bits for every a: a NaN a
                // yields c in both, v_max_f32 orders -0 below +0 and
                // v_min_f32 +0 above -0 (measured on gfx950), so they agree
                // unless c is the zero the ternary would pass over: +0 for a
                // max, -0 for a min.  relu(v) = maximum(v, 0.0f) is one
                // instruction instead of a compare and a select.
                const knode& c = k.at(n.b);
                const bool constant = c.op == kop::constant && !std::isnan(c.value);
                // The other zero: the compiler itself turns a ternary against
                // a constant into v_min_f32 / v_max_f32 (measured: x < 0.0f ?
                // x : 0.0f became v_min_f32, giving -0 for x = -0 where the
                // ternary gives +0; an added 0.0f was folded away too), so
                // these two fix the zero's sign on the bits
                // (porch_min_pos0 / porch_max_neg0).
                const bool other_zero = constant && c.value == 0.0F && std::signbit(c.value) == is_max;
                const bool hardware = constant && !other_zero;
                const char* cmp = is_max ? " > " : " < ";
                for (int e = 0; e < width; ++e) {
                    const std::string name = fresh("v");
                    if (hardware)
                        line("const float " + name + " = " + (is_max ? "__builtin_fmaxf(" : "__builtin_fminf(") + a[e] +
                             ", " + b[e] + ");");
                    else if (other_zero)
                        line("const float " + name + " = " + (is_max ? "porch_max_neg0(" : "porch_min_pos0(") + a[e] +
                             ");");
                    else
                        line("const float " + name + " = (" + a[e] + cmp + b[e] + ") ? " + a[e] + " : " + b[e] + ";");
                    result[e] = name;
                }
                break;
            }
            case kop::exp: {
                // exp(0 - v) is exp(-v): the two arguments differ only in the
                // sign of zero, and exp(+0) = exp(-0) = 1.  The negation then
                // folds into the first multiply as a source modifier.
                const knode& arg = k.at(n.a);
                const bool negate = arg.op == kop::subtract && k.at(arg.a).op == kop::constant &&
                                    k.at(arg.a).value == 0.0F && !std::signbit(k.at(arg.a).value);
                const std::vector<std::string> a = emit(negate ? arg.b : n.a);
                // Arguments proven <= 88 cannot overflow: porch_exp skips the
                // overflow handling (and the NaN test when NaN is impossible).
                const vrange& r = range_of(n.a);
                const char* fn = "expf";
                if (relaxed && relaxed(id) && !std::isnan(r.hi) && r.hi <= 0.0F &&
                    only_added_to_constants(id, 1.0F)) {
                    // exp2(x log2 e): relative error <= |x| 2^-24 + 1 ulp, so
                    // for x <= 0 an absolute error below 2^-22.4, under one
                    // ulp of every constant (>= 1 in magnitude) it is added to.
                    fn = "porch_exp_relaxed";
                }
                else if (!std::isnan(r.hi) && r.hi <= 88.0F) {
                    // Where denormal results vanish in the consumer, the
                    // shorter sequence that flushes them is exact enough.
                    if (denormals_absorbed(id)) fn = r.nan ? "porch_exp_flush" : "porch_exp_flush_finite";
                    else fn = r.nan ? "porch_exp" : "porch_exp_finite";
                }
                for (int e = 0; e < width; ++e) {
                    const std::string name = fresh("v");
                    const std::string x = negate ? "-" + a[e] : a[e];
                    line("const float " + name + " = " + fn + "(" + x + ");");
                    result[e] = name;
                }
                break;
            }
            case kop::reciprocal: {
                const std::vector<std::string> a = emit(n.a);
                // Operands within |x| in [2^-125, 2^125] take the hardware
                // reciprocal plus one Newton step, which is the correctly
                // rounded 1/x there.
                const bool tame = reciprocal_is_tame(range_of(n.a));
                // In a relaxed context the hardware reciprocal alone (1 ulp).
                const char* fast = (relaxed && relaxed(id)) ? "__builtin_amdgcn_rcpf(" : "porch_rcp(";
                for (int e = 0; e < width; ++e) {
                    const std::string name = fresh("v");
                    line("const float " + name + " = " +
                         (tame ? fast + a[e] + ")" : "1.0f / " + a[e]) + ";");
                    result[e] = name;
                }
                break;
            }
            case kop::select: {
                const int forced = forced_branch ? forced_branch(id) : -1;
                if (forced >= 0) {
                    result = emit(forced == 0 ? n.a : n.b);
                    break;
                }
                std::vector<std::string> names(static_cast<size_t>(width));
                std::string decl = "float ";
                for (int e = 0; e < width; ++e) {
                    names[e] = fresh("s");
                    decl += names[e] + (e + 1 < width ? ", " : ";");
                }
                line(decl);
                line("if (" + condition(n.cond) + ") {");
                const std::string saved = indent;
                indent += "    ";
                frames_.emplace_back();
                const std::vector<std::string> a = emit(n.a);
                for (int e = 0; e < width; ++e) line(names[e] + " = " + a[e] + ";");
                frames_.pop_back();
                indent = saved;
                line("} else {");
                indent += "    ";
                frames_.emplace_back();
                const std::vector<std::string> b = emit(n.b);
                for (int e = 0; e < width; ++e) line(names[e] + " = " + b[e] + ";");
                frames_.pop_back();
                indent = saved;
                line("}");
                result = names;
                break;
            }
        }
        frames_.back()[id] = result;
        return result;
    }

    void emitter::open_scope(const std::string& condition) {
        line("if (" + condition + ") {");
        indent += "    ";
        frames_.emplace_back();
    }

    void emitter::close_scope() {
        frames_.pop_back();
        indent.resize(indent.size() - 4);
        line("}");
    }

    std::string index_text(const ival& v, const std::vector<std::string>& names) {
        if (!v.is_affine) {
            // Generic code refers to q{d}; the kernel declares those names.
            return "(" + v.code + ")";
        }
        std::string s;
        for (size_t d = 0; d < v.w.size(); ++d) {
            if (v.w[d] == 0) continue;
            if (!s.empty()) s += " + ";
            s += names[d];
            if (v.w[d] != 1) s += " * " + std::to_string(v.w[d]);
        }
        if (s.empty()) return std::to_string(v.c0);
        if (v.c0 > 0) s += " + " + std::to_string(v.c0);
        if (v.c0 < 0) s += " - " + std::to_string(-v.c0);
        return "(" + s + ")";
    }

    std::string decompose(const std::string& flat, const std::vector<int64_t>& shape,
                          const std::vector<bool>& needed, const char* type,
                          const std::string& indent) {
        std::string code;
        const size_t rank = shape.size();
        if (rank == 0) return code;
        int64_t stride = 1;
        std::vector<int64_t> strides(rank, 1);
        for (size_t d = rank; d > 0; --d) {
            strides[d - 1] = stride;
            stride *= shape[d - 1];
        }
        for (size_t d = 0; d < rank; ++d) {
            if (!needed[d]) continue;
            std::string value;
            if (shape[d] == 1) value = "0";
            else if (d == 0) value = flat + " / " + std::to_string(strides[d]);
            else if (strides[d] == 1) value = flat + " % " + std::to_string(shape[d]);
            else
                value = "(" + flat + " / " + std::to_string(strides[d]) + ") % " +
                        std::to_string(shape[d]);
            if (d == 0 && strides[d] == 1) value = flat;
            code += indent + "const " + type + " q" + std::to_string(d) + " = " +
                    value + ";\n";
        }
        return code;
    }

    std::vector<bool> used_coordinates(const kexpr& k, int root, size_t rank) {
        std::vector<bool> used(rank, false);
        auto mark = [&](const ival& v) {
            if (!v.is_affine) {
                for (size_t d = 0; d < rank; ++d) {
                    if (v.code.find("q" + std::to_string(d)) != std::string::npos)
                        used[d] = true;
                }
                // names like q1 also match q10..q19: over-marking is harmless.
                return;
            }
            for (size_t d = 0; d < rank; ++d) {
                if (v.w[d] != 0) used[d] = true;
            }
        };
        for (const int id : k.postorder(root)) {
            const knode& n = k.at(id);
            if (n.op == kop::load) mark(n.index);
            if (n.op == kop::select) mark(n.cond.lhs);
        }
        return used;
    }

    std::string kernel_params(int n_slots) {
        std::string params;
        for (int s = 0; s < n_slots; ++s) {
            params += "const float* __restrict__ a" + std::to_string(s) + ", ";
        }
        params += "float* __restrict__ out";
        return params;
    }

    namespace {
        // Device helpers the emitters call where value ranges allow.
        //
        // porch_rcp: hardware reciprocal (about 1 ulp) refined by one
        // Newton-Raphson step with fused multiply-adds.  For |d| in
        // [2^-125, 2^125] this equals the IEEE quotient 1.0f / d bit for bit
        // (verified exhaustively on gfx950 over every float with |d| in
        // [2^-125, 2^125], both signs); NaN propagates.
        //
        // porch_exp / porch_exp_finite: exp(x) for x <= 88 by Cody-Waite
        // style reduction onto the hardware exp2: k = rint(x log2 e) with
        // x log2 e carried as a hi + lo pair, exp2 of the small remainder,
        // then ldexp by k (which also produces denormal and zero results).
        // Below -104 every result rounds to zero, so x is clamped there.
        // Max error 1 ulp against the correctly rounded exp over every float
        // in [-104, 88.72] (verified exhaustively on gfx950), the same as
        // expf.  porch_exp keeps NaN; porch_exp_finite assumes no NaN.
        //
        // porch_exp_flush / porch_exp_flush_finite: exp(x) for x <= 88 as
        // exp2(p) (1 + u) with p = RN(x log2 e) and u = x - p ln 2 (ln 2 as a
        // hi + lo pair), one fused multiply-add.  Max error 1 ulp for normal
        // results over every float in [-104, 88.72] (verified exhaustively on
        // gfx950), but denormal results come out as zero: only used where
        // every consumer adds a constant that absorbs denormals.
        //
        // porch_exp_relaxed: exp2(x log2 e) in two instructions, relative
        // error <= |x| 2^-24 + 1 ulp, denormal results flushed; only for
        // arguments <= 0 whose result is added to constants of magnitude
        // >= 1 on its way into a sum that is the kernel's result.
        const char* math_helpers() {
            return R"(__device__ __forceinline__ float porch_rcp(float d) {
    const float r = __builtin_amdgcn_rcpf(d);
    return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
}
__device__ __forceinline__ float porch_exp_reduced(float x) {
    const float L = 1.44269502162933349609375f;
    const float Llo = 1.925963033500011079013347625732421875e-8f;
    const float ph = x * L;
    const float pl = __builtin_fmaf(x, Llo, __builtin_fmaf(x, L, -ph));
    const float k = __builtin_rintf(ph);
    const float r = __builtin_amdgcn_exp2f((ph - k) + pl);
    return __builtin_ldexpf(r, (int)k);
}
__device__ __forceinline__ float porch_exp(float x) {
    return porch_exp_reduced(x < -104.0f ? -104.0f : x);
}
__device__ __forceinline__ float porch_exp_finite(float x) {
    return porch_exp_reduced(__builtin_fmaxf(x, -104.0f));
}
__device__ __forceinline__ float porch_exp_relaxed(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269502162933349609375f);
}
__device__ __forceinline__ float porch_exp_flush_reduced(float x) {
    const float L = 1.44269502162933349609375f;
    const float ph = x * L;
    float u = __builtin_fmaf(-ph, 0.693145751953125f, x);
    u = __builtin_fmaf(-ph, 1.428606765330187045e-06f, u);
    const float r = __builtin_amdgcn_exp2f(ph);
    return __builtin_fmaf(r, u, r);
}
__device__ __forceinline__ float porch_exp_flush(float x) {
    return porch_exp_flush_reduced(x < -104.0f ? -104.0f : x);
}
__device__ __forceinline__ float porch_exp_flush_finite(float x) {
    return porch_exp_flush_reduced(__builtin_fmaxf(x, -104.0f));
}
// The reference's ternaries against the zero they pass over, x < +0 ? x : +0
// and x > -0 ? x : -0 (v_min_f32 gives -0 for (-0, +0), v_max_f32 +0 for
// (+0, -0); the sign is set on the bits, which the compiler keeps).
__device__ __forceinline__ float porch_min_pos0(float x) {
    const int i = __builtin_bit_cast(int, __builtin_fminf(x, 0.0f));
    return __builtin_bit_cast(float, i == (int)0x80000000 ? 0 : i);
}
__device__ __forceinline__ float porch_max_neg0(float x) {
    const int i = __builtin_bit_cast(int, __builtin_fmaxf(x, -0.0f));
    return __builtin_bit_cast(float, i == 0 ? (int)0x80000000 : i);
}
// Order-free max for folds and lane reductions (v_maximum3_f32): NaN if
// either operand is NaN, and -0 < +0, so every grouping gives the same
// value and a NaN anywhere reaches the result.
__device__ __forceinline__ float porch_fmax(float a, float b) {
    return __builtin_elementwise_maximum(a, b);
}
// The reference's max step, t = t > v ? t : v (src/tensor.cpp:849-851,
// 939-958): NaN survives only as the right operand, and a tie between
// +0 and -0 goes to the right operand.
__device__ __forceinline__ float porch_refmax(float a, float b) {
    return a > b ? a : b;
}
// Can a max reduction's order-free result differ from the reference's
// block order?  Only for NaN (which survives there by position) and for a
// +0 maximum (a -0 in the row may win the tie there).  A -0 maximum means
// every zero is -0; any other value is unique.
__device__ __forceinline__ bool porch_max_order_matters(float m) {
    return m != m || __builtin_bit_cast(unsigned, m) == 0u;
}
)";
        }
    } // namespace

    std::string kernel_prologue(int n_slots, const char* index_type) {
        (void)n_slots;
        std::string s;
        s += "// porch fused kernel (gfx950, wave64)\n";
        s += "typedef ";
        s += index_type;
        s += " idx_t;\n";
        s += "#define PORCH_FLT_MAX 3.40282346638528859812e+38f\n";
        s += "typedef float porch_v4f __attribute__((ext_vector_type(4)));\n";
        s += math_helpers();
        return s;
    }

} // namespace porch::cg
