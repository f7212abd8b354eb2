#include "emit_expr.hpp"

#include <stdexcept>

namespace porch::cg {

    emitter::emitter(const kexpr& expr, std::string& target, int lanes)
        : k(expr), code(target), width(lanes) {
        frames_.emplace_back();
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
            case kop::add: binary("+"); break;
            case kop::subtract: binary("-"); break;
            case kop::multiply: binary("*"); break;
            case kop::divide: binary("/"); break;
            case kop::maximum:
            case kop::minimum: {
                const std::vector<std::string> a = emit(n.a);
                const std::vector<std::string> b = emit(n.b);
                const char* cmp = n.op == kop::maximum ? " > " : " < ";
                for (int e = 0; e < width; ++e) {
                    const std::string name = fresh("v");
                    line("const float " + name + " = (" + a[e] + cmp + b[e] +
                         ") ? " + a[e] + " : " + b[e] + ";");
                    result[e] = name;
                }
                break;
            }
            case kop::exp: {
                const std::vector<std::string> a = emit(n.a);
                for (int e = 0; e < width; ++e) {
                    const std::string name = fresh("v");
                    line("const float " + name + " = expf(" + a[e] + ");");
                    result[e] = name;
                }
                break;
            }
            case kop::reciprocal: {
                const std::vector<std::string> a = emit(n.a);
                for (int e = 0; e < width; ++e) {
                    const std::string name = fresh("v");
                    line("const float " + name + " = 1.0f / " + a[e] + ";");
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

    std::string kernel_prologue(int n_slots, const char* index_type) {
        (void)n_slots;
        std::string s;
        s += "// porch fused kernel (gfx950, wave64)\n";
        s += "typedef ";
        s += index_type;
        s += " idx_t;\n";
        s += "#define PORCH_FLT_MAX 3.40282346638528859812e+38f\n";
        return s;
    }

} // namespace porch::cg
