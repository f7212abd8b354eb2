#include "lower.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <stdexcept>

namespace porch::cg {

    ival ival::constant(int64_t value, size_t rank) {
        ival v;
        v.c0 = value;
        v.w.assign(rank, 0);
        return v;
    }

    ival ival::coordinate(size_t d, size_t rank) {
        ival v = constant(0, rank);
        v.w[d] = 1;
        return v;
    }

    bool ival::is_constant() const {
        if (!is_affine) return false;
        for (const int64_t x : w) {
            if (x != 0) return false;
        }
        return true;
    }

    std::string ival::str() const {
        if (!is_affine) return "(" + code + ")";
        std::string s;
        for (size_t d = 0; d < w.size(); ++d) {
            if (w[d] == 0) continue;
            if (!s.empty()) s += " + ";
            if (w[d] == 1) s += "q" + std::to_string(d);
            else s += "q" + std::to_string(d) + " * " + std::to_string(w[d]);
        }
        if (s.empty()) return "(" + std::to_string(c0) + ")";
        if (c0 > 0) s += " + " + std::to_string(c0);
        if (c0 < 0) s += " - " + std::to_string(-c0);
        return "(" + s + ")";
    }

    std::string ival::key() const {
        if (!is_affine) return "g" + code;
        std::string k = "a" + std::to_string(c0);
        for (const int64_t x : w) k += "," + std::to_string(x);
        return k;
    }

    namespace {

        ival add(const ival& a, const ival& b) {
            if (a.is_affine && b.is_affine) {
                ival r = a;
                r.c0 += b.c0;
                for (size_t d = 0; d < r.w.size(); ++d) r.w[d] += b.w[d];
                return r;
            }
            ival r;
            r.is_affine = false;
            r.w.assign(a.w.size(), 0);
            r.code = a.str() + " + " + b.str();
            return r;
        }

        ival scale(const ival& a, int64_t k) {
            if (a.is_affine) {
                ival r = a;
                r.c0 *= k;
                for (int64_t& x : r.w) x *= k;
                return r;
            }
            if (k == 1) return a;
            ival r = a;
            r.code = a.str() + " * " + std::to_string(k);
            return r;
        }

        ival add_constant(const ival& a, int64_t k) {
            if (a.is_affine) {
                ival r = a;
                r.c0 += k;
                return r;
            }
            ival r = a;
            r.code = a.str() + (k >= 0 ? " + " : " - ") +
                     std::to_string(k >= 0 ? k : -k);
            return r;
        }

    } // namespace

    int kexpr::add(knode n) {
        std::string key;
        key += std::to_string(static_cast<int>(n.op));
        key += '|' + std::to_string(n.a) + '|' + std::to_string(n.b);
        switch (n.op) {
            case kop::load:
                key += '|' + std::to_string(n.slot) + '|' + n.index.key();
                break;
            case kop::constant: {
                uint32_t bits = 0;
                std::memcpy(&bits, &n.value, sizeof bits);
                key += '|' + std::to_string(bits);
                break;
            }
            case kop::select:
                key += '|' + n.cond.lhs.key() + '<' +
                       std::to_string(n.cond.bound);
                break;
            case kop::row_value:
                key += '|' + std::to_string(n.row);
                break;
            default:
                break;
        }
        auto found = interned.find(key);
        if (found != interned.end()) {
            knode& known = nodes[static_cast<size_t>(found->second)];
            for (size_t d = 0; d < known.box.size() && d < n.box.size(); ++d) {
                known.box[d].first = std::min(known.box[d].first, n.box[d].first);
                known.box[d].second = std::max(known.box[d].second, n.box[d].second);
            }
            return found->second;
        }
        const int id = static_cast<int>(nodes.size());
        nodes.push_back(std::move(n));
        interned.emplace(std::move(key), id);
        return id;
    }

    std::vector<int> kexpr::postorder(int root) const {
        std::vector<int> order;
        std::vector<char> seen(nodes.size(), 0);
        std::function<void(int)> visit = [&](int id) {
            if (id < 0 || seen[id]) return;
            seen[id] = 1;
            visit(nodes[id].a);
            visit(nodes[id].b);
            order.push_back(id);
        };
        visit(root);
        return order;
    }

    std::vector<int> kexpr::loads(int root) const {
        std::vector<int> result;
        for (const int id : postorder(root)) {
            if (nodes[id].op == kop::load) result.push_back(id);
        }
        return result;
    }

    lowering::lowering(
        const ir::graph& graph, kexpr& arena, std::vector<int64_t> extents
    )
        : g(graph), out(arena), extent(std::move(extents)) {
        box.reserve(extent.size());
        for (const int64_t e : extent) box.emplace_back(0, e);
        input_slot.assign(static_cast<size_t>(g.n_inputs), -1);
    }

    std::vector<ival> lowering::identity() const {
        std::vector<ival> coords;
        for (size_t d = 0; d < extent.size(); ++d)
            coords.push_back(ival::coordinate(d, extent.size()));
        return coords;
    }

    std::pair<int64_t, int64_t> lowering::range(const ival& v) const {
        int64_t lo = v.c0;
        int64_t hi = v.c0;
        for (size_t d = 0; d < v.w.size(); ++d) {
            if (v.w[d] == 0) continue;
            const int64_t a = v.w[d] * box[d].first;
            const int64_t b = v.w[d] * (box[d].second - 1);
            lo += std::min(a, b);
            hi += std::max(a, b);
        }
        return {lo, hi};
    }

    ival lowering::linearize(
        const std::vector<ival>& coords, const std::vector<int64_t>& shape
    ) const {
        const std::vector<int64_t> strides = ir::contiguous_strides(shape);
        ival lin = ival::constant(0, extent.size());
        for (size_t k = 0; k < shape.size(); ++k) {
            if (shape[k] == 1) continue; // coordinate is always 0
            lin = add(lin, scale(coords[k], strides[k]));
        }
        return lin;
    }

    std::vector<ival> lowering::delinearize(
        const ival& lin, const std::vector<int64_t>& shape
    ) const {
        const size_t rank = extent.size();
        const size_t n = shape.size();
        const std::vector<int64_t> strides = ir::contiguous_strides(shape);
        std::vector<ival> coords(n, ival::constant(0, rank));
        if (n == 0) return coords;

        if (lin.is_affine) {
            // Carry-free test: write the (box-shifted) constant and every
            // weight in the mixed radix of `shape`; if no digit position can
            // overflow anywhere in the box, each coordinate is the digit-wise
            // sum, which is affine.
            bool ok = true;
            int64_t base = lin.c0;
            for (size_t d = 0; d < rank; ++d) {
                if (lin.w[d] < 0) ok = false;
                base += lin.w[d] * box[d].first;
            }
            if (base < 0) ok = false;
            auto digits = [&](int64_t value) {
                std::vector<int64_t> dig(n, 0);
                for (size_t j = 0; j < n; ++j) {
                    if (shape[j] == 0) continue;
                    dig[j] = (value / strides[j]) % shape[j];
                }
                // leading digit absorbs anything beyond the shape
                if (strides[0] > 0) dig[0] = value / strides[0];
                return dig;
            };
            if (ok) {
                const std::vector<int64_t> base_digits = digits(base);
                std::vector<std::vector<int64_t>> weight_digits(rank);
                std::vector<int64_t> max_digit = base_digits;
                for (size_t d = 0; d < rank && ok; ++d) {
                    if (lin.w[d] == 0) continue;
                    weight_digits[d] = digits(lin.w[d]);
                    const int64_t span = box[d].second - 1 - box[d].first;
                    for (size_t j = 0; j < n; ++j)
                        max_digit[j] += weight_digits[d][j] * span;
                }
                for (size_t j = 0; j < n && ok; ++j) {
                    if (max_digit[j] >= shape[j]) ok = false;
                }
                if (ok) {
                    for (size_t j = 0; j < n; ++j) {
                        ival c = ival::constant(base_digits[j], rank);
                        for (size_t d = 0; d < rank; ++d) {
                            if (lin.w[d] == 0) continue;
                            c.w[d] = weight_digits[d][j];
                            c.c0 -= weight_digits[d][j] * box[d].first;
                        }
                        coords[j] = c;
                    }
                    return coords;
                }
            }
        }

        // Generic: runtime div/mod of the linear index.
        const std::string text = lin.str();
        for (size_t j = 0; j < n; ++j) {
            if (shape[j] == 1) continue;
            ival c;
            c.is_affine = false;
            c.w.assign(rank, 0);
            if (j == 0) c.code = text + " / " + std::to_string(strides[j]);
            else if (strides[j] == 1)
                c.code = text + " % " + std::to_string(shape[j]);
            else
                c.code = "(" + text + " / " + std::to_string(strides[j]) +
                         ") % " + std::to_string(shape[j]);
            coords[j] = c;
        }
        return coords;
    }

    int lowering::at_linear(int id, const ival& lin) {
        const ir::node& n = g.at(id);
        if (n.kind == ir::op::input) {
            knode load;
            load.op = kop::load;
            load.slot = input_slot[static_cast<size_t>(n.input)];
            load.index = lin;
            load.box = box;
            return out.add(load);
        }
        auto bound_it = bound.find(id);
        if (bound_it != bound.end() &&
            bound_it->second.what == binding::kind::slot) {
            knode load;
            load.op = kop::load;
            load.slot = bound_it->second.slot;
            load.index = bound_it->second.offset != 0 ? add_constant(lin, bound_it->second.offset) : lin;
            load.box = box;
            return out.add(load);
        }
        if (n.is_scalar) return at(id, {});
        return at(id, delinearize(lin, n.out));
    }

    int lowering::at(int id, const std::vector<ival>& coords) {
        const ir::node& n = g.at(id);
        const size_t rank = extent.size();

        auto bound_it = bound.find(id);
        if (bound_it != bound.end()) {
            if (bound_it->second.what == binding::kind::row_value) {
                knode v;
                v.op = kop::row_value;
                v.row = bound_it->second.row;
                return out.add(v);
            }
            knode load;
            load.op = kop::load;
            load.slot = bound_it->second.slot;
            load.index = linearize(coords, n.out);
            if (bound_it->second.offset != 0) load.index = add_constant(load.index, bound_it->second.offset);
            load.box = box;
            return out.add(load);
        }

        switch (n.kind) {
            case ir::op::input: {
                knode load;
                load.op = kop::load;
                load.slot = input_slot[static_cast<size_t>(n.input)];
                if (load.slot < 0)
                    throw std::logic_error("input without a kernel slot");
                load.index = linearize(coords, n.out);
                load.box = box;
                return out.add(load);
            }
            case ir::op::scalar: {
                knode c;
                c.op = kop::constant;
                c.value = n.scalar;
                return out.add(c);
            }
            case ir::op::add:
            case ir::op::subtract:
            case ir::op::multiply:
            case ir::op::divide:
            case ir::op::maximum:
            case ir::op::minimum: {
                const ir::node& l = g.at(n.lhs);
                const ir::node& r = g.at(n.rhs);
                knode b;
                b.a = at(n.lhs, l.is_scalar ? std::vector<ival>{} : coords);
                b.b = at(n.rhs, r.is_scalar ? std::vector<ival>{} : coords);
                switch (n.kind) {
                    case ir::op::add: b.op = kop::add; break;
                    case ir::op::subtract: b.op = kop::subtract; break;
                    case ir::op::multiply: b.op = kop::multiply; break;
                    case ir::op::divide: b.op = kop::divide; break;
                    case ir::op::maximum: b.op = kop::maximum; break;
                    default: b.op = kop::minimum; break;
                }
                return out.add(b);
            }
            case ir::op::exp:
            case ir::op::reciprocal: {
                knode u;
                u.op = n.kind == ir::op::exp ? kop::exp : kop::reciprocal;
                u.a = at(n.lhs, coords);
                return out.add(u);
            }
            case ir::op::slice: {
                ival lin = ival::constant(n.offset, rank);
                for (size_t k = 0; k < n.shape.size(); ++k) {
                    if (n.shape[k] == 1 || n.strides[k] == 0) continue;
                    lin = add(lin, scale(coords[k], n.strides[k]));
                }
                return at_linear(n.lhs, lin);
            }
            case ir::op::reshape:
                return at_linear(n.lhs, linearize(coords, n.out));
            case ir::op::unsqueeze: {
                std::vector<ival> child = coords;
                child.erase(child.begin() + n.axis);
                return at(n.lhs, child);
            }
            case ir::op::transpose:
                return at(n.lhs, {coords[1], coords[0]});
            case ir::op::permute: {
                // output dimension i is operand dimension shape[i]
                std::vector<ival> child(coords.size());
                for (size_t i = 0; i < coords.size(); ++i)
                    child[static_cast<size_t>(n.shape[i])] = coords[i];
                return at(n.lhs, child);
            }
            case ir::op::broadcast: {
                const ir::node& src = g.at(n.lhs);
                if (src.is_scalar) return at(n.lhs, {});
                const size_t offset = n.out.size() - src.out.size();
                std::vector<ival> child;
                for (size_t k = 0; k < src.out.size(); ++k) {
                    child.push_back(
                        src.out[k] == 1 ? ival::constant(0, rank)
                                        : coords[offset + k]
                    );
                }
                return at(n.lhs, child);
            }
            case ir::op::concat: {
                const ir::node& l = g.at(n.lhs);
                const int64_t split = l.out[n.axis];
                const ival& axis_coord = coords[n.axis];
                knode s;
                s.op = kop::select;
                s.cond.lhs = axis_coord;
                s.cond.bound = split;
                // Branch-local coordinate ranges: when the axis coordinate
                // is one kernel coordinate (plus a constant), each branch
                // narrows that coordinate's range.
                int single = -1;
                if (axis_coord.is_affine) {
                    for (size_t d = 0; d < rank; ++d) {
                        if (axis_coord.w[d] == 0) continue;
                        if (axis_coord.w[d] == 1 && single < 0)
                            single = static_cast<int>(d);
                        else {
                            single = -2;
                            break;
                        }
                    }
                }
                const auto saved = box;
                bool lhs_live = true;
                bool rhs_live = true;
                if (single >= 0) {
                    const auto& r = box[static_cast<size_t>(single)];
                    const int64_t cut = split - axis_coord.c0;
                    lhs_live = r.first < std::min(r.second, cut);
                    rhs_live = std::max(r.first, cut) < r.second;
                }
                std::vector<ival> rcoords = coords;
                rcoords[n.axis] = add_constant(axis_coord, -split);
                // A branch no element of the current range takes is not
                // lowered at all (e.g. concat with an empty operand).
                if (!lhs_live) {
                    auto& r = box[static_cast<size_t>(single)];
                    r.first = std::max(r.first, split - axis_coord.c0);
                    const int result = at(n.rhs, rcoords);
                    box = saved;
                    return result;
                }
                if (!rhs_live) {
                    auto& r = box[static_cast<size_t>(single)];
                    r.second = std::min(r.second, split - axis_coord.c0);
                    const int result = at(n.lhs, coords);
                    box = saved;
                    return result;
                }
                if (single >= 0) {
                    auto& r = box[static_cast<size_t>(single)];
                    r.second = std::min(r.second, split - axis_coord.c0);
                }
                s.a = at(n.lhs, coords);
                box = saved;
                if (single >= 0) {
                    auto& r = box[static_cast<size_t>(single)];
                    r.first = std::max(r.first, split - axis_coord.c0);
                }
                s.b = at(n.rhs, rcoords);
                box = saved;
                return out.add(s);
            }
            case ir::op::sum:
            case ir::op::max:
            case ir::op::matmul:
            case ir::op::batched_matmul:
                throw std::logic_error(
                    "reduction or matmul reached the pointwise lowering"
                );
        }
        throw std::invalid_argument("unknown tensor expression node");
    }

    std::string float_literal(float value) {
        uint32_t bits = 0;
        std::memcpy(&bits, &value, sizeof bits);
        char text[64];
        if (std::isfinite(value)) {
            // 9 significant digits round-trip every finite float exactly.
            std::snprintf(text, sizeof text, "%.9g", static_cast<double>(value));
            std::string s{text};
            if (s.find_first_of(".eE") == std::string::npos) s += ".0";
            return s + "f";
        }
        // Infinities and NaNs by bit pattern.
        std::snprintf(text, sizeof text, "__uint_as_float(0x%08xu)", bits);
        return text;
    }

} // namespace porch::cg
