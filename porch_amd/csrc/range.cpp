#include "range.hpp"

#include <algorithm>
#include <cmath>
#include <limits>

namespace porch::cg {

    namespace {
        constexpr float inf = std::numeric_limits<float>::infinity();

        vrange hull(const vrange& a, const vrange& b) {
            return {std::min(a.lo, b.lo), std::max(a.hi, b.hi), a.nan || b.nan};
        }

        // The node can only be NaN (e.g. a NaN constant).
        bool nan_only(const vrange& r) {
            return r.lo > r.hi;
        }

        vrange only_nan() {
            return {inf, -inf, true};
        }

        bool unbounded(const vrange& r) {
            return std::isinf(r.lo) || std::isinf(r.hi);
        }

        bool contains_zero(const vrange& r) {
            return r.lo <= 0.0F && r.hi >= 0.0F;
        }

        // Extremes of f over the four endpoint pairs (none may be NaN).
        template <typename F>
        vrange corners(const vrange& a, const vrange& b, bool nan, F f) {
            const float c[4] = {f(a.lo, b.lo), f(a.lo, b.hi), f(a.hi, b.lo), f(a.hi, b.hi)};
            vrange r{c[0], c[0], nan};
            for (const float v : c) {
                if (std::isnan(v)) return vrange::any();
                r.lo = std::min(r.lo, v);
                r.hi = std::max(r.hi, v);
            }
            return r;
        }

        // Volatile operands keep the host compiler from contracting or
        // reassociating: each endpoint is one binary32 operation.
        float add(float a, float b) { volatile float r = a + b; return r; }
        float sub(float a, float b) { volatile float r = a - b; return r; }
        float mul(float a, float b) { volatile float r = a * b; return r; }
        float div(float a, float b) { volatile float r = a / b; return r; }

        vrange range_add(const vrange& a, const vrange& b) {
            if (nan_only(a) || nan_only(b)) return only_nan();
            // inf + -inf is the only NaN source
            const bool nan = a.nan || b.nan || (a.hi == inf && b.lo == -inf) ||
                             (a.lo == -inf && b.hi == inf);
            return {add(a.lo, b.lo), add(a.hi, b.hi), nan};
        }

        vrange range_sub(const vrange& a, const vrange& b) {
            if (nan_only(a) || nan_only(b)) return only_nan();
            const bool nan = a.nan || b.nan || (a.hi == inf && b.hi == inf) ||
                             (a.lo == -inf && b.lo == -inf);
            return {sub(a.lo, b.hi), sub(a.hi, b.lo), nan};
        }

        vrange range_mul(const vrange& a, const vrange& b) {
            if (nan_only(a) || nan_only(b)) return only_nan();
            if ((contains_zero(a) && unbounded(b)) || (contains_zero(b) && unbounded(a)))
                return vrange::any();
            return corners(a, b, a.nan || b.nan, mul);
        }

        vrange range_div(const vrange& a, const vrange& b) {
            if (nan_only(a) || nan_only(b)) return only_nan();
            if (contains_zero(b) || (unbounded(a) && unbounded(b))) return vrange::any();
            return corners(a, b, a.nan || b.nan, div);
        }
    } // namespace

    vrange vrange::any() {
        return {-inf, inf, true};
    }

    vrange vrange::exactly(float v) {
        if (std::isnan(v)) return only_nan();
        return {v, v, false};
    }

    bool reciprocal_is_tame(const vrange& r) {
        const float small = std::ldexp(1.0F, -125);
        const float large = std::ldexp(1.0F, 125);
        // NaN propagates through the fast sequence unchanged.
        if (nan_only(r)) return true;
        return (r.lo >= small && r.hi <= large) || (r.hi <= -small && r.lo >= -large);
    }

    std::vector<vrange> value_ranges(
        const kexpr& k, const std::function<vrange(int row)>& row_value_range,
        const std::function<vrange(int id, const vrange& computed)>& refine
    ) {
        std::vector<vrange> r(k.nodes.size(), vrange::any());
        // Operands always precede their users in the arena.
        for (size_t i = 0; i < k.nodes.size(); ++i) {
            const knode& n = k.nodes[i];
            vrange v = vrange::any();
            switch (n.op) {
                case kop::constant: v = vrange::exactly(n.value); break;
                case kop::load: v = vrange::any(); break;
                case kop::row_value:
                    v = row_value_range ? row_value_range(n.row) : vrange::any();
                    break;
                case kop::add: v = range_add(r[n.a], r[n.b]); break;
                case kop::subtract: v = range_sub(r[n.a], r[n.b]); break;
                case kop::multiply: v = range_mul(r[n.a], r[n.b]); break;
                case kop::divide: v = range_div(r[n.a], r[n.b]); break;
                case kop::maximum: {
                    // a > b ? a : b — a NaN a yields b; a NaN b yields b.
                    const vrange& a = r[n.a];
                    const vrange& b = r[n.b];
                    v = {a.nan ? b.lo : std::max(a.lo, b.lo), std::max(a.hi, b.hi), b.nan};
                    if (nan_only(a) || nan_only(b)) v = b;
                    break;
                }
                case kop::minimum: {
                    // a < b ? a : b
                    const vrange& a = r[n.a];
                    const vrange& b = r[n.b];
                    v = {std::min(a.lo, b.lo), a.nan ? b.hi : std::min(a.hi, b.hi), b.nan};
                    if (nan_only(a) || nan_only(b)) v = b;
                    break;
                }
                case kop::exp: {
                    const vrange& a = r[n.a];
                    // exp is monotone; widen by far more than its few-ulp
                    // error so rounding never escapes the bounds.
                    double lo = std::exp(static_cast<double>(a.lo)) * (1.0 - 1e-6);
                    if (lo < 1e-30) lo = 0.0; // denormal results: no relative bound
                    const double hi = std::exp(static_cast<double>(a.hi)) * (1.0 + 1e-6);
                    v = {static_cast<float>(std::max(lo, 0.0)),
                         hi > 3.4e38 ? inf : static_cast<float>(hi), a.nan};
                    if (nan_only(a)) v = a;
                    break;
                }
                case kop::reciprocal: {
                    const vrange& a = r[n.a];
                    if (nan_only(a)) v = a;
                    else if (contains_zero(a)) v = vrange::any();
                    else v = {div(1.0F, a.hi), div(1.0F, a.lo), a.nan};
                    break;
                }
                case kop::select: v = hull(r[n.a], r[n.b]); break;
            }
            if (refine) v = refine(static_cast<int>(i), v);
            r[i] = v;
        }
        return r;
    }

} // namespace porch::cg
