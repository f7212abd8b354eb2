#pragma once

// Emission of a kernel expression as straight-line HIP with common
// subexpressions shared, `width` lanes of values per node (1 or 4), and
// select nodes emitted as real branches so a branch's loads only run when
// it is taken.  Arithmetic is IEEE binary32 exactly as written (kernels are
// compiled with -ffp-contract=off); maximum/minimum keep the reference's
// ternary NaN behaviour (reference src/tensor.cpp:677-682).

#include "lower.hpp"
#include "range.hpp"

#include <functional>
#include <map>
#include <string>
#include <vector>

namespace porch::cg {

    struct emitter {
        const kexpr& k;
        std::string& code;
        std::string indent = "    ";
        int width = 1;

        // Values of a load node, one expression per lane (may emit
        // statements first).
        std::function<std::vector<std::string>(int id)> load;
        // Optional override for any node (e.g. LDS-staged subtrees);
        // returns an empty vector to fall through.
        std::function<std::vector<std::string>(int id)> override_node;
        // The value of row reduction `row` (uniform across lanes).
        std::function<std::string(int row)> row_value;
        // Condition text of a select (evaluated once; uniform across lanes).
        std::function<std::string(const kcond& c)> condition;
        // Optional: the branch select `id` takes wherever this code runs
        // (0: first operand, 1: second), or -1 to branch at run time.
        std::function<int(int id)> forced_branch;
        // Optional inputs of the value-range analysis (range.hpp) that picks
        // the fast exact reciprocal and the overflow-free exp.
        std::function<vrange(int row)> row_value_range;
        std::function<vrange(int id, const vrange& computed)> refine_range;

        emitter(const kexpr& expr, std::string& target, int lanes);

        std::vector<std::string> emit(int id);
        std::string fresh(const char* prefix);
        void line(const std::string& text);
        // `if (condition) {` with a scope of its own: values emitted until
        // close_scope() are not reused after it.
        void open_scope(const std::string& condition);
        void close_scope();

        // Range of node `id` (computed once, on first use).
        const vrange& range_of(int id);

        // The nodes whose values leave the expression (stored, reduced,
        // staged).  Until they are declared, no node counts as consumed only
        // inside the expression.
        void declare_roots(std::vector<int> ids);
        // Is every use of `id` an addition or subtraction of a constant c
        // with |c| >= 2^-100?  Then c + v rounds to c for any denormal v, so a
        // denormal value of `id` may be flushed to zero unseen.
        bool denormals_absorbed(int id);
        // Is every use of `id` an addition or subtraction of a constant of
        // magnitude >= `least` (and is there at least one)?
        bool only_added_to_constants(int id, float least);

        // Optional: nodes whose values reach the kernel's result only through
        // a sum that is the result itself (a row program's final sum).  The
        // result is compared within a relative tolerance, so these nodes may
        // use instruction sequences a few ulp from correctly rounded.
        std::function<bool(int id)> relaxed;

        // The multiply operand of add/subtract `id` that may fuse into it as
        // an fma: both relaxed, the product used nowhere else and not yet
        // emitted; -1 if none.
        int fusable_product(int id);

      private:
        std::vector<std::map<int, std::vector<std::string>>> frames_;
        std::vector<vrange> ranges_;
        std::vector<int> roots_;
        bool roots_declared_ = false;
        int counter_ = 0;
        const std::vector<std::string>* find(int id) const;
    };

    // Index text of an affine/generic ival with coordinate q_d renamed
    // through `names` (names[d] is the C expression for coordinate d).
    std::string index_text(const ival& v, const std::vector<std::string>& names);

    // Declarations `const T q{d} = ...;` decomposing a flat index over
    // `shape` (only coordinates in `needed` are declared).
    std::string decompose(const std::string& flat, const std::vector<int64_t>& shape,
                          const std::vector<bool>& needed, const char* type,
                          const std::string& indent);

    // Which kernel coordinates any index or condition under `root` uses.
    std::vector<bool> used_coordinates(const kexpr& k, int root, size_t rank);

    std::string kernel_prologue(int n_slots, const char* index_type);
    std::string kernel_params(int n_slots);

} // namespace porch::cg
