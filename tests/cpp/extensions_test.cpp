// The C++ API of this backend's IR extensions (permute, batched_matmul and
// tensors over strided storage), exercised the way porch's own test program
// exercises the rest of the API: one named case per run, exit status 0 on
// success.  Built by tests/cpp/Makefile against include/porch/*.hpp and
// libporch_amd.so; driven by tests/test_cpp_extensions.py.

#include <porch/ops.hpp>
#include <porch/tensor.hpp>

#include <cstdio>
#include <functional>
#include <map>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

    using porch::index_t;

    void require(bool condition, const std::string& what) {
        if (!condition) throw std::runtime_error("check failed: " + what);
    }

    template <class Fn>
    void require_invalid(Fn&& fn, const std::string& message) {
        try {
            fn();
        }
        catch (const std::invalid_argument& e) {
            require(std::string(e.what()) == message,
                    "message '" + std::string(e.what()) + "' == '" + message + "'");
            return;
        }
        throw std::runtime_error("expected std::invalid_argument: " + message);
    }

    std::vector<float> iota(size_t n, float from = 0.0F) {
        std::vector<float> v(n);
        std::iota(v.begin(), v.end(), from);
        return v;
    }

    // ---- no device needed ----

    void permute_shape_is_lazy_metadata() {
        const porch::tensor empty({0, 3, 4}, {});
        const porch::tensor_expr p = porch::permute(empty, {2, 0, 1});
        require(p.shape() == std::vector<index_t>{4, 0, 3}, "permuted shape");
    }

    void permute_rejects_non_permutations() {
        const porch::tensor empty({0, 3, 4}, {});
        for (const std::vector<size_t>& dims :
             {std::vector<size_t>{0, 0, 1}, std::vector<size_t>{0, 1}, std::vector<size_t>{0, 1, 3}}) {
            require_invalid([&] { (void)porch::permute(empty, dims).shape(); },
                            "permute axes must be a permutation of the operand's dimensions");
        }
        require_invalid([] { (void)porch::permute(porch::tensor_expr{1.0F}, {}).shape(); },
                        "permute operand must be a tensor");
    }

    void batched_matmul_rejects_shapes() {
        const porch::tensor a({0, 3, 4}, {});
        const porch::tensor b({2, 4, 0}, {});
        const porch::tensor c({0, 5, 6}, {});
        const porch::tensor m({3, 0}, {});
        require_invalid([&] { (void)porch::batched_matmul(a, b).shape(); },
                        "batched_matmul batch dimensions must match");
        require_invalid([&] { (void)porch::batched_matmul(a, c).shape(); },
                        "batched_matmul inner dimensions must match");
        require_invalid([&] { (void)porch::batched_matmul(m, m).shape(); },
                        "batched_matmul requires rank-3 tensors");
        const porch::tensor d({0, 4, 7}, {});
        require(porch::batched_matmul(a, d).shape() == std::vector<index_t>{0, 3, 7}, "batched shape");
    }

    void strided_storage_must_cover_the_layout() {
        require_invalid(
            [] {
                porch::tensor t(porch::tensor_layout({4, 4}, {1, 4}, 0), porch::cuda_jit::device_buffer{});
            },
            "tensor device storage is too small");
    }

    // ---- on the device ----

    void permute_values() {
        const porch::tensor x({2, 3, 4}, iota(24));
        const porch::tensor y = porch::permute(x, {2, 0, 1});
        require(y.shape()[0] == 4 && y.shape()[1] == 2 && y.shape()[2] == 3, "shape");
        const std::vector<float> v = y.cpu();
        for (index_t i = 0; i < 4; ++i)
            for (index_t j = 0; j < 2; ++j)
                for (index_t k = 0; k < 3; ++k)
                    require(v[static_cast<size_t>((i * 2 + j) * 3 + k)] ==
                                static_cast<float>(j * 12 + k * 4 + i),
                            "permuted value");
    }

    void batched_matmul_values() {
        const porch::tensor a({2, 2, 3}, iota(12, 1.0F));
        const porch::tensor b({2, 3, 2}, iota(12, -5.0F));
        const porch::tensor c = porch::relu(porch::batched_matmul(a, b) + 1.0F);
        const std::vector<float> v = c.cpu();
        for (int e = 0; e < 2; ++e)
            for (int i = 0; i < 2; ++i)
                for (int j = 0; j < 2; ++j) {
                    float s = 0.0F;
                    for (int k = 0; k < 3; ++k)
                        s += (1.0F + static_cast<float>(e * 6 + i * 3 + k)) *
                             (-5.0F + static_cast<float>(e * 6 + k * 2 + j));
                    const float expected = s + 1.0F > 0.0F ? s + 1.0F : 0.0F;
                    require(v[static_cast<size_t>((e * 2 + i) * 2 + j)] == expected, "product value");
                }
    }

    void strided_tensor_reads_its_layout() {
        const porch::tensor base({30}, iota(30));
        // a [3, 4] view with strides {1, 5} at offset 2: x[i][j] = 2 + i + 5j
        const porch::tensor t(porch::tensor_layout({3, 4}, {1, 5}, 2), base.device_data());
        require(!t.is_contiguous() && t.storage_offset() == 2 && t.strides()[1] == 5, "layout");
        const std::vector<float> v = t.cpu();
        for (int i = 0; i < 3; ++i)
            for (int j = 0; j < 4; ++j)
                require(v[static_cast<size_t>(i * 4 + j)] == static_cast<float>(2 + i + 5 * j), "gathered");
        const porch::tensor doubled = t * 2.0F + 1.0F;
        const std::vector<float> d = doubled.cpu();
        for (int i = 0; i < 3; ++i)
            for (int j = 0; j < 4; ++j)
                require(d[static_cast<size_t>(i * 4 + j)] == 2.0F * static_cast<float>(2 + i + 5 * j) + 1.0F,
                        "expression over strided storage");
        // slicing composes with the layout: rows 0 and 2, columns 1..3
        const porch::tensor s = t[{porch::slice{0, 3, 2}, porch::slice{1, 4}}];
        const std::vector<float> sv = s.cpu();
        require(sv.size() == 6, "slice size");
        for (int i = 0; i < 2; ++i)
            for (int j = 0; j < 3; ++j)
                require(sv[static_cast<size_t>(i * 3 + j)] == static_cast<float>(2 + 2 * i + 5 * (j + 1)),
                        "sliced strided value");
    }

    const std::map<std::string, std::function<void()>>& cases() {
        static const std::map<std::string, std::function<void()>> all{
            {"permute_shape_is_lazy_metadata", permute_shape_is_lazy_metadata},
            {"permute_rejects_non_permutations", permute_rejects_non_permutations},
            {"batched_matmul_rejects_shapes", batched_matmul_rejects_shapes},
            {"strided_storage_must_cover_the_layout", strided_storage_must_cover_the_layout},
            {"permute_values", permute_values},
            {"batched_matmul_values", batched_matmul_values},
            {"strided_tensor_reads_its_layout", strided_tensor_reads_its_layout},
        };
        return all;
    }

} // namespace

int main(int argc, char** argv) {
    if (argc != 2) {
        for (const auto& [name, fn] : cases()) std::printf("%s\n", name.c_str());
        return 0;
    }
    const auto found = cases().find(argv[1]);
    if (found == cases().end()) {
        std::fprintf(stderr, "unknown case %s\n", argv[1]);
        return 2;
    }
    try {
        found->second();
    }
    catch (const std::exception& e) {
        std::fprintf(stderr, "%s: %s\n", argv[1], e.what());
        return 1;
    }
    std::printf("%s: ok\n", argv[1]);
    return 0;
}
