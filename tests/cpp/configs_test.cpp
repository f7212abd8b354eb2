// The five benchmark graphs built with porch's public C++ API (porch::tensor,
// porch::ops, the tensor_expr operators) over the seeded synthetic inputs
// (porch_synth_*, the generator the Python side uses), materialised on the
// GPU, with the result's values written to a file.  Built by
// tests/cpp/Makefile; tests/test_cpp_configs.py compares the files with the
// oracle and with the same graphs materialised through the Python mirror.
//
//   configs_test <config> <output file> [sizes]
//     elementwise      n              (a + b) * 2 - 1
//     view_chain       n              concat(transpose(x[0::2, 1::2]),
//                                            transpose(x[1::2, 0::2]), 0) + 1
//     softmax          rows cols      softmax(x, 1)
//     logistic_rowsum  rows cols      sum(logistic(relu(x * w + bias)), 1)
//     matmul_epilogue  m k n          relu(A @ B + bias) - 0.5
// Without sizes, each graph runs at its benchmark size.

#include <porch/ops.hpp>
#include <porch/tensor.hpp>

#include "porch_amd.h"

#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

    using porch::index_t;

    std::vector<float> uniform(size_t n, uint64_t seed, double lo, double hi) {
        std::vector<float> v(n);
        porch_synth_uniform(v.data(), n, seed, lo, hi);
        return v;
    }

    std::vector<float> normal(size_t n, uint64_t seed, double mean, double stddev) {
        std::vector<float> v(n);
        porch_synth_normal(v.data(), n, seed, mean, stddev);
        return v;
    }

    index_t size_arg(int argc, char** argv, int i, index_t fallback) {
        return argc > i ? static_cast<index_t>(std::stoll(argv[i])) : fallback;
    }

    porch::tensor run(const std::string& name, int argc, char** argv) {
        if (name == "elementwise") {
            const index_t n = size_arg(argc, argv, 3, index_t{1} << 20);
            const porch::tensor a({n}, uniform(n, 101, -1.0, 1.0));
            const porch::tensor b({n}, uniform(n, 102, -1.0, 1.0));
            return (a + b) * 2.0F - 1.0F;
        }
        if (name == "view_chain") {
            const index_t n = size_arg(argc, argv, 3, 4096);
            const porch::tensor x({n, n}, normal(static_cast<size_t>(n * n), 201, 0.0, 1.0));
            return porch::concat(porch::transpose(x[{porch::slice{0, n, 2}, porch::slice{1, n, 2}}]),
                                 porch::transpose(x[{porch::slice{1, n, 2}, porch::slice{0, n, 2}}]), 0) +
                   1.0F;
        }
        if (name == "softmax") {
            const index_t rows = size_arg(argc, argv, 3, 8192);
            const index_t cols = size_arg(argc, argv, 4, 4096);
            std::vector<float> values = normal(static_cast<size_t>(rows * cols), 301, 0.0, 3.0);
            porch_synth_replace(values.data(), values.size(), 302, 0.01, 20.0F);
            const porch::tensor x({rows, cols}, std::move(values));
            return porch::softmax(x, 1);
        }
        if (name == "logistic_rowsum") {
            const index_t rows = size_arg(argc, argv, 3, 16384);
            const index_t cols = size_arg(argc, argv, 4, 2048);
            const porch::tensor x({rows, cols}, normal(static_cast<size_t>(rows * cols), 401, 0.0, 1.0));
            const porch::tensor w({1, cols}, uniform(static_cast<size_t>(cols), 402, 0.5, 1.5));
            const porch::tensor bias({1, cols}, normal(static_cast<size_t>(cols), 403, 0.0, 0.1));
            return porch::sum(porch::logistic(porch::relu(x * porch::broadcast_to(w, {rows, cols}) +
                                                          porch::broadcast_to(bias, {rows, cols}))),
                              1);
        }
        if (name == "matmul_epilogue") {
            const index_t m = size_arg(argc, argv, 3, 4096);
            const index_t k = size_arg(argc, argv, 4, 4096);
            const index_t n = size_arg(argc, argv, 5, 4096);
            std::vector<float> a = uniform(static_cast<size_t>(m * k), 501, -1.0, 1.0);
            std::vector<float> b = uniform(static_cast<size_t>(k * n), 502, -1.0, 1.0);
            for (float& v : a) v /= 64.0F;
            for (float& v : b) v /= 64.0F;
            const porch::tensor ta({m, k}, std::move(a));
            const porch::tensor tb({k, n}, std::move(b));
            const porch::tensor bias({1, n}, normal(static_cast<size_t>(n), 503, 0.0, 0.01));
            return porch::relu(porch::matmul(ta, tb) + porch::broadcast_to(bias, {m, n})) - 0.5F;
        }
        throw std::invalid_argument("unknown config: " + name);
    }

} // namespace

int main(int argc, char** argv) {
    if (argc < 3) {
        std::puts("elementwise view_chain softmax logistic_rowsum matmul_epilogue");
        return argc == 1 ? 0 : 2;
    }
    try {
        const porch::tensor result = run(argv[1], argc, argv);
        const std::span<const float> values = result.data();
        std::FILE* f = std::fopen(argv[2], "wb");
        if (f == nullptr) throw std::runtime_error(std::string("cannot write ") + argv[2]);
        const bool ok = std::fwrite(values.data(), sizeof(float), values.size(), f) == values.size();
        if (std::fclose(f) != 0 || !ok) throw std::runtime_error(std::string("write failed: ") + argv[2]);
        std::printf("%s: %zu values, shape", argv[1], values.size());
        for (const index_t d : result.shape()) std::printf(" %lld", static_cast<long long>(d));
        std::printf("\n");
        return 0;
    }
    catch (const std::exception& e) {
        std::fprintf(stderr, "%s\n", e.what());
        return 1;
    }
}
