// Seeded synthetic inputs.  Output i of a splitmix64 stream depends only on
// (seed, i): the state after i+1 steps is seed + (i+1) * 0x9E3779B97F4A7C15,
// so the generator is filled in parallel and is identical in every process
// and on every machine.

#include "porch_amd.h"

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

namespace {

    constexpr uint64_t golden = 0x9E3779B97F4A7C15ULL;

    inline uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
        uint64_t z = seed + (i + 1) * golden;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        return z ^ (z >> 31);
    }

    // 24-bit uniform in [0, 1).
    inline double unit(uint64_t x) { return static_cast<double>(x >> 40) * 0x1.0p-24; }

    template <typename F>
    void parallel_for(size_t count, F&& body) {
        const size_t hw = std::max(1U, std::thread::hardware_concurrency());
        const size_t workers = std::min<size_t>(std::min<size_t>(hw, 16), (count >> 16) + 1);
        if (workers <= 1) {
            body(size_t{0}, count);
            return;
        }
        std::vector<std::thread> threads;
        const size_t chunk = (count + workers - 1) / workers;
        for (size_t w = 0; w < workers; ++w) {
            const size_t begin = std::min(count, w * chunk);
            const size_t end = std::min(count, begin + chunk);
            threads.emplace_back([&body, begin, end] { body(begin, end); });
        }
        for (std::thread& t : threads) t.join();
    }

} // namespace

extern "C" {

void porch_synth_uniform(float* out, size_t count, uint64_t seed, double lo, double hi) {
    if (out == nullptr) return;
    parallel_for(count, [=](size_t begin, size_t end) {
        for (size_t i = begin; i < end; ++i)
            out[i] = static_cast<float>(lo + (hi - lo) * unit(splitmix64_at(seed, i)));
    });
}

void porch_synth_normal(float* out, size_t count, uint64_t seed, double mean, double stddev) {
    if (out == nullptr) return;
    const size_t pairs = (count + 1) / 2;
    parallel_for(pairs, [=](size_t begin, size_t end) {
        constexpr double two_pi = 6.283185307179586476925286766559;
        for (size_t j = begin; j < end; ++j) {
            // u1 in (0, 1] keeps the logarithm finite.
            const double u1 =
                static_cast<double>((splitmix64_at(seed, 2 * j) >> 40) + 1) * 0x1.0p-24;
            const double u2 = unit(splitmix64_at(seed, 2 * j + 1));
            const double radius = std::sqrt(-2.0 * std::log(u1));
            const double angle = two_pi * u2;
            out[2 * j] = static_cast<float>(mean + stddev * radius * std::cos(angle));
            if (2 * j + 1 < count)
                out[2 * j + 1] = static_cast<float>(mean + stddev * radius * std::sin(angle));
        }
    });
}

void porch_synth_replace(float* out, size_t count, uint64_t seed, double p, float value) {
    if (out == nullptr) return;
    parallel_for(count, [=](size_t begin, size_t end) {
        for (size_t i = begin; i < end; ++i) {
            if (unit(splitmix64_at(seed, i)) < p) out[i] = value;
        }
    });
}

} // extern "C"
