// Runs a kernel over its grid on the CPU (see prelude.hpp), with every
// buffer placed against an inaccessible guard region.  TEST INFRASTRUCTURE.
#pragma once

#include <sys/mman.h>
#include <unistd.h>

#include <barrier>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <memory>
#include <string>
#include <thread>
#include <vector>

namespace emu {

    // `floats` floats with PROT_NONE guards of `guard` bytes on both sides;
    // the data ends at the upper guard (tail = true: a read past the end
    // faults) or starts at the lower one (tail = false: a read before the
    // start faults).  Starts stay 16-byte aligned, as device allocations
    // are (at least) and as the kernels' 128-bit accesses assume, so a tail
    // buffer ends up to 12 bytes short of its guard: reads into that part
    // of the last 16-byte block go unseen, as they stay inside a device
    // allocation.
    inline float* guarded(size_t floats, bool tail) {
        const size_t page = static_cast<size_t>(sysconf(_SC_PAGESIZE));
        const size_t guard = size_t{1} << 30;
        const size_t bytes = floats * sizeof(float);
        const size_t span = (bytes + page - 1) / page * page + page;
        char* base = static_cast<char*>(mmap(nullptr, guard + span + guard, PROT_NONE,
                                             MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0));
        if (base == MAP_FAILED) {
            std::perror("mmap");
            std::exit(3);
        }
        char* data_region = base + guard;
        if (mprotect(data_region, span, PROT_READ | PROT_WRITE) != 0) {
            std::perror("mprotect");
            std::exit(3);
        }
        char* start = tail ? data_region + ((span - bytes) & ~size_t{15}) : data_region;
        float* f = reinterpret_cast<float*>(start);
        for (size_t i = 0; i < floats; ++i) f[i] = static_cast<float>(static_cast<int>(i % 7) - 3);
        return f;
    }

    // Values mode: buffer i takes the floats of <dir>/b<i>.bin when that
    // file exists, and the destination is written to <dir>/out.bin.
    inline void load(float* b, size_t floats, const char* dir, int i) {
        if (dir == nullptr) return;
        const std::string path = std::string(dir) + "/b" + std::to_string(i) + ".bin";
        FILE* f = std::fopen(path.c_str(), "rb");
        if (f == nullptr) return;
        if (std::fread(b, sizeof(float), floats, f) != floats) std::exit(4);
        std::fclose(f);
    }
    inline void save(const float* b, size_t floats, const char* dir) {
        if (dir == nullptr) return;
        const std::string path = std::string(dir) + "/out.bin";
        FILE* f = std::fopen(path.c_str(), "wb");
        if (f == nullptr || std::fwrite(b, sizeof(float), floats, f) != floats) std::exit(4);
        std::fclose(f);
    }

    // Runs every block of `grid`, or only the x indices in `only` (the
    // grid size seen by the kernel stays `grid`).
    inline void run(dim3 grid, unsigned block, const std::function<void()>& kernel,
                    std::vector<unsigned> only = {}) {
        grid_dim = grid;
        block_dim = {block, 1, 1};
        std::barrier<> blocks(static_cast<std::ptrdiff_t>(block));
        std::barrier<> sync(static_cast<std::ptrdiff_t>(block));
        std::vector<std::unique_ptr<std::barrier<>>> waves;
        for (unsigned w = 0; w < (block + 63) / 64; ++w) {
            waves.push_back(std::make_unique<std::barrier<>>(static_cast<std::ptrdiff_t>(block - 64 * w < 64 ? block - 64 * w : 64)));
            wave_barrier[w] = waves.back().get();
        }
        block_barrier = &sync;
        std::vector<std::thread> threads;
        for (unsigned t = 0; t < block; ++t) {
            threads.emplace_back([&, t] {
                thread_idx = {t, 0, 0};
                for (unsigned z = 0; z < grid.z; ++z)
                    for (unsigned y = 0; y < grid.y; ++y)
                        for (unsigned i = 0; i < (only.empty() ? grid.x : only.size()); ++i) {
                            block_idx = {only.empty() ? i : only[i], y, z};
                            kernel();
                            blocks.arrive_and_wait();
                        }
            });
        }
        for (std::thread& t : threads) t.join();
    }

} // namespace emu
