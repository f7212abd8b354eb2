#pragma once

// Process-wide HIP device, per-thread streams, stream-ordered buffers,
// hiprtc code-object cache and module launches.  The MI355X counterpart of
// the reference's cuda_environment / stream_handle / device_buffer_state
// (reference src/cuda_jit.cpp:437-627), re-designed around HIP:
//   * one device (ordinal 0) initialised once; no contexts (hipCtx* is
//     deprecated on ROCm);
//   * one non-blocking, default-priority stream per thread, held by
//     shared_ptr so buffers can outlive the thread that made them;
//   * cross-stream order by hipEventRecord + hipStreamWaitEvent instead of
//     host synchronisation; the host waits only in copy_to_host and
//     synchronize();
//   * hipMallocAsync/hipFreeAsync from the default pool with an unbounded
//     release threshold, so steady-state allocation never reaches the OS;
//   * code objects cached by (source, options); modules and kernel handles
//     cached by code object, so no launch loads a module.

#include "hip_api.hpp"

#include <chrono>
#include <memory>
#include <mutex>
#include <string>
#include <string_view>
#include <vector>

namespace porch::rt {

    struct device_info {
        int ordinal = 0;
        int compute_units = 0;
        int clock_khz = 0;
        int l2_bytes = 0;
        std::string arch; // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
    };

    // Initialises HIP and device 0 on first use; throws runtime_error.
    const device_info& device();

    class stream {
      public:
        stream();
        ~stream();
        stream(const stream&) = delete;
        stream& operator=(const stream&) = delete;

        [[nodiscard]] hip::stream_t handle() const noexcept { return handle_; }
        void synchronize() const;

      private:
        hip::stream_t handle_ = nullptr;
    };

    // The calling thread's stream (created on first use).
    std::shared_ptr<stream> current_stream();

    // Device blocks come from hipMallocAsync on a stream; a released block
    // goes to that stream's free list and is handed to the next allocation
    // of a fitting size on the same stream with no HIP call (stream order
    // already puts the new user after the old one).  Cached blocks beyond
    // a limit, and all of a stream's blocks when the stream is destroyed,
    // go back through hipFreeAsync.
    void* allocate_block(size_t bytes, const stream& s, size_t* capacity);
    void release_block(void* ptr, size_t capacity, const stream& s);
    void release_stream_blocks(const stream& s);
    size_t cached_block_bytes();
    // Returns every cached block to the stream-ordered pool (hipFreeAsync
    // on its stream); the bytes released.
    size_t release_cached_blocks();

    // Makes `consumer` wait for all work queued so far on `producer`.
    void order_after(const stream& consumer, const stream& producer);

    // A host-to-device copy that returns before the DMA ends: the source is
    // copied (by several host threads when large) into pinned staging chunks
    // (hipHostMalloc) in pieces of at most 32 MiB, each piece's DMA is queued
    // on `s` as soon as it is staged, and a chunk is reused once an event
    // recorded after its DMA has completed.  Chunks (powers of two from
    // 1 MiB) are pooled up to 512 MiB of pinned memory.  Returns false,
    // having done nothing, only when no chunk can be had.
    bool upload_staged(void* dst, const void* src, size_t bytes, const stream& s);
    // A device-to-host copy through the same pinned chunks, pipelined:
    // waits until `dst` holds the data.  Returns false, having done
    // nothing, only when no chunk can be had.
    bool download_staged(void* dst, const void* src, size_t bytes, const stream& s);
    // Pinned bytes held by the staging pool.
    size_t staging_bytes();

    struct buffer_state {
        explicit buffer_state(size_t requested_bytes);
        ~buffer_state();
        buffer_state(const buffer_state&) = delete;
        buffer_state& operator=(const buffer_state&) = delete;

        void* ptr = nullptr;
        size_t bytes = 0;
        size_t capacity = 0; // size of the block behind ptr (>= bytes)

        // Orders stream `s` after the last write (and, for writes, after
        // readers on other streams) and records the access.
        void before_read(const std::shared_ptr<stream>& s);
        void before_write(const std::shared_ptr<stream>& s);
        void after_write(const std::shared_ptr<stream>& s);
        std::shared_ptr<stream> producer_stream() const;

      private:
        mutable std::mutex mutex_;
        std::shared_ptr<stream> producer_;
        std::vector<std::shared_ptr<stream>> readers_;
    };

    // hiprtc compile for the current GPU architecture, cached by
    // (source, options).  Failure throws compilation_error with the log.
    struct code_object {
        std::string bytes;
        double compile_ms = 0.0; // 0 on a cache hit
    };
    std::shared_ptr<const code_object> compile(
        std::string_view source, const std::vector<std::string>& extra_options
    );
    // The options every porch kernel is compiled with (arch, -O3,
    // -ffp-contract=off, packed-FP32 disabled).
    std::vector<std::string> default_options();
    std::string target_arch();

    struct kernel_handle {
        hip::function_t function = nullptr;
        int registers = 0;
        int lds_bytes = 0;
        int scratch_bytes = 0;
    };
    // Loads (once per code object) and returns the kernel.
    kernel_handle load_kernel(
        const std::shared_ptr<const code_object>& code, std::string_view name
    );

    // Launches on stream `s`.  With `start`/`stop` the launch goes through
    // hipExtModuleLaunchKernel, whose events are timestamped by the
    // dispatch itself (no extra barrier packets between them).
    void launch(
        const kernel_handle& kernel, unsigned grid_x, unsigned grid_y,
        unsigned grid_z, unsigned block_x, unsigned shared_bytes,
        void** params, const stream& s, hip::event_t start = nullptr,
        hip::event_t stop = nullptr
    );

    void clear_caches();

    struct jit_counters {
        uint64_t plan_hits = 0;
        uint64_t plan_misses = 0;
        uint64_t compiles = 0;
        uint64_t launches = 0;
        double codegen_ms = 0;
        double compile_ms = 0;
        double module_load_ms = 0;
        double last_miss_ms = 0;
        double last_hit_us = 0;
        uint64_t disk_hits = 0;  // code objects read from the on-disk cache
        double disk_ms = 0;      // host time reading them
    };
    jit_counters& counters();
    std::mutex& counters_mutex();

    // Scratch writes that evict L2 and the Infinity Cache (benchmarks).
    void flush_caches(size_t bytes);

    inline double elapsed_ms(std::chrono::steady_clock::time_point start) {
        return std::chrono::duration<double, std::milli>(
                   std::chrono::steady_clock::now() - start
        )
            .count();
    }

} // namespace porch::rt
