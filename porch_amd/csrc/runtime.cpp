#include "runtime.hpp"

#include "disk_cache.hpp"

#include "porch/hip_jit.hpp"

#include <sys/syscall.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <optional>
#include <stdexcept>
#include <thread>
#include <unordered_map>

namespace porch::rt {
    namespace {

        struct device_state {
            device_info info;
        };

        device_state* init_device() {
            const hip::api& h = hip::runtime();
            hip::check(h.init(0), "hipInit");
            int count = 0;
            hip::check(h.get_device_count(&count), "hipGetDeviceCount");
            if (count < 1) {
                throw std::runtime_error(
                    "porch GPU execution requires a HIP device"
                );
            }
            auto* state = new device_state();
            device_info& info = state->info;
            info.ordinal = 0;
            hip::check(h.set_device(0), "hipSetDevice");
            hip::check(
                h.device_get_attribute(
                    &info.compute_units, hip::attr_multiprocessor_count, 0
                ),
                "hipDeviceGetAttribute"
            );
            hip::check(
                h.device_get_attribute(&info.clock_khz, hip::attr_clock_rate, 0),
                "hipDeviceGetAttribute"
            );
            (void)h.device_get_attribute(
                &info.l2_bytes, hip::attr_l2_cache_size, 0
            );
            std::vector<char> props(hip::device_prop_size + 1024, 0);
            if (h.get_device_properties(props.data(), 0) == hip::success) {
                const char* name = props.data() + hip::device_prop_arch_offset;
                info.arch.assign(name, strnlen(name, 256));
            }
            // Keep freed blocks in the pool: stream-ordered reuse without
            // returning memory to the driver at every synchronisation.
            hip::mem_pool_t pool = nullptr;
            if (h.device_get_default_mem_pool(&pool, 0) == hip::success &&
                pool != nullptr) {
                uint64_t threshold = std::numeric_limits<uint64_t>::max();
                (void)h.mem_pool_set_attribute(
                    pool, hip::mem_pool_attr_release_threshold, &threshold
                );
            }
            return state;
        }

        device_state& device_singleton() {
            static device_state* instance = init_device();
            return *instance;
        }

        struct rtc_program {
            hip::rtc_program_t program = nullptr;
            ~rtc_program() {
                if (program != nullptr)
                    (void)hip::compiler().rtc_destroy_program(&program);
            }
        };

        std::string program_log(hip::rtc_program_t program) {
            const hip::api& c = hip::compiler();
            size_t size = 0;
            hip::check_rtc(
                c.rtc_get_program_log_size(program, &size),
                "hiprtcGetProgramLogSize"
            );
            if (size == 0) return {};
            std::string log(size, '\0');
            hip::check_rtc(
                c.rtc_get_program_log(program, log.data()),
                "hiprtcGetProgramLog"
            );
            while (!log.empty() && log.back() == '\0') log.pop_back();
            return log;
        }

        struct code_cache {
            std::mutex mutex;
            std::unordered_map<std::string, std::shared_ptr<const code_object>>
                entries;
        };
        code_cache& codes() {
            static code_cache* cache = new code_cache();
            return *cache;
        }

        struct loaded_module {
            hip::module_t module = nullptr;
            std::unordered_map<std::string, kernel_handle> kernels;
        };
        struct module_cache {
            std::mutex mutex;
            // keyed by the code object's bytes
            std::unordered_map<std::string, loaded_module> entries;
        };
        module_cache& modules() {
            static module_cache* cache = new module_cache();
            return *cache;
        }

        std::string cache_key(
            std::string_view source, const std::vector<std::string>& options
        ) {
            std::string key;
            key.reserve(source.size() + 64);
            key += std::to_string(source.size());
            key += ':';
            key += source;
            for (const std::string& option : options) {
                key += '\0';
                key += std::to_string(option.size());
                key += ':';
                key += option;
            }
            return key;
        }

    } // namespace

    const device_info& device() { return device_singleton().info; }

    stream::stream() {
        const hip::api& h = hip::runtime();
        (void)device();
        hip::check(h.set_device(0), "hipSetDevice");
        hip::check(
            h.stream_create_with_flags(&handle_, hip::stream_non_blocking),
            "hipStreamCreateWithFlags"
        );
    }

    stream::~stream() {
        if (handle_ == nullptr) return;
        try {
            release_stream_blocks(*this);
            const hip::api& h = hip::runtime();
            (void)h.stream_synchronize(handle_);
            (void)h.stream_destroy(handle_);
        }
        catch (...) {
        }
    }

    void stream::synchronize() const {
        hip::check(
            hip::runtime().stream_synchronize(handle_), "hipStreamSynchronize"
        );
    }

    namespace {
        // The calling thread's stream.  A worker thread's stream is
        // released when the thread exits (buffers it produced keep it
        // alive).  The process's initial thread only exits inside exit(),
        // where thread-local destructors run before the HIP runtime and any
        // attached tool have shut down: that stream is left to the OS.
        struct thread_stream {
            std::shared_ptr<stream> s = std::make_shared<stream>();
            ~thread_stream() {
                if (static_cast<pid_t>(syscall(SYS_gettid)) == getpid())
                    new std::shared_ptr<stream>(std::move(s)); // never freed
            }
        };
    } // namespace

    std::shared_ptr<stream> current_stream() {
        thread_local thread_stream mine;
        return mine.s;
    }

    void order_after(const stream& consumer, const stream& producer) {
        if (&consumer == &producer) return;
        const hip::api& h = hip::runtime();
        hip::event_t event = nullptr;
        hip::check(
            h.event_create_with_flags(&event, hip::event_disable_timing),
            "hipEventCreateWithFlags"
        );
        hip::error_t recorded = h.event_record(event, producer.handle());
        hip::error_t waited =
            recorded == hip::success
                ? h.stream_wait_event(consumer.handle(), event, 0)
                : recorded;
        (void)h.event_destroy(event);
        hip::check(recorded, "hipEventRecord");
        hip::check(waited, "hipStreamWaitEvent");
    }

    namespace {
        struct staging_chunk {
            void* host = nullptr;
            size_t bytes = 0;
            hip::event_t done = nullptr;
            bool busy = false;    // being filled by a caller
            bool pending = false; // DMA queued, `done` not yet observed
        };
        struct staging_pool {
            std::mutex mutex;
            std::vector<std::unique_ptr<staging_chunk>> chunks;
            size_t total = 0;
        };
        staging_pool& staging() {
            static staging_pool* instance = new staging_pool();
            return *instance;
        }
        constexpr size_t staging_cap = size_t{512} << 20;
        constexpr size_t staging_largest = size_t{32} << 20;

        // memcpy into pinned memory, split over host threads for large
        // copies: one thread copies ~9 GiB/s here, below the host link.
        void staged_copy(void* dst, const void* src, size_t bytes) {
            constexpr size_t per_thread = size_t{4} << 20;
            const unsigned hw = std::max(1U, std::thread::hardware_concurrency());
            const size_t parts = std::min<size_t>({bytes / per_thread, hw, 16});
            if (parts < 2) {
                std::memcpy(dst, src, bytes);
                return;
            }
            const size_t piece = (bytes / parts + 63) / 64 * 64;
            std::vector<std::thread> workers;
            workers.reserve(parts - 1);
            for (size_t i = 1; i < parts; ++i) {
                const size_t begin = std::min(bytes, i * piece);
                const size_t end = std::min(bytes, begin + piece);
                if (begin >= end) break;
                workers.emplace_back([=] {
                    std::memcpy(static_cast<char*>(dst) + begin,
                                static_cast<const char*>(src) + begin, end - begin);
                });
            }
            std::memcpy(dst, src, std::min(bytes, piece));
            for (std::thread& w : workers) w.join();
        }

        bool chunk_idle(const hip::api& h, staging_chunk& c) {
            if (c.busy) return false;
            if (!c.pending) return true;
            const hip::error_t state = h.event_query(c.done);
            if (state == hip::error_not_ready) return false;
            hip::check(state, "hipEventQuery");
            c.pending = false;
            return true;
        }
    } // namespace

    namespace {
        // A chunk of at least `bytes`, marked busy; nullptr when the pool is
        // full of chunks other callers are filling or draining.
        staging_chunk* acquire_chunk(const hip::api& h, size_t bytes) {
            size_t size = size_t{1} << 20;
            while (size < bytes) size <<= 1;
            staging_pool& pool = staging();
            std::scoped_lock lock{pool.mutex};
            for (auto& c : pool.chunks) {
                if (c->bytes == size && chunk_idle(h, *c)) {
                    c->busy = true;
                    return c.get();
                }
            }
            // Make room: free idle chunks of other sizes, then wait for
            // pending ones, until the new chunk fits under the cap.
            for (const bool wait : {false, true}) {
                for (auto it = pool.chunks.begin();
                     it != pool.chunks.end() && pool.total + size > staging_cap;) {
                    staging_chunk& c = **it;
                    if (wait && c.pending && !c.busy)
                        hip::check(h.event_synchronize(c.done), "hipEventSynchronize");
                    if (chunk_idle(h, c)) {
                        (void)h.host_free(c.host);
                        (void)h.event_destroy(c.done);
                        pool.total -= c.bytes;
                        it = pool.chunks.erase(it);
                    }
                    else {
                        ++it;
                    }
                }
            }
            if (pool.total + size > staging_cap) return nullptr;
            auto fresh = std::make_unique<staging_chunk>();
            hip::check(h.host_malloc(&fresh->host, size, 0), "hipHostMalloc");
            const hip::error_t made = h.event_create_with_flags(&fresh->done, hip::event_disable_timing);
            if (made != hip::success) (void)h.host_free(fresh->host);
            hip::check(made, "hipEventCreateWithFlags");
            fresh->bytes = size;
            fresh->busy = true;
            pool.total += size;
            pool.chunks.push_back(std::move(fresh));
            return pool.chunks.back().get();
        }

        // Hands a chunk back; `pending`: its event was recorded behind work
        // that still reads or writes it.
        void release_chunk(staging_chunk* c, bool pending) {
            std::scoped_lock lock{staging().mutex};
            c->busy = false;
            c->pending = pending;
        }

        constexpr size_t staging_piece = size_t{32} << 20;
    } // namespace

    bool upload_staged(void* dst, const void* src, size_t bytes, const stream& s) {
        // Pieces of at most 32 MiB, each through its own chunk: the host
        // copy of one piece overlaps the DMA of the previous one.
        const hip::api& h = hip::runtime();
        for (size_t done = 0; done < bytes;) {
            const size_t n = std::min(staging_piece, bytes - done);
            char* to = static_cast<char*>(dst) + done;
            const char* from = static_cast<const char*>(src) + done;
            staging_chunk* chunk = acquire_chunk(h, n);
            if (chunk == nullptr) {
                if (done == 0) return false;
                // Chunks all taken by other threads: copy the rest directly.
                hip::check(h.memcpy_htod_async(to, from, bytes - done, s.handle()), "hipMemcpyHtoDAsync");
                s.synchronize();
                return true;
            }
            staged_copy(chunk->host, from, n);
            hip::error_t queued = h.memcpy_htod_async(to, chunk->host, n, s.handle());
            if (queued == hip::success) queued = h.event_record(chunk->done, s.handle());
            if (queued != hip::success) {
                // The copy may be in flight: wait before the chunk is reused.
                (void)h.stream_synchronize(s.handle());
                release_chunk(chunk, false);
                hip::check(queued, "hipMemcpyHtoDAsync");
            }
            release_chunk(chunk, true);
            done += n;
        }
        return true;
    }

    bool download_staged(void* dst, const void* src, size_t bytes, const stream& s) {
        // Rounds of up to four 32 MiB pieces: all of a round's DMAs are
        // queued into pinned chunks, then each piece is copied out as soon
        // as its DMA is done, while the later ones still run.
        const hip::api& h = hip::runtime();
        constexpr size_t round = 4;
        void* device = const_cast<void*>(src);
        size_t done = 0;
        while (done < bytes) {
            staging_chunk* chunks[round] = {};
            size_t sizes[round] = {};
            size_t count = 0;
            hip::error_t queued = hip::success;
            for (size_t at = done; count < round && at < bytes && queued == hip::success;) {
                const size_t n = std::min(staging_piece, bytes - at);
                staging_chunk* chunk = acquire_chunk(h, n);
                if (chunk == nullptr) break;
                chunks[count] = chunk;
                sizes[count] = n;
                ++count;
                queued = h.memcpy_dtoh_async(chunk->host, static_cast<char*>(device) + at, n, s.handle());
                if (queued == hip::success) queued = h.event_record(chunk->done, s.handle());
                at += n;
            }
            if (queued != hip::success) (void)h.stream_synchronize(s.handle());
            hip::error_t waited = hip::success;
            for (size_t i = 0; i < count; ++i) {
                if (queued == hip::success && waited == hip::success) {
                    waited = h.event_synchronize(chunks[i]->done);
                    if (waited == hip::success)
                        staged_copy(static_cast<char*>(dst) + done, chunks[i]->host, sizes[i]);
                }
                done += sizes[i];
                // After a failed wait this piece's DMA, and the later ones',
                // may still be queued: the chunk stays pending, so it is
                // reused only once its event reports the DMA done.
                release_chunk(chunks[i], waited != hip::success);
            }
            hip::check(queued, "hipMemcpyDtoHAsync");
            hip::check(waited, "hipEventSynchronize");
            if (count == 0) {
                if (done == 0) return false;
                // Chunks all taken by other threads: copy the rest directly.
                hip::check(h.memcpy_dtoh_async(static_cast<char*>(dst) + done,
                                               static_cast<char*>(device) + done, bytes - done,
                                               s.handle()),
                           "hipMemcpyDtoHAsync");
                s.synchronize();
                return true;
            }
        }
        return true;
    }

    size_t staging_bytes() {
        std::scoped_lock lock{staging().mutex};
        return staging().total;
    }

    namespace {
        struct block_cache {
            std::mutex mutex;
            std::unordered_map<const stream*, std::multimap<size_t, void*>> free;
            size_t cached = 0;
        };
        block_cache& blocks() {
            static block_cache* instance = new block_cache();
            return *instance;
        }
        // Cached bytes kept across all streams (of 288 GB of HBM3E).
        constexpr size_t block_cache_limit = size_t{32} << 30;
        constexpr hip::error_t error_out_of_memory = 2;

        size_t block_size(size_t bytes) {
            constexpr size_t small = size_t{1} << 20;
            if (bytes <= small) return (bytes + 511) & ~size_t{511};
            return (bytes + small - 1) & ~(small - 1);
        }

        // Frees every cached block (all streams); caller holds the mutex.
        void drain(block_cache& c) {
            const hip::api& h = hip::runtime();
            for (auto& [owner, list] : c.free) {
                for (auto& [size, ptr] : list) {
                    (void)h.free_async(ptr, owner->handle());
                    c.cached -= size;
                }
                list.clear();
            }
        }
    } // namespace

    void* allocate_block(size_t bytes, const stream& s, size_t* capacity) {
        const size_t want = block_size(bytes);
        block_cache& c = blocks();
        {
            std::scoped_lock lock{c.mutex};
            auto list = c.free.find(&s);
            if (list != c.free.end()) {
                auto fit = list->second.lower_bound(want);
                if (fit != list->second.end() && fit->first <= want + want / 4) {
                    void* ptr = fit->second;
                    *capacity = fit->first;
                    c.cached -= fit->first;
                    list->second.erase(fit);
                    return ptr;
                }
            }
        }
        const hip::api& h = hip::runtime();
        void* ptr = nullptr;
        hip::error_t rc = h.malloc_async(&ptr, want, s.handle());
        if (rc == error_out_of_memory) {
            {
                std::scoped_lock lock{c.mutex};
                drain(c);
            }
            rc = h.malloc_async(&ptr, want, s.handle());
        }
        hip::check(rc, "hipMallocAsync");
        *capacity = want;
        return ptr;
    }

    void release_block(void* ptr, size_t capacity, const stream& s) {
        block_cache& c = blocks();
        std::scoped_lock lock{c.mutex};
        c.free[&s].emplace(capacity, ptr);
        c.cached += capacity;
        if (c.cached <= block_cache_limit) return;
        const hip::api& h = hip::runtime();
        // Over the limit: return the largest cached blocks to the pool.
        while (c.cached > block_cache_limit / 2) {
            const stream* owner = nullptr;
            std::multimap<size_t, void*>::iterator largest;
            for (auto& [st, list] : c.free) {
                if (list.empty()) continue;
                auto last = std::prev(list.end());
                if (owner == nullptr || last->first > largest->first) {
                    owner = st;
                    largest = last;
                }
            }
            if (owner == nullptr) break;
            (void)h.free_async(largest->second, owner->handle());
            c.cached -= largest->first;
            c.free[owner].erase(largest);
        }
    }

    void release_stream_blocks(const stream& s) {
        block_cache& c = blocks();
        std::scoped_lock lock{c.mutex};
        auto list = c.free.find(&s);
        if (list == c.free.end()) return;
        const hip::api& h = hip::runtime();
        for (auto& [size, ptr] : list->second) {
            (void)h.free_async(ptr, s.handle());
            c.cached -= size;
        }
        c.free.erase(list);
    }

    size_t release_cached_blocks() {
        block_cache& c = blocks();
        std::scoped_lock lock{c.mutex};
        const size_t before = c.cached;
        drain(c);
        return before - c.cached;
    }

    size_t cached_block_bytes() {
        std::scoped_lock lock{blocks().mutex};
        return blocks().cached;
    }

    buffer_state::buffer_state(size_t requested_bytes)
        : bytes(requested_bytes) {
        if (bytes == 0) return;
        std::shared_ptr<stream> s = current_stream();
        ptr = allocate_block(bytes, *s, &capacity);
        producer_ = std::move(s);
    }

    buffer_state::~buffer_state() {
        if (ptr == nullptr) return;
        try {
            std::shared_ptr<stream> owner =
                producer_ != nullptr ? producer_ : current_stream();
            for (const std::shared_ptr<stream>& reader : readers_) {
                if (reader != owner) order_after(*owner, *reader);
            }
            release_block(ptr, capacity, *owner);
        }
        catch (...) {
        }
    }

    void buffer_state::before_read(const std::shared_ptr<stream>& s) {
        std::scoped_lock lock{mutex_};
        if (producer_ == nullptr || producer_ == s) return;
        order_after(*s, *producer_);
        for (const std::shared_ptr<stream>& reader : readers_) {
            if (reader == s) return;
        }
        readers_.push_back(s);
    }

    void buffer_state::before_write(const std::shared_ptr<stream>& s) {
        std::scoped_lock lock{mutex_};
        if (producer_ != nullptr && producer_ != s) order_after(*s, *producer_);
        for (const std::shared_ptr<stream>& reader : readers_) {
            if (reader != s) order_after(*s, *reader);
        }
        readers_.clear();
    }

    void buffer_state::after_write(const std::shared_ptr<stream>& s) {
        std::scoped_lock lock{mutex_};
        producer_ = s;
    }

    std::shared_ptr<stream> buffer_state::producer_stream() const {
        std::scoped_lock lock{mutex_};
        return producer_;
    }

    std::string target_arch() {
        if (const char* arch = std::getenv("PORCH_HIP_ARCH")) return arch;
        return "gfx950";
    }

    std::vector<std::string> default_options() {
        return {
            "--offload-arch=" + target_arch(),
            "-O3",
            "-std=c++17",
            "-ffp-contract=off",
            // Packed FP32 (v_pk_*_f32) stays off in every kernel.
            "-Xclang",
            "-target-feature",
            "-Xclang",
            "-packed-fp32-ops",
        };
    }

    std::shared_ptr<const code_object> compile(
        std::string_view source, const std::vector<std::string>& extra_options
    ) {
        std::vector<std::string> options = default_options();
        options.insert(
            options.end(), extra_options.begin(), extra_options.end()
        );
        const std::string key = cache_key(source, options);
        {
            std::scoped_lock lock{codes().mutex};
            auto found = codes().entries.find(key);
            if (found != codes().entries.end()) return found->second;
        }

        const hip::api& c = hip::compiler();
        // The on-disk entry is valid only for the compiler that wrote it.
        static const std::string compiler_tag = [&] {
            int major = 0;
            int minor = 0;
            if (c.rtc_version != nullptr) (void)c.rtc_version(&major, &minor);
            using namespace std::string_literals;
            return "\0hiprtc "s + std::to_string(major) + "." + std::to_string(minor) +
                   "\0porch code object 1"s;
        }();
        const std::string disk_key = key + compiler_tag;
        {
            const auto read_start = std::chrono::steady_clock::now();
            if (std::optional<std::string> stored = disk::load(disk_key)) {
                auto object = std::make_shared<code_object>();
                object->bytes = std::move(*stored);
                {
                    std::scoped_lock lock{counters_mutex()};
                    counters().disk_hits += 1;
                    counters().disk_ms += elapsed_ms(read_start);
                }
                std::scoped_lock lock{codes().mutex};
                if (codes().entries.size() >= 4096) codes().entries.clear();
                auto [it, inserted] = codes().entries.emplace(key, object);
                return it->second;
            }
        }

        const auto start = std::chrono::steady_clock::now();
        rtc_program program;
        const std::string text{source};
        hip::check_rtc(
            c.rtc_create_program(
                &program.program, text.c_str(), "porch_kernel.hip", 0, nullptr,
                nullptr
            ),
            "hiprtcCreateProgram"
        );
        std::vector<const char*> option_ptrs;
        option_ptrs.reserve(options.size());
        for (const std::string& option : options)
            option_ptrs.push_back(option.c_str());
        const hip::rtc_result_t result = c.rtc_compile_program(
            program.program, static_cast<int>(option_ptrs.size()),
            option_ptrs.data()
        );
        if (result != hip::rtc_success) {
            std::string log = program_log(program.program);
            if (log.empty()) {
                const char* text_error = c.rtc_get_error_string(result);
                log = text_error != nullptr ? text_error : "hiprtc failed";
            }
            throw hip_jit::compilation_error(std::move(log));
        }
        size_t size = 0;
        hip::check_rtc(
            c.rtc_get_code_size(program.program, &size), "hiprtcGetCodeSize"
        );
        auto object = std::make_shared<code_object>();
        object->bytes.assign(size, '\0');
        hip::check_rtc(
            c.rtc_get_code(program.program, object->bytes.data()),
            "hiprtcGetCode"
        );
        object->compile_ms = elapsed_ms(start);
        {
            std::scoped_lock lock{counters_mutex()};
            counters().compiles += 1;
            counters().compile_ms += object->compile_ms;
        }
        disk::store(disk_key, object->bytes);
        std::scoped_lock lock{codes().mutex};
        // Bounded; modules of dropped code objects stay loaded (plans may
        // still launch their kernels), and a recompiled identical object
        // reuses its module.
        if (codes().entries.size() >= 4096) codes().entries.clear();
        auto [it, inserted] = codes().entries.emplace(key, object);
        return it->second;
    }

    kernel_handle load_kernel(
        const std::shared_ptr<const code_object>& code, std::string_view name
    ) {
        const hip::api& h = hip::runtime();
        (void)device();
        std::scoped_lock lock{modules().mutex};
        loaded_module& entry = modules().entries[code->bytes];
        if (entry.module == nullptr) {
            const auto start = std::chrono::steady_clock::now();
            hip::check(
                h.module_load_data(&entry.module, code->bytes.data()),
                "hipModuleLoadData"
            );
            std::scoped_lock counters_lock{counters_mutex()};
            counters().module_load_ms += elapsed_ms(start);
        }
        const std::string function_name{name};
        auto found = entry.kernels.find(function_name);
        if (found != entry.kernels.end()) return found->second;
        kernel_handle kernel;
        hip::check(
            h.module_get_function(
                &kernel.function, entry.module, function_name.c_str()
            ),
            "hipModuleGetFunction"
        );
        (void)h.func_get_attribute(
            &kernel.registers, hip::func_attr_num_regs, kernel.function
        );
        (void)h.func_get_attribute(
            &kernel.lds_bytes, hip::func_attr_shared_size_bytes, kernel.function
        );
        (void)h.func_get_attribute(
            &kernel.scratch_bytes, hip::func_attr_local_size_bytes,
            kernel.function
        );
        entry.kernels.emplace(function_name, kernel);
        return kernel;
    }

    void launch(
        const kernel_handle& kernel, unsigned grid_x, unsigned grid_y,
        unsigned grid_z, unsigned block_x, unsigned shared_bytes,
        void** params, const stream& s, hip::event_t start, hip::event_t stop
    ) {
        const hip::api& h = hip::runtime();
        if (start == nullptr && stop == nullptr) {
            hip::check(
                h.module_launch_kernel(
                    kernel.function, grid_x, grid_y, grid_z, block_x, 1, 1,
                    shared_bytes, s.handle(), params, nullptr
                ),
                "hipModuleLaunchKernel"
            );
        }
        else {
            const uint64_t threads = static_cast<uint64_t>(grid_x) * block_x;
            if (threads > 0xffffffffULL || grid_y != 1 || grid_z != 1)
                throw std::invalid_argument("timed launch grid is too large");
            hip::check(
                h.ext_module_launch_kernel(
                    kernel.function, static_cast<uint32_t>(threads), 1, 1,
                    block_x, 1, 1, shared_bytes, s.handle(), params, nullptr,
                    start, stop, 0
                ),
                "hipExtModuleLaunchKernel"
            );
        }
        std::scoped_lock lock{counters_mutex()};
        counters().launches += 1;
    }

    void clear_caches() {
        {
            std::scoped_lock lock{codes().mutex};
            codes().entries.clear();
        }
        // Modules stay loaded: kernels of cached plans may still be queued.
        // A cleared code cache forces recompilation; a recompiled code
        // object that is byte-identical reuses its module.
    }

    jit_counters& counters() {
        static jit_counters* instance = new jit_counters();
        return *instance;
    }

    std::mutex& counters_mutex() {
        static std::mutex* instance = new std::mutex();
        return *instance;
    }

    void flush_caches(size_t bytes) {
        static std::mutex mutex;
        static void* scratch = nullptr;
        static size_t scratch_bytes = 0;
        std::scoped_lock lock{mutex};
        std::shared_ptr<stream> s = current_stream();
        const hip::api& h = hip::runtime();
        bytes = (bytes + 3) & ~size_t{3};
        if (scratch_bytes < bytes) {
            if (scratch != nullptr) {
                hip::check(h.free_async(scratch, s->handle()), "hipFreeAsync");
            }
            scratch = nullptr;
            hip::check(
                h.malloc_async(&scratch, bytes, s->handle()), "hipMallocAsync"
            );
            scratch_bytes = bytes;
        }
        static int pattern = 0;
        pattern += 1;
        hip::check(
            h.memset_d32_async(scratch, pattern, bytes / 4, s->handle()),
            "hipMemsetD32Async"
        );
    }

} // namespace porch::rt
