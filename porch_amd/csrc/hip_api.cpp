#include "hip_api.hpp"

#include <dlfcn.h>

#include <atomic>
#include <cstdlib>
#include <mutex>
#include <stdexcept>

namespace porch::hip {
    namespace {

        void* open_first(std::initializer_list<const char*> names) {
            for (const char* name : names) {
                if (void* handle = dlopen(name, RTLD_NOW | RTLD_LOCAL))
                    return handle;
            }
            return nullptr;
        }

        template <typename F>
        bool bind(void* library, F& slot, const char* name) {
            slot = reinterpret_cast<F>(dlsym(library, name));
            return slot != nullptr;
        }

        // Counting wrappers around the entry points that allocate: each
        // adds one to its counter and calls the library's function.
        struct counted_entry_points {
            decltype(api::malloc_async) malloc_async = nullptr;
            decltype(api::free_async) free_async = nullptr;
            decltype(api::host_malloc) host_malloc = nullptr;
            decltype(api::host_free) host_free = nullptr;
            decltype(api::module_load_data) module_load_data = nullptr;
            std::atomic<uint64_t> device_allocs{0}, device_frees{0}, host_allocs{0}, host_frees{0},
                module_loads{0};
        };
        counted_entry_points& counted() {
            static counted_entry_points* c = new counted_entry_points();
            return *c;
        }
        error_t counting_malloc_async(void** ptr, size_t bytes, stream_t s) {
            counted().device_allocs.fetch_add(1, std::memory_order_relaxed);
            return counted().malloc_async(ptr, bytes, s);
        }
        error_t counting_free_async(void* ptr, stream_t s) {
            counted().device_frees.fetch_add(1, std::memory_order_relaxed);
            return counted().free_async(ptr, s);
        }
        error_t counting_host_malloc(void** ptr, size_t bytes, unsigned flags) {
            counted().host_allocs.fetch_add(1, std::memory_order_relaxed);
            return counted().host_malloc(ptr, bytes, flags);
        }
        error_t counting_host_free(void* ptr) {
            counted().host_frees.fetch_add(1, std::memory_order_relaxed);
            return counted().host_free(ptr);
        }
        error_t counting_module_load_data(module_t* module, const void* image) {
            counted().module_loads.fetch_add(1, std::memory_order_relaxed);
            return counted().module_load_data(module, image);
        }

        void count_allocations(api& t) {
            counted_entry_points& c = counted();
            c.malloc_async = t.malloc_async;
            c.free_async = t.free_async;
            c.host_malloc = t.host_malloc;
            c.host_free = t.host_free;
            c.module_load_data = t.module_load_data;
            t.malloc_async = counting_malloc_async;
            t.free_async = counting_free_async;
            t.host_malloc = counting_host_malloc;
            t.host_free = counting_host_free;
            t.module_load_data = counting_module_load_data;
        }

        struct loaded {
            api table{};
            bool runtime_ok = false;
            bool compiler_ok = false;
            std::string runtime_error;
            std::string compiler_error;
        };

        loaded load() {
            loaded result;
            // PORCH_HIP_LIBRARY / PORCH_HIPRTC_LIBRARY override the search
            // (tests point them at a missing file to exercise the
            // unavailable path).
            const char* hip_override = std::getenv("PORCH_HIP_LIBRARY");
            const char* rtc_override = std::getenv("PORCH_HIPRTC_LIBRARY");

            void* hip_library =
                hip_override != nullptr
                    ? open_first({hip_override})
                    : open_first(
                          {"libamdhip64.so.7", "libamdhip64.so",
                           "/opt/rocm/lib/libamdhip64.so.7"}
                      );
            api& t = result.table;
            if (hip_library == nullptr) {
                result.runtime_error =
                    "porch GPU execution requires libamdhip64 at runtime";
            }
            else {
                bool ok = true;
                ok &= bind(hip_library, t.init, "hipInit");
                ok &= bind(hip_library, t.get_device_count, "hipGetDeviceCount");
                ok &= bind(hip_library, t.set_device, "hipSetDevice");
                ok &= bind(
                    hip_library, t.device_get_attribute, "hipDeviceGetAttribute"
                );
                ok &= bind(
                    hip_library, t.get_device_properties,
                    "hipGetDevicePropertiesR0600"
                );
                ok &= bind(
                    hip_library, t.stream_create_with_flags,
                    "hipStreamCreateWithFlags"
                );
                ok &= bind(hip_library, t.stream_destroy, "hipStreamDestroy");
                ok &= bind(
                    hip_library, t.stream_synchronize, "hipStreamSynchronize"
                );
                ok &= bind(hip_library, t.stream_wait_event, "hipStreamWaitEvent");
                ok &= bind(
                    hip_library, t.event_create_with_flags,
                    "hipEventCreateWithFlags"
                );
                ok &= bind(hip_library, t.event_record, "hipEventRecord");
                ok &= bind(hip_library, t.event_synchronize, "hipEventSynchronize");
                ok &= bind(
                    hip_library, t.event_elapsed_time, "hipEventElapsedTime"
                );
                ok &= bind(hip_library, t.event_destroy, "hipEventDestroy");
                ok &= bind(hip_library, t.event_query, "hipEventQuery");
                ok &= bind(hip_library, t.host_malloc, "hipHostMalloc");
                ok &= bind(hip_library, t.host_free, "hipHostFree");
                ok &= bind(hip_library, t.malloc_async, "hipMallocAsync");
                ok &= bind(hip_library, t.free_async, "hipFreeAsync");
                ok &= bind(
                    hip_library, t.device_get_default_mem_pool,
                    "hipDeviceGetDefaultMemPool"
                );
                ok &= bind(
                    hip_library, t.mem_pool_set_attribute,
                    "hipMemPoolSetAttribute"
                );
                ok &= bind(hip_library, t.memcpy_htod_async, "hipMemcpyHtoDAsync");
                ok &= bind(hip_library, t.memcpy_dtoh_async, "hipMemcpyDtoHAsync");
                ok &= bind(hip_library, t.memset_d32_async, "hipMemsetD32Async");
                ok &= bind(hip_library, t.module_load_data, "hipModuleLoadData");
                ok &= bind(hip_library, t.module_unload, "hipModuleUnload");
                ok &= bind(
                    hip_library, t.module_get_function, "hipModuleGetFunction"
                );
                ok &= bind(
                    hip_library, t.module_launch_kernel, "hipModuleLaunchKernel"
                );
                ok &= bind(
                    hip_library, t.ext_module_launch_kernel,
                    "hipExtModuleLaunchKernel"
                );
                ok &= bind(
                    hip_library, t.func_get_attribute, "hipFuncGetAttribute"
                );
                ok &= bind(hip_library, t.get_error_name, "hipGetErrorName");
                ok &= bind(hip_library, t.get_error_string, "hipGetErrorString");
                result.runtime_ok = ok;
                if (ok) count_allocations(t);
                if (!ok) {
                    result.runtime_error =
                        "libamdhip64 lacks an entry point porch requires";
                }
            }

            void* rtc_library =
                rtc_override != nullptr
                    ? open_first({rtc_override})
                    : open_first(
                          {"libhiprtc.so.7", "libhiprtc.so",
                           "/opt/rocm/lib/libhiprtc.so.7"}
                      );
            if (rtc_library == nullptr) {
                result.compiler_error =
                    "porch JIT compilation requires libhiprtc at runtime";
            }
            else {
                bool ok = true;
                ok &= bind(
                    rtc_library, t.rtc_create_program, "hiprtcCreateProgram"
                );
                ok &= bind(
                    rtc_library, t.rtc_compile_program, "hiprtcCompileProgram"
                );
                ok &= bind(rtc_library, t.rtc_get_code_size, "hiprtcGetCodeSize");
                ok &= bind(rtc_library, t.rtc_get_code, "hiprtcGetCode");
                ok &= bind(
                    rtc_library, t.rtc_get_program_log_size,
                    "hiprtcGetProgramLogSize"
                );
                ok &= bind(
                    rtc_library, t.rtc_get_program_log, "hiprtcGetProgramLog"
                );
                ok &= bind(
                    rtc_library, t.rtc_destroy_program, "hiprtcDestroyProgram"
                );
                ok &= bind(
                    rtc_library, t.rtc_get_error_string, "hiprtcGetErrorString"
                );
                ok &= bind(rtc_library, t.rtc_version, "hiprtcVersion");
                result.compiler_ok = ok;
                if (!ok) {
                    result.compiler_error =
                        "libhiprtc lacks an entry point porch requires";
                }
            }
            // The libraries stay loaded for the life of the process.
            return result;
        }

        const loaded& libraries() {
            static const loaded* instance = new loaded(load());
            return *instance;
        }

    } // namespace

    const api& runtime() {
        const loaded& l = libraries();
        if (!l.runtime_ok) throw std::runtime_error(l.runtime_error);
        return l.table;
    }

    const api& compiler() {
        const loaded& l = libraries();
        if (!l.compiler_ok) throw std::runtime_error(l.compiler_error);
        return l.table;
    }

    bool libraries_present() noexcept {
        try {
            const loaded& l = libraries();
            return l.runtime_ok && l.compiler_ok;
        }
        catch (...) {
            return false;
        }
    }

    allocation_calls allocation_counts() noexcept {
        const counted_entry_points& c = counted();
        allocation_calls a;
        a.device_allocs = c.device_allocs.load(std::memory_order_relaxed);
        a.device_frees = c.device_frees.load(std::memory_order_relaxed);
        a.host_allocs = c.host_allocs.load(std::memory_order_relaxed);
        a.host_frees = c.host_frees.load(std::memory_order_relaxed);
        a.module_loads = c.module_loads.load(std::memory_order_relaxed);
        return a;
    }

    void check(error_t result, std::string_view operation) {
        if (result == success) return;
        std::string message{operation};
        message += " failed: ";
        const api& t = libraries().table;
        const char* name =
            t.get_error_name != nullptr ? t.get_error_name(result) : nullptr;
        const char* text =
            t.get_error_string != nullptr ? t.get_error_string(result) : nullptr;
        message += name != nullptr ? name
                                   : ("hipError " + std::to_string(result));
        if (text != nullptr) {
            message += ": ";
            message += text;
        }
        throw std::runtime_error(message);
    }

    void check_rtc(rtc_result_t result, std::string_view operation) {
        if (result == rtc_success) return;
        std::string message{operation};
        message += " failed: ";
        const api& t = libraries().table;
        const char* text = t.rtc_get_error_string != nullptr
                               ? t.rtc_get_error_string(result)
                               : nullptr;
        message +=
            text != nullptr ? text : ("hiprtc error " + std::to_string(result));
        throw std::runtime_error(message);
    }

} // namespace porch::hip
