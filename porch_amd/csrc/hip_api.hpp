#pragma once

#include <cstdint>

// Thin loader over the C ABI of libamdhip64 and libhiprtc (ROCm 7).  The
// library resolves every entry point with dlsym at first use, so porch links
// against neither and loads on machines without ROCm; such machines report
// is_available() == false.  Replaces the reference's libcuda/NVRTC loader
// (reference src/cuda_jit.cpp:30-295).
//
// Types are opaque handles and plain integers with the values of
// hip/hip_runtime_api.h and hip/hiprtc.h (ROCm 7.2).

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <string_view>

namespace porch::hip {

    using error_t = int;
    using stream_t = void*;
    using event_t = void*;
    using module_t = void*;
    using function_t = void*;
    using mem_pool_t = void*;
    using rtc_result_t = int;
    using rtc_program_t = void*;

    inline constexpr error_t success = 0;
    inline constexpr error_t error_not_ready = 600;
    inline constexpr rtc_result_t rtc_success = 0;
    inline constexpr rtc_result_t rtc_error_compilation = 6;

    inline constexpr unsigned stream_non_blocking = 1;
    inline constexpr unsigned event_default = 0;
    inline constexpr unsigned event_disable_timing = 2;

    // hipDeviceAttribute_t values
    inline constexpr int attr_clock_rate = 5;
    inline constexpr int attr_l2_cache_size = 19;
    inline constexpr int attr_memory_clock_rate = 60;
    inline constexpr int attr_multiprocessor_count = 63;
    // hipMemPoolAttr value
    inline constexpr int mem_pool_attr_release_threshold = 4;
    // hipFunction_attribute values
    inline constexpr int func_attr_shared_size_bytes = 1;
    inline constexpr int func_attr_local_size_bytes = 3;
    inline constexpr int func_attr_num_regs = 4;

    // hipDeviceProp_t (R0600) size and the offset of gcnArchName[256].
    inline constexpr size_t device_prop_size = 1472;
    inline constexpr size_t device_prop_arch_offset = 1160;

    struct api {
        error_t (*init)(unsigned);
        error_t (*get_device_count)(int*);
        error_t (*set_device)(int);
        error_t (*device_get_attribute)(int*, int, int);
        error_t (*get_device_properties)(void*, int);
        error_t (*stream_create_with_flags)(stream_t*, unsigned);
        error_t (*stream_destroy)(stream_t);
        error_t (*stream_synchronize)(stream_t);
        error_t (*stream_wait_event)(stream_t, event_t, unsigned);
        error_t (*event_create_with_flags)(event_t*, unsigned);
        error_t (*event_record)(event_t, stream_t);
        error_t (*event_synchronize)(event_t);
        error_t (*event_elapsed_time)(float*, event_t, event_t);
        error_t (*event_destroy)(event_t);
        error_t (*event_query)(event_t);
        error_t (*host_malloc)(void**, size_t, unsigned);
        error_t (*host_free)(void*);
        error_t (*malloc_async)(void**, size_t, stream_t);
        error_t (*free_async)(void*, stream_t);
        error_t (*device_get_default_mem_pool)(mem_pool_t*, int);
        error_t (*mem_pool_set_attribute)(mem_pool_t, int, void*);
        error_t (*memcpy_htod_async)(void*, const void*, size_t, stream_t);
        error_t (*memcpy_dtoh_async)(void*, void*, size_t, stream_t);
        error_t (*memset_d32_async)(void*, int, size_t, stream_t);
        error_t (*module_load_data)(module_t*, const void*);
        error_t (*module_unload)(module_t);
        error_t (*module_get_function)(function_t*, module_t, const char*);
        error_t (*module_launch_kernel)(
            function_t, unsigned, unsigned, unsigned, unsigned, unsigned,
            unsigned, unsigned, stream_t, void**, void**
        );
        error_t (*ext_module_launch_kernel)(
            function_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
            size_t, stream_t, void**, void**, event_t, event_t, uint32_t
        );
        error_t (*func_get_attribute)(int*, int, function_t);
        const char* (*get_error_name)(error_t);
        const char* (*get_error_string)(error_t);

        rtc_result_t (*rtc_create_program)(
            rtc_program_t*, const char*, const char*, int, const char**,
            const char**
        );
        rtc_result_t (*rtc_compile_program)(rtc_program_t, int, const char**);
        rtc_result_t (*rtc_get_code_size)(rtc_program_t, size_t*);
        rtc_result_t (*rtc_get_code)(rtc_program_t, char*);
        rtc_result_t (*rtc_get_program_log_size)(rtc_program_t, size_t*);
        rtc_result_t (*rtc_get_program_log)(rtc_program_t, char*);
        rtc_result_t (*rtc_destroy_program)(rtc_program_t*);
        const char* (*rtc_get_error_string)(rtc_result_t);
        rtc_result_t (*rtc_version)(int*, int*);
    };

    // The HIP runtime entry points; throws std::runtime_error when
    // libamdhip64 is missing or lacks a symbol.
    const api& runtime();
    // The hiprtc entry points (a separate library that needs no device).
    const api& compiler();

    // True when both libraries load with every symbol resolved.
    bool libraries_present() noexcept;

    // Calls made through runtime() that allocate or release memory, counted
    // from the start of the process.
    struct allocation_calls {
        uint64_t device_allocs = 0; // hipMallocAsync
        uint64_t device_frees = 0;  // hipFreeAsync
        uint64_t host_allocs = 0;   // hipHostMalloc
        uint64_t host_frees = 0;    // hipHostFree
        uint64_t module_loads = 0;  // hipModuleLoadData (code memory)
    };
    allocation_calls allocation_counts() noexcept;

    // Throws std::runtime_error("<operation> failed: <name>: <description>")
    // for a failing HIP call (reference src/cuda_jit.cpp:315-339 format).
    void check(error_t result, std::string_view operation);
    void check_rtc(rtc_result_t result, std::string_view operation);

} // namespace porch::hip
