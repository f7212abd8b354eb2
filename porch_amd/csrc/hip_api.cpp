#include "hip_api.hpp"

#include <dlfcn.h>

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
