// porch_materialize_noalloc: porch_materialize into a caller-provided
// output, allocating no device memory.  For callers that cannot call
// hipMalloc (code under HIP graph capture, serving loops that forbid it).
//
// The kernels are the ones porch_materialize launches.  Their temporaries
// (memoised reductions, the partials of a split column reduction, product
// operands materialised once) come from `scratch`, a fixed device array of
// PORCH_NOALLOC_SCRATCH_BYTES that each GPU holds from the first call on it
// until the process ends.  The array's device address is looked up once
// per device, with that device current, and only that address is passed to
// kernels: in host code the array's name stands for a host-side shadow,
// not device memory.
//
// Every call on a GPU shares that GPU's array, so calls that overlap on
// one GPU (from threads with different streams) race; calls on one stream
// are ordered.  Nothing in the array needs to start at zero: each
// temporary is written in full by its producing kernel before any kernel
// reads it, so the contents a previous call left are never read.
//
// This file is compiled by hipcc (the array and its registration need the
// HIP runtime's own fat-binary support); the rest of the library reaches
// libamdhip64 through its loader.

#include <hip/hip_runtime.h>

#include "capi_internal.hpp"

#include <map>
#include <mutex>
#include <stdexcept>
#include <string>

static_assert(PORCH_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch is 256-byte granular");

static __device__ __align__(256) unsigned char scratch[PORCH_NOALLOC_SCRATCH_BYTES];

namespace {

    // The device address of `scratch` on the calling thread's current
    // device, looked up on the first call there with that device current.
    char* scratch_on_current_device() {
        int device = -1;
        hipError_t rc = hipGetDevice(&device);
        if (rc != hipSuccess)
            throw std::runtime_error(std::string("hipGetDevice: ") + hipGetErrorString(rc));
        static std::mutex mutex;
        static std::map<int, char*> addresses;
        std::scoped_lock lock{mutex};
        auto found = addresses.find(device);
        if (found != addresses.end()) return found->second;
        void* ptr = nullptr;
        rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (rc != hipSuccess || ptr == nullptr)
            throw std::runtime_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(rc));
        addresses.emplace(device, static_cast<char*>(ptr));
        return static_cast<char*>(ptr);
    }

} // namespace

extern "C" porch_status porch_materialize_noalloc(const porch_graph* graph,
                                                  const porch_buffer* const* inputs,
                                                  int32_t n_inputs, porch_buffer* out,
                                                  int64_t* out_shape, int32_t capacity,
                                                  int32_t* out_rank) {
    return porch::capi::guarded_call([&] {
        if (out == nullptr) throw std::invalid_argument("output buffer is null");
        const porch::capi::prepared_graph entry = porch::capi::prepare(graph);
        if (n_inputs < entry.n_inputs) throw std::invalid_argument("graph needs more input buffers");
        if (n_inputs > 0 && inputs == nullptr) throw std::invalid_argument("inputs are null");
        porch::capi::write_result_shape(entry.out_shape, out_shape, capacity, out_rank);
        if (entry.plan == nullptr) return; // empty result: nothing to write
        size_t need = 0;
        (void)porch::plan::workspace_layout(*entry.plan, &need);
        if (need > PORCH_NOALLOC_SCRATCH_BYTES)
            throw std::invalid_argument(
                "porch_materialize_noalloc: the graph's temporaries need " + std::to_string(need) +
                " bytes; at most " + std::to_string(PORCH_NOALLOC_SCRATCH_BYTES) +
                " (PORCH_NOALLOC_SCRATCH_BYTES) are available");
        porch::rt::buffer_state* target = porch::hip_jit::buffer_access::state(out->handle).get();
        if (target == nullptr) throw std::invalid_argument("output device buffer is too small");
        // The runtime first: the thread's stream exists and its device is
        // current before the array's address is looked up.
        (void)porch::rt::current_stream();
        char* workspace = scratch_on_current_device();
        porch::plan::run_in_workspace(*entry.plan, porch::capi::input_states(inputs, n_inputs), *target,
                                      workspace, PORCH_NOALLOC_SCRATCH_BYTES);
    });
}
