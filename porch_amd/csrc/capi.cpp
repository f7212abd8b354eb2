// The extern "C" boundary declared in include/porch_amd.h.

#include "porch_amd.h"
#include "capi_internal.hpp"
#include "disk_cache.hpp"

#include "internal.hpp"
#include "planner.hpp"

#include <chrono>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <stdexcept>
#include <string>

struct porch_code_object {
    std::shared_ptr<const porch::rt::code_object> object;
};

struct porch_event {
    porch::hip::event_t event = nullptr;
};

namespace {

    using namespace porch;

    std::string& last_error() {
        thread_local std::string message;
        return message;
    }

    template <typename F>
    porch_status guarded(F&& body) {
        try {
            body();
            last_error().clear();
            return PORCH_OK;
        }
        catch (const hip_jit::compilation_error& e) {
            last_error() = e.log();
            return PORCH_ERR_COMPILATION;
        }
        catch (const std::invalid_argument& e) {
            last_error() = e.what();
            return PORCH_ERR_INVALID_ARGUMENT;
        }
        catch (const std::out_of_range& e) {
            last_error() = e.what();
            return PORCH_ERR_OUT_OF_RANGE;
        }
        catch (const std::exception& e) {
            last_error() = e.what();
            return PORCH_ERR_RUNTIME;
        }
        catch (...) {
            last_error() = "unknown error";
            return PORCH_ERR_RUNTIME;
        }
    }

    void require(bool condition, const char* message) {
        if (!condition) throw std::invalid_argument(message);
    }

    ir::graph validated(const porch_graph* table) {
        ir::graph g = ir::from_c(table);
        ir::infer(g);
        if (g.n_inputs == 0) {
            // Only nodes reachable from the root count as references.
            bool any = false;
            for (const ir::node& n : g.nodes) any = any || n.kind == ir::op::input;
            if (!any)
                throw std::invalid_argument(
                    "tensor expression must reference at least one tensor"
                );
        }
        return g;
    }

    void write_shape(const std::vector<int64_t>& shape, int64_t* out, int32_t capacity,
                     int32_t* rank) {
        if (rank) *rank = static_cast<int32_t>(shape.size());
        if (out == nullptr) return;
        for (size_t i = 0; i < shape.size() && static_cast<int32_t>(i) < capacity; ++i)
            out[i] = shape[i];
    }

    void copy_text(const std::string& text, char* out, size_t capacity) {
        if (out == nullptr || capacity == 0) return;
        const size_t n = std::min(text.size(), capacity - 1);
        std::memcpy(out, text.data(), n);
        out[n] = '\0';
    }

} // namespace

extern "C" {

const char* porch_last_error(void) { return last_error().c_str(); }

int32_t porch_is_available(void) { return hip_jit::is_available() ? 1 : 0; }

porch_status porch_synchronize(void) {
    return guarded([] { hip_jit::synchronize(); });
}

porch_status porch_device_info(int32_t* compute_units, int32_t* clock_khz, char* arch,
                               size_t arch_capacity) {
    return guarded([&] {
        const rt::device_info& info = rt::device();
        if (compute_units) *compute_units = info.compute_units;
        if (clock_khz) *clock_khz = info.clock_khz;
        copy_text(info.arch, arch, arch_capacity);
    });
}

porch_status porch_buffer_create(size_t bytes, porch_buffer** out) {
    return guarded([&] {
        require(out != nullptr, "output pointer is null");
        *out = nullptr;
        auto* b = new porch_buffer();
        try {
            b->handle = hip_jit::device_buffer{bytes};
        }
        catch (...) {
            delete b;
            throw;
        }
        *out = b;
    });
}

void porch_buffer_release(porch_buffer* buffer) { delete buffer; }

size_t porch_buffer_size(const porch_buffer* buffer) {
    return buffer == nullptr ? 0 : buffer->handle.size_bytes();
}

uint64_t porch_buffer_device_pointer(const porch_buffer* buffer) {
    return buffer == nullptr
               ? 0
               : static_cast<uint64_t>(
                     reinterpret_cast<uintptr_t>(buffer->handle.device_pointer())
                 );
}

porch_status porch_copy_to_device(porch_buffer* buffer, const float* source, size_t count) {
    return guarded([&] {
        require(buffer != nullptr, "buffer is null");
        require(source != nullptr || count == 0, "source is null");
        hip_jit::copy_to_device(buffer->handle, {source, count});
    });
}

porch_status porch_copy_to_host(const porch_buffer* buffer, float* target, size_t count) {
    return guarded([&] {
        require(buffer != nullptr, "buffer is null");
        require(target != nullptr || count == 0, "target is null");
        hip_jit::copy_to_host(buffer->handle, {target, count});
    });
}

porch_status porch_compile(const char* source, const char* const* options, int32_t n_options,
                           porch_code_object** out) {
    return guarded([&] {
        require(source != nullptr, "source is null");
        require(out != nullptr, "output pointer is null");
        require(n_options >= 0 && (n_options == 0 || options != nullptr), "options are malformed");
        std::vector<std::string> extra;
        for (int32_t i = 0; i < n_options; ++i) {
            require(options[i] != nullptr, "option is null");
            extra.emplace_back(options[i]);
        }
        auto* code = new porch_code_object();
        try {
            code->object = rt::compile(source, extra);
        }
        catch (...) {
            delete code;
            throw;
        }
        *out = code;
    });
}

size_t porch_code_object_size(const porch_code_object* code) {
    return code == nullptr ? 0 : code->object->bytes.size();
}

const void* porch_code_object_data(const porch_code_object* code) {
    return code == nullptr ? nullptr : code->object->bytes.data();
}

void porch_code_object_release(porch_code_object* code) { delete code; }

namespace {
    porch_status raw_launch(const void* code, size_t code_size, const char* function,
                            const porch_buffer* const* inputs, int32_t n_inputs,
                            porch_buffer* out, size_t count, bool reduction) {
        return guarded([&] {
            require(code != nullptr && code_size > 0, "code object is empty");
            require(function != nullptr, "function name is null");
            require(out != nullptr, "output buffer is null");
            require(n_inputs >= 0 && (n_inputs == 0 || inputs != nullptr), "inputs are malformed");
            std::vector<const hip_jit::device_buffer*> list;
            for (int32_t i = 0; i < n_inputs; ++i)
                list.push_back(inputs[i] == nullptr ? nullptr : &inputs[i]->handle);
            const std::string_view bytes{static_cast<const char*>(code), code_size};
            if (reduction)
                hip_jit::launch_fused_reduction(bytes, function, list, out->handle, count);
            else
                hip_jit::launch_fused_elementwise(bytes, function, list, out->handle, count);
        });
    }
} // namespace

porch_status porch_launch_fused_elementwise(const void* code, size_t code_size,
                                            const char* function,
                                            const porch_buffer* const* inputs,
                                            int32_t n_inputs, porch_buffer* out,
                                            size_t count) {
    return raw_launch(code, code_size, function, inputs, n_inputs, out, count, false);
}

porch_status porch_launch_fused_reduction(const void* code, size_t code_size,
                                          const char* function,
                                          const porch_buffer* const* inputs,
                                          int32_t n_inputs, porch_buffer* out,
                                          size_t count) {
    return raw_launch(code, code_size, function, inputs, n_inputs, out, count, true);
}

porch_status porch_infer_shape(const porch_graph* graph, int64_t* shape, int32_t capacity,
                               int32_t* rank, int32_t* is_scalar) {
    return guarded([&] {
        ir::graph g = ir::from_c(graph);
        ir::infer(g);
        const ir::node& root = g.at(g.root());
        write_shape(root.out, shape, capacity, rank);
        if (is_scalar) *is_scalar = root.is_scalar ? 1 : 0;
    });
}

namespace {
    // Graphs already validated and planned, keyed by the exact bytes of the
    // node table and dims: a repeated table skips validation, shape
    // inference, compaction and key building.
    struct table_entry {
        std::shared_ptr<plan::graph_plan> plan;
        std::vector<int64_t> out_shape;
        int n_inputs = 0;
    };
    struct table_cache {
        std::mutex mutex;
        std::unordered_map<std::string, table_entry> entries;
    };
    table_cache& tables() {
        static table_cache* instance = new table_cache();
        return *instance;
    }

    std::string table_key(const porch_graph* graph) {
        std::string key;
        if (graph == nullptr || graph->nodes == nullptr || graph->n_nodes <= 0 ||
            graph->n_dims < 0 || (graph->n_dims > 0 && graph->dims == nullptr))
            return key;
        const size_t node_bytes = static_cast<size_t>(graph->n_nodes) * sizeof(porch_node);
        const size_t dim_bytes = static_cast<size_t>(graph->n_dims) * sizeof(int64_t);
        key.resize(node_bytes + dim_bytes);
        std::memcpy(key.data(), graph->nodes, node_bytes);
        if (dim_bytes) std::memcpy(key.data() + node_bytes, graph->dims, dim_bytes);
        return key;
    }

    porch_status materialize_impl(const porch_graph* graph, const porch_buffer* const* inputs,
                                  int32_t n_inputs, porch_buffer** out, int64_t* out_shape,
                                  int32_t capacity, int32_t* out_rank, porch_event* start,
                                  porch_event* stop) {
        return guarded([&] {
            const auto begin = std::chrono::steady_clock::now();
            require(out != nullptr, "output pointer is null");
            *out = nullptr;
            const capi::prepared_graph entry = capi::prepare(graph);
            const bool hit = entry.hit;
            require(n_inputs >= entry.n_inputs, "graph needs more input buffers");
            require(n_inputs == 0 || inputs != nullptr, "inputs are null");
            write_shape(entry.out_shape, out_shape, capacity, out_rank);
            auto* result = new porch_buffer();
            if (entry.plan == nullptr) { // empty result
                *out = result;
                return;
            }
            try {
                std::vector<rt::buffer_state*> buffers = capi::input_states(inputs, n_inputs);
                std::shared_ptr<rt::buffer_state> state = plan::run(
                    *entry.plan, buffers,
                    [](size_t bytes) -> std::shared_ptr<rt::buffer_state> {
                        return std::make_shared<hip_jit::device_buffer_state>(bytes);
                    },
                    start ? start->event : nullptr, stop ? stop->event : nullptr
                );
                result->handle = hip_jit::buffer_access::wrap(
                    std::static_pointer_cast<hip_jit::device_buffer_state>(state)
                );
                const double ms = rt::elapsed_ms(begin);
                std::scoped_lock lock{rt::counters_mutex()};
                if (hit) {
                    rt::counters().plan_hits += 1;
                    rt::counters().last_hit_us = ms * 1000.0;
                }
                else {
                    rt::counters().plan_misses += 1;
                    rt::counters().last_miss_ms = ms;
                }
            }
            catch (...) {
                delete result;
                throw;
            }
            *out = result;
        });
    }
} // namespace

extern "C++" {
namespace porch::capi {

    porch_status guarded_call(const std::function<void()>& body) {
        return guarded(body);
    }

    prepared_graph prepare(const porch_graph* graph) {
        const std::string key = table_key(graph);
        prepared_graph entry;
        if (!key.empty()) {
            std::scoped_lock lock{tables().mutex};
            auto found = tables().entries.find(key);
            if (found != tables().entries.end()) {
                entry.plan = found->second.plan;
                entry.out_shape = found->second.out_shape;
                entry.n_inputs = found->second.n_inputs;
                entry.hit = true;
                return entry;
            }
        }
        ir::graph g = validated(graph);
        const ir::node& root = g.at(g.root());
        if (root.is_scalar)
            throw std::invalid_argument("scalar expression cannot materialize to a tensor");
        table_entry table;
        table.out_shape = root.out;
        table.n_inputs = g.n_inputs;
        if (ir::checked_numel(root.out) > 0) {
            bool plan_hit = false;
            table.plan = plan::lookup(ir::compact(g), &plan_hit);
            entry.hit = plan_hit;
            if (!key.empty()) {
                std::scoped_lock lock{tables().mutex};
                // Bounded: a caller producing ever new tables (say, changing
                // shapes) must not grow this without end.  Entries are
                // rebuilt cheaply from the plan cache.
                if (tables().entries.size() >= 4096) tables().entries.clear();
                tables().entries.emplace(key, table);
            }
        }
        entry.plan = table.plan;
        entry.out_shape = table.out_shape;
        entry.n_inputs = table.n_inputs;
        return entry;
    }

    std::vector<rt::buffer_state*> input_states(const porch_buffer* const* inputs, int32_t n_inputs) {
        std::vector<rt::buffer_state*> buffers(static_cast<size_t>(std::max(n_inputs, 0)));
        for (int32_t i = 0; i < n_inputs; ++i) {
            buffers[static_cast<size_t>(i)] =
                inputs[i] == nullptr ? nullptr : hip_jit::buffer_access::state(inputs[i]->handle).get();
        }
        return buffers;
    }

    void write_result_shape(const std::vector<int64_t>& shape, int64_t* out, int32_t capacity,
                            int32_t* rank) {
        write_shape(shape, out, capacity, rank);
    }

} // namespace porch::capi
} // extern "C++"

porch_status porch_materialize(const porch_graph* graph, const porch_buffer* const* inputs,
                               int32_t n_inputs, porch_buffer** out, int64_t* out_shape,
                               int32_t capacity, int32_t* out_rank) {
    return materialize_impl(graph, inputs, n_inputs, out, out_shape, capacity, out_rank,
                            nullptr, nullptr);
}

porch_status porch_materialize_timed(const porch_graph* graph, const porch_buffer* const* inputs,
                                     int32_t n_inputs, porch_buffer** out, int64_t* out_shape,
                                     int32_t capacity, int32_t* out_rank, porch_event* start,
                                     porch_event* stop) {
    return materialize_impl(graph, inputs, n_inputs, out, out_shape, capacity, out_rank,
                            start, stop);
}

porch_status porch_plan(const porch_graph* graph, int32_t compile, char* json, size_t capacity) {
    return guarded([&] {
        ir::graph g = validated(graph);
        const ir::graph compacted = ir::compact(g);
        int cus = 256;
        if (hip_jit::is_available()) cus = rt::device().compute_units;
        std::shared_ptr<plan::graph_plan> p = plan::build(compacted, cus);
        if (compile) plan::compile(*p);
        copy_text(p->describe(), json, capacity);
    });
}

porch_status porch_plan_source(const porch_graph* graph, int32_t index, char* source,
                               size_t capacity, size_t* length) {
    return guarded([&] {
        ir::graph g = validated(graph);
        const ir::graph compacted = ir::compact(g);
        std::shared_ptr<plan::graph_plan> p = plan::build(compacted, 256);
        if (index < 0 || static_cast<size_t>(index) >= p->steps.size())
            throw std::out_of_range("plan has no kernel with that index");
        const std::string& text = p->steps[static_cast<size_t>(index)].code.source;
        if (length) *length = text.size();
        copy_text(text, source, capacity);
    });
}

porch_status porch_get_jit_stats(porch_jit_stats* stats) {
    return guarded([&] {
        require(stats != nullptr, "stats is null");
        std::scoped_lock lock{rt::counters_mutex()};
        const rt::jit_counters& c = rt::counters();
        stats->plan_hits = c.plan_hits;
        stats->plan_misses = c.plan_misses;
        stats->compiles = c.compiles;
        stats->launches = c.launches;
        stats->codegen_ms = c.codegen_ms;
        stats->compile_ms = c.compile_ms;
        stats->module_load_ms = c.module_load_ms;
        stats->last_miss_ms = c.last_miss_ms;
        stats->last_hit_us = c.last_hit_us;
        stats->disk_hits = c.disk_hits;
        stats->disk_ms = c.disk_ms;
        const hip::allocation_calls a = hip::allocation_counts();
        stats->device_allocs = a.device_allocs;
        stats->device_frees = a.device_frees;
        stats->host_allocs = a.host_allocs;
        stats->host_frees = a.host_frees;
        stats->module_loads = a.module_loads;
    });
}

porch_status porch_set_disk_cache(const char* directory) {
    return guarded([&] { rt::disk::set_directory(directory == nullptr ? "" : directory); });
}

porch_status porch_disk_cache_directory(char* out, size_t capacity) {
    return guarded([&] {
        require(out != nullptr && capacity > 0, "output buffer is empty");
        const std::string dir = rt::disk::directory();
        const size_t n = std::min(dir.size(), capacity - 1);
        std::memcpy(out, dir.data(), n);
        out[n] = '\0';
    });
}

porch_status porch_reset_jit_cache(void) {
    return guarded([] {
        {
            std::scoped_lock lock{tables().mutex};
            tables().entries.clear();
        }
        plan::clear_cache();
        rt::clear_caches();
    });
}

porch_status porch_event_create(porch_event** out) {
    return guarded([&] {
        require(out != nullptr, "output pointer is null");
        auto* e = new porch_event();
        hip::error_t rc = hip::runtime().event_create_with_flags(&e->event, hip::event_default);
        if (rc != hip::success) {
            delete e;
            hip::check(rc, "hipEventCreateWithFlags");
        }
        *out = e;
    });
}

porch_status porch_event_record(porch_event* event) {
    return guarded([&] {
        require(event != nullptr, "event is null");
        hip::check(
            hip::runtime().event_record(event->event, rt::current_stream()->handle()),
            "hipEventRecord"
        );
    });
}

porch_status porch_event_synchronize(porch_event* event) {
    return guarded([&] {
        require(event != nullptr, "event is null");
        hip::check(hip::runtime().event_synchronize(event->event), "hipEventSynchronize");
    });
}

porch_status porch_event_elapsed_ms(const porch_event* start, const porch_event* stop,
                                    float* ms) {
    return guarded([&] {
        require(start != nullptr && stop != nullptr && ms != nullptr, "argument is null");
        hip::check(hip::runtime().event_elapsed_time(ms, start->event, stop->event),
                   "hipEventElapsedTime");
    });
}

void porch_event_release(porch_event* event) {
    if (event == nullptr) return;
    try {
        (void)hip::runtime().event_destroy(event->event);
    }
    catch (...) {
    }
    delete event;
}

porch_status porch_release_cached_memory(size_t* released) {
    return guarded([&] {
        const size_t bytes = hip_jit::is_available() ? rt::release_cached_blocks() : 0;
        if (released != nullptr) *released = bytes;
    });
}

porch_status porch_flush_caches(size_t bytes) {
    return guarded([&] { rt::flush_caches(bytes); });
}

} // extern "C"
