/*
 * porch_amd.h — C ABI of the MI355X (gfx950) fused-graph backend for porch.
 *
 * Plain pointers, sizes and status codes; no C++ or torch types cross this
 * boundary.  The C++ API in include/porch/ (the .hpp headers) is a client of the same
 * library, and so are the Python mirror (porch_amd/) and the tests (ctypes).
 *
 * Every function that can fail returns a porch_status; the message of the
 * last failure on the calling thread is returned by porch_last_error().
 * Status codes map one-to-one onto the exception types porch throws:
 *   PORCH_ERR_INVALID_ARGUMENT  std::invalid_argument
 *   PORCH_ERR_OUT_OF_RANGE      std::out_of_range
 *   PORCH_ERR_RUNTIME           std::runtime_error (loader, driver)
 *   PORCH_ERR_COMPILATION       porch::cuda_jit::compilation_error (hiprtc log)
 *
 * Each line "replaces:" names the reference interface (file:line in
 * AkhilSamavedam/porch) whose behaviour the entry point provides.
 */
#ifndef PORCH_AMD_H
#define PORCH_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t porch_status;

#define PORCH_OK 0
#define PORCH_ERR_INVALID_ARGUMENT 1
#define PORCH_ERR_OUT_OF_RANGE 2
#define PORCH_ERR_RUNTIME 3
#define PORCH_ERR_COMPILATION 4

/* Message of the last failing call on this thread ("" if none).
 * replaces: the what() text of the exceptions thrown in src/cuda_jit.cpp:304-339
 * and src/tensor.cpp:190-496. */
const char* porch_last_error(void);

/* ------------------------------------------------------------------ */
/* Device and streams                                                  */
/* ------------------------------------------------------------------ */

/* 1 when libamdhip64 + libhiprtc load and device 0 initialises, else 0.
 * Never fails.  replaces: cuda_jit::is_available, src/cuda_jit.cpp:634-645. */
int32_t porch_is_available(void);

/* Waits for all work queued on the calling thread's current stream.
 * replaces: cuda_jit::synchronize, src/cuda_jit.cpp:761. */
porch_status porch_synchronize(void);

/* Device facts read at init: compute units, shader clock (kHz), arch name
 * (e.g. "gfx950:sramecc+:xnack-"), copied into arch[arch_capacity].
 * No reference counterpart (the reference hard-codes device 0,
 * src/cuda_jit.cpp:446-450); used to state rooflines. */
porch_status porch_device_info(int32_t* compute_units, int32_t* clock_khz,
                               char* arch, size_t arch_capacity);

/* ------------------------------------------------------------------ */
/* Device buffers (stream-ordered hipMallocAsync / hipFreeAsync)       */
/* ------------------------------------------------------------------ */

typedef struct porch_buffer porch_buffer;

/* Allocates `bytes` on the calling thread's stream; bytes == 0 gives an
 * empty buffer with no device memory.
 * replaces: device_buffer::device_buffer(size_t), src/cuda_jit.cpp:533-547,617-619. */
porch_status porch_buffer_create(size_t bytes, porch_buffer** out);

/* Drops this handle; the memory is freed stream-ordered once every stream
 * that used it has passed that use.
 * replaces: ~device_buffer_state, src/cuda_jit.cpp:552-566. */
void porch_buffer_release(porch_buffer* buffer);

/* replaces: device_buffer::size_bytes, src/cuda_jit.cpp:625-627. */
size_t porch_buffer_size(const porch_buffer* buffer);

/* Device address of the allocation (0 for an empty buffer). */
uint64_t porch_buffer_device_pointer(const porch_buffer* buffer);

/* Host -> device copy of `count` floats, synchronous for the host.
 * replaces: cuda_jit::copy_to_device, src/cuda_jit.cpp:711-734. */
porch_status porch_copy_to_device(porch_buffer* buffer, const float* source,
                                  size_t count);

/* Device -> host copy of `count` floats after the producing work finished.
 * replaces: cuda_jit::copy_to_host, src/cuda_jit.cpp:736-759. */
porch_status porch_copy_to_host(const porch_buffer* buffer, float* target,
                                size_t count);

/* ------------------------------------------------------------------ */
/* hiprtc compilation and raw launches                                 */
/* ------------------------------------------------------------------ */

typedef struct porch_code_object porch_code_object;

/* Compiles HIP source to a gfx950 code object with hiprtc; results are
 * cached by (source, options).  Compile failure returns
 * PORCH_ERR_COMPILATION with the hiprtc log as the error message.
 * replaces: cuda_jit::compile_to_ptx, src/cuda_jit.cpp:647-703 (PTX text
 * becomes an AMDGPU ELF code object). */
porch_status porch_compile(const char* source, const char* const* options,
                           int32_t n_options, porch_code_object** out);
size_t porch_code_object_size(const porch_code_object* code);
const void* porch_code_object_data(const porch_code_object* code);
void porch_code_object_release(porch_code_object* code);

/* Launches `function` of a code object with the reference's fixed
 * geometry (256 threads per block, ceil(count/256) blocks) and parameters
 * (in0..in{n-1}, out, uint64 count).
 * replaces: cuda_jit::launch_fused_elementwise, src/cuda_jit.cpp:789-868. */
porch_status porch_launch_fused_elementwise(
    const void* code, size_t code_size, const char* function,
    const porch_buffer* const* inputs, int32_t n_inputs, porch_buffer* out,
    size_t count);

/* Same parameters; one 256-thread block per output element.
 * replaces: cuda_jit::launch_fused_reduction, src/cuda_jit.cpp:870-948. */
porch_status porch_launch_fused_reduction(
    const void* code, size_t code_size, const char* function,
    const porch_buffer* const* inputs, int32_t n_inputs, porch_buffer* out,
    size_t count);

/* ------------------------------------------------------------------ */
/* Lazy graphs                                                         */
/* ------------------------------------------------------------------ */

/* Node kinds: the reference's expr_kind, src/tensor.cpp:26-46, same order. */
#define PORCH_OP_INPUT 0
#define PORCH_OP_SCALAR 1
#define PORCH_OP_ADD 2
#define PORCH_OP_SUBTRACT 3
#define PORCH_OP_MULTIPLY 4
#define PORCH_OP_DIVIDE 5
#define PORCH_OP_MATMUL 6
#define PORCH_OP_SLICE 7
#define PORCH_OP_RESHAPE 8
#define PORCH_OP_UNSQUEEZE 9
#define PORCH_OP_TRANSPOSE 10
#define PORCH_OP_BROADCAST 11
#define PORCH_OP_CONCAT 12
#define PORCH_OP_SUM 13
#define PORCH_OP_MAX 14
#define PORCH_OP_MAXIMUM 15
#define PORCH_OP_MINIMUM 16
#define PORCH_OP_EXP 17
#define PORCH_OP_RECIPROCAL 18
/* Rank-N axis permutation.  No counterpart in the reference, whose only
 * axis reordering is the rank-2 transpose (src/tensor.cpp:424-438 for its
 * shape rule, 562-571 for its index map, 1425-1429 for its builder); this
 * generalises it.  rank/dims hold the permutation: output dimension i is
 * operand dimension dims[i]. */
#define PORCH_OP_PERMUTE 19
/* Batched matmul: [B, M, K] @ [B, K, N] -> [B, M, N], each batch entry the
 * rank-2 matmul's sequential fp32 sum over k.  No counterpart in the
 * reference, whose matmul is rank-2 only (src/tensor.cpp:366-385); lhs and
 * rhs are the operands, as for MATMUL.  A shared operand is a broadcast_to
 * of a rank-2 tensor to [B, K, N] (a view: it is not copied). */
#define PORCH_OP_BATCHED_MATMUL 20

/* One IR node; the flattened form of tensor_expr::node, src/tensor.cpp:48-60.
 * Operands refer to earlier entries, so a node table is topologically
 * ordered and the last entry is the root. */
typedef struct porch_node {
    int32_t op;      /* PORCH_OP_* */
    int32_t lhs;     /* operand node index, or -1 */
    int32_t rhs;     /* second operand node index, or -1 */
    int32_t input;   /* INPUT: index into the inputs array */
    float scalar;    /* SCALAR: the value */
    int32_t axis;    /* UNSQUEEZE, CONCAT, SUM, MAX */
    int32_t keepdim; /* SUM, MAX */
    int32_t rank;    /* INPUT, SLICE, RESHAPE, BROADCAST: extents in dims;
                        PERMUTE: the permutation's length */
    int64_t dims;    /* offset into porch_graph.dims: shape[rank], then for
                        SLICE strides[rank] */
    int64_t offset;  /* SLICE: storage offset into the source */
} porch_node;

typedef struct porch_graph {
    const porch_node* nodes;
    int32_t n_nodes;
    const int64_t* dims;
    int64_t n_dims;
} porch_graph;

/* Shape inference and validation only (no device needed).  Writes the
 * root's extents (up to capacity), its rank, and whether it is a scalar.
 * replaces: infer_expression, src/tensor.cpp:341-496, and
 * tensor_expr::shape, src/tensor.cpp:1336-1341. */
porch_status porch_infer_shape(const porch_graph* graph, int64_t* shape,
                               int32_t capacity, int32_t* rank,
                               int32_t* is_scalar);

/* Plans, compiles (cached by graph hash), allocates the output on the
 * calling thread's stream and launches the fused kernels.  `inputs[i]`
 * backs every INPUT node with input == i; each must hold at least the
 * node's extent product of floats.  The returned buffer holds the root's
 * values in contiguous row-major order.
 * replaces: materialize_expression, src/tensor.cpp:1002-1066 (with
 * lower_nested_reductions 970-989 and the launches 1036-1061). */
porch_status porch_materialize(const porch_graph* graph,
                               const porch_buffer* const* inputs,
                               int32_t n_inputs, porch_buffer** out,
                               int64_t* out_shape, int32_t capacity,
                               int32_t* out_rank);

/* Size of the device array porch_materialize_noalloc takes temporaries
 * from: one per GPU, held from the first call there until the process
 * ends. */
#define PORCH_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* porch_materialize into `out`, an existing buffer of at least the result's
 * size, allocating no memory once it has run once for the graph's
 * structure on the calling thread and device: such a call makes no
 * hipMalloc, hipFree, hipHostMalloc or hipModuleLoadData call, or their
 * async forms, in the library or any routine it calls.  The first call for
 * a structure (make it outside any HIP graph capture, as a warm-up) may:
 * it compiles and loads the graph's kernels (hipModuleLoadData allocates
 * code memory), may create the thread's stream, and on the first call on a
 * device looks up the array's address, which makes the runtime load the
 * array.  The same kernels run;
 * the graph's temporaries (memoised reductions, split-reduction partials,
 * materialised product operands) come from the fixed per-GPU array of
 * PORCH_NOALLOC_SCRATCH_BYTES, and a graph that needs more fails with
 * PORCH_ERR_INVALID_ARGUMENT.  Every call on a GPU shares that array:
 * calls that overlap on one GPU (threads with different streams) race;
 * calls on one stream are ordered.  The first call for a graph's structure
 * compiles and loads its kernels as porch_materialize does.  Exported by
 * the companion library libporch_amd_noalloc.so, which holds the array.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid it). */
porch_status porch_materialize_noalloc(const porch_graph* graph,
                                       const porch_buffer* const* inputs,
                                       int32_t n_inputs, porch_buffer* out,
                                       int64_t* out_shape, int32_t capacity,
                                       int32_t* out_rank);

/* porch_materialize with HIP events attached to the first and the last
 * kernel launch (hipExtModuleLaunchKernel), so elapsed time between them is
 * the kernels' own execution on the calling thread's stream.  Events come
 * from porch_event_create (declared below).
 * No reference counterpart: measurement support for the same path. */
typedef struct porch_event porch_event;
porch_status porch_materialize_timed(const porch_graph* graph,
                                     const porch_buffer* const* inputs,
                                     int32_t n_inputs, porch_buffer** out,
                                     int64_t* out_shape, int32_t capacity,
                                     int32_t* out_rank, porch_event* start,
                                     porch_event* stop);

/* Plans and compiles the graph without a device and without launching
 * (hiprtc runs on the host).  Writes a JSON description of the plan
 * (kernel classes, launch geometry, temporaries) into json[capacity].
 * No reference counterpart: offline form of the codegen in
 * src/tensor.cpp:874-962 for tests and the build check. */
porch_status porch_plan(const porch_graph* graph, int32_t compile, char* json,
                        size_t capacity);

/* HIP source of kernel `index` of the graph's plan, into source[capacity];
 * *length receives the full length. */
porch_status porch_plan_source(const porch_graph* graph, int32_t index,
                               char* source, size_t capacity, size_t* length);

/* JIT statistics since process start (or the last reset). */
typedef struct porch_jit_stats {
    uint64_t plan_hits;      /* materializations served from the graph cache */
    uint64_t plan_misses;    /* graphs planned + compiled */
    uint64_t compiles;       /* hiprtc invocations */
    uint64_t launches;       /* kernels launched */
    double codegen_ms;       /* host time planning and emitting source */
    double compile_ms;       /* host time inside hiprtc */
    double module_load_ms;   /* host time in hipModuleLoadData */
    double last_miss_ms;     /* last cold materialize: plan+compile+load */
    double last_hit_us;      /* last cache-hit materialize, call to return */
    uint64_t disk_hits;      /* code objects read from the on-disk cache */
    double disk_ms;          /* host time reading them */
    /* Calls into libamdhip64 that allocate or release memory, counted from
     * the start of the process (no reference counterpart). */
    uint64_t device_allocs;  /* hipMallocAsync */
    uint64_t device_frees;   /* hipFreeAsync */
    uint64_t host_allocs;    /* hipHostMalloc (pinned staging chunks) */
    uint64_t host_frees;     /* hipHostFree */
    uint64_t module_loads;   /* hipModuleLoadData (device code memory) */
} porch_jit_stats;

porch_status porch_get_jit_stats(porch_jit_stats* stats);

/* Drops every cached plan, code object and module (for cold-JIT timing).
 * The on-disk cache is left as it is. */
porch_status porch_reset_jit_cache(void);

/* Directory of the persistent code-object cache: compiled kernels are
 * written there and read back by later processes instead of compiling
 * again.  NULL or "" turns it off for the rest of the process.  By default
 * the cache is off unless the environment variable PORCH_CACHE_DIR names a
 * directory.  Entries are checked (full key, hiprtc version, checksum) on
 * every read, so a stale or damaged file is recompiled, never loaded.
 * No reference counterpart: the reference's cache lives in memory only,
 * src/cuda_jit.cpp:358-378. */
porch_status porch_set_disk_cache(const char* directory);

/* The directory in use ("" when off), copied into out[capacity]. */
porch_status porch_disk_cache_directory(char* out, size_t capacity);

/* ------------------------------------------------------------------ */
/* Timing support (HIP events on the calling thread's current stream)   */
/* ------------------------------------------------------------------ */

porch_status porch_event_create(porch_event** out);
porch_status porch_event_record(porch_event* event);
porch_status porch_event_synchronize(porch_event* event);
porch_status porch_event_elapsed_ms(const porch_event* start,
                                    const porch_event* stop, float* ms);
void porch_event_release(porch_event* event);

/* Writes `bytes` of a scratch buffer on the current stream so that the
 * next kernel finds neither L2 nor the Infinity Cache warm. */
porch_status porch_flush_caches(size_t bytes);

/* Returns the device memory the allocator keeps cached for reuse (blocks
 * of released buffers, at most 32 GiB over all streams) to the
 * stream-ordered pool, each on the stream that last used it; `released`
 * (may be NULL) receives the bytes.  Live buffers are not touched.
 * No reference counterpart: for callers under memory pressure (the
 * reference keeps no cache: each buffer is freed when its last handle
 * goes, src/cuda_jit.cpp:552-566). */
porch_status porch_release_cached_memory(size_t* released);

/* ------------------------------------------------------------------ */
/* Seeded synthetic inputs (host side, splitmix64)                      */
/* ------------------------------------------------------------------ */

/* u_i = (splitmix64_i(seed) >> 40) * 2^-24; out_i = lo + (hi - lo) * u_i
 * evaluated in double and rounded to float. */
void porch_synth_uniform(float* out, size_t count, uint64_t seed, double lo,
                         double hi);
/* Box-Muller in double over consecutive uniform pairs; out = mean + std*z. */
void porch_synth_normal(float* out, size_t count, uint64_t seed, double mean,
                        double stddev);
/* Replaces out_i by `value` where a second splitmix64 stream (seeded with
 * `seed`) draws u_i < p. */
void porch_synth_replace(float* out, size_t count, uint64_t seed, double p,
                         float value);

#ifdef __cplusplus
}
#endif

#endif /* PORCH_AMD_H */
