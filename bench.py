"""Benchmark of porch's fused-graph path on one MI355X.

A step is one materialisation of a benchmark graph over one batch of
inputs already resident in HBM: porch_materialize on the graph's node
table (graph-cache lookup, stream-ordered output allocation, kernel launch)
and the release of the output.  Consecutive steps rotate over enough input
copies that no step finds its inputs in L2 or the 256 MB Infinity Cache.

Two timed regions run per config: region A (the whole-job `value`, K steps
back to back, wall clock between synchronisations) and region B (the same K
steps with a HIP event pair attached to each kernel dispatch; their mean is
the per-launch duration behind `roofline.achieved`).

The headline line is the view chain (strided slices + transposes + concat
over x fp32 [4096, 4096]): HBM GB/s of algorithmic bytes (all of x read, the
output written).  The other workloads are reported beside it under
"configs", each with its roofline fraction and JIT latency, followed by
workloads of the IR extensions (a batched transpose and a head permute via
permute, a batched matmul with an epilogue, attention scores q @ k^T over 16
heads, a softmax over 262144-value rows) and two products with one short
side (16 columns, 32 rows: a kernel split over K and its combine, timed from
the first kernel's start to the second's end).  The host evaluator (the
oracle, OpenMP) is timed on this machine's cores as the CPU baseline: 10 s of
CPU work for the headline workload, 4 s for each other one.

`roofline.traffic` is the HBM bytes per launch that rocprofv3's FETCH_SIZE
and WRITE_SIZE counters read for the same kernel, scaled by what they read
for a copy kernel of known size; both come from the counter summaries under
profiles/ (null when a workload has none).

    python bench.py [--steps K] [--warmup W] [--configs view_chain,...] [--no-cpu]
    python bench.py --controls LAUNCHES   (control kernels beside the elementwise, view
                                          chain, vocabulary-softmax and wide-product
                                          workloads, under rocprofv3)
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
# Cold JIT is measured as a real hiprtc compile: comgr's own on-disk compile
# cache (which survives between processes) stays off in this process.
os.environ.setdefault("AMD_COMGR_CACHE", "0")

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E
FP32_MFMA_PEAK_TFLOPS = 157.3    # 256 CU x 256 flop/clk x 2.4 GHz

METRIC = "fused-graph HBM GB/s (% of peak); fp32 matmul TFLOP/s (% MFMA peak); JIT ms"

# Algorithmic work per step (bytes for HBM-bound graphs, flops for the matmul).
WORK = {
    "elementwise": ("hbm", 3 * 4 * (1 << 20)),
    "view_chain": ("hbm", 4096 * 4096 * 4 + 4096 * 2048 * 4),
    "softmax": ("hbm", 2 * 8192 * 4096 * 4),
    "logistic_rowsum": ("hbm", 16384 * 2048 * 4 + 2 * 2048 * 4 + 16384 * 4),
    "matmul_epilogue": ("mfma", 2 * 4096 ** 3),
    "copy": ("hbm", 2 * 8192 * 8192 * 4),
    "batched_transpose": ("hbm", 2 * 64 * 512 * 512 * 4),
    "heads_permute": ("hbm", 2 * 32 * 1024 * 16 * 128 * 4),
    "batched_matmul": ("mfma", 2 * 32 * 1024 ** 3),
    "attention_scores": ("mfma", 2 * 16 * 4096 * 64 * 4096),
    "vocab_softmax": ("hbm", 2 * 512 * 262144 * 4),
    # A and B read once, C written (the partial products between the two
    # kernels are not algorithmic bytes)
    "narrow_product": ("hbm", (4096 * 4096 + 4096 * 16 + 4096 * 16) * 4),
    "wide_product": ("hbm", (32 * 4096 + 4096 * 4096 + 32 * 4096) * 4),
}
DESCRIPTION = {
    "elementwise": "(a + b) * 2 - 1, a, b fp32 [1048576]",
    "view_chain": "concat(transpose(x[0::2,1::2]), transpose(x[1::2,0::2]), 0) + 1, x fp32 [4096,4096]",
    "softmax": "softmax(x, 1), x fp32 [8192,4096]",
    "logistic_rowsum": "sum(logistic(relu(x*bcast(w) + bcast(bias))), 1), x fp32 [16384,2048]",
    "matmul_epilogue": "relu(A @ B + bcast(bias)) - 0.5, A, B fp32 [4096,4096]",
    "copy": "reshape(x) copy, x fp32 [8192,8192] (byte-counter calibration)",
    "batched_transpose": "permute(x, [0,2,1]), x fp32 [64,512,512]",
    "heads_permute": "permute(x, [0,2,1,3]), x fp32 [32,1024,16,128]",
    "batched_matmul": "relu(batched_matmul(A, B) + bcast(bias)) - 0.5, A, B fp32 [32,1024,1024]",
    "attention_scores": "batched_matmul(q, k) * 0.125, q fp32 [16,4096,64], k fp32 [16,64,4096]",
    "vocab_softmax": "softmax(x, 1), x fp32 [512,262144]",
    "narrow_product": "A @ B, A fp32 [4096,4096], B fp32 [4096,16]",
    "wide_product": "A @ B, A fp32 [32,4096], B fp32 [4096,4096]",
}
# Minimum length of each workload's untimed warm-up (see run_config).
WARM_SECONDS = 0.25
# Input copies rotated through so that a step never re-reads cached data.
ROTATION = {"elementwise": 48, "view_chain": 8, "softmax": 4, "logistic_rowsum": 6,
            "matmul_epilogue": 1, "copy": 2, "batched_transpose": 4, "heads_permute": 2,
            "batched_matmul": 1, "attention_scores": 1, "vocab_softmax": 1, "narrow_product": 8,
            "wide_product": 8}
# Counter summaries (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE) per workload.
PROFILES = os.path.join(ROOT, "profiles")


def profiled_traffic(name: str):
    """HBM bytes per launch from the workload's committed counter summary."""
    if not os.path.isdir(PROFILES):
        return None
    for entry in sorted(os.listdir(PROFILES)):
        if not (entry.startswith(name + ".") and entry.endswith(".txt")):
            continue
        with open(os.path.join(PROFILES, entry)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    return None


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def run_config(porch, name: str, steps: int, warmup: int) -> dict:
    from porch_amd import _lib, synth
    from porch_amd.workloads import config_graph, config_inputs, config_shapes

    shapes = config_shapes(name)
    host = config_inputs(name)
    copies = ROTATION[name]
    sets = [[porch.tensor(s, v) for s, v in zip(shapes, host)] for _ in range(copies)]
    expr = config_graph(name, sets[0])
    nodes, dims, n_dims, inputs, _ = porch.serialize(expr)
    graph = porch._graph(nodes, dims, n_dims)
    # The node table is the same for every copy; only the buffers differ.
    handles = []
    for s in sets:
        _, _, _, ins, _ = porch.serialize(config_graph(name, s))
        handles.append((ctypes.c_void_p * len(ins))(*[t.device_data().handle for t in ins]))
    n_in = len(inputs)
    out = ctypes.c_void_p()

    def step(i: int, start=None, stop=None) -> None:
        if start is None:
            _lib.check(_lib.lib.porch_materialize(ctypes.byref(graph), handles[i % copies], n_in,
                                                  ctypes.byref(out), None, 0, None))
        else:
            _lib.check(_lib.lib.porch_materialize_timed(
                ctypes.byref(graph), handles[i % copies], n_in, ctypes.byref(out), None, 0, None,
                start.handle, stop.handle))
        _lib.lib.porch_buffer_release(out)

    # Cold JIT: codegen + hiprtc + module load of this graph in this process
    # (the persistent code-object cache off, so hiprtc really runs).
    porch.set_disk_cache(None)
    porch.reset_jit_cache()
    before = porch.jit_stats()
    step(0)
    porch.synchronize()
    after = porch.jit_stats()
    cold_ms = after["last_miss_ms"]
    cold_split = {part: after[part] - before[part]
                  for part in ("codegen_ms", "compile_ms", "module_load_ms")}

    # Disk-warm JIT: a later process whose code objects are in the persistent
    # cache.  The code objects are written here; a child process then times
    # its first materialisation of the graph (codegen + file read + module
    # load + launch; no hiprtc).
    with tempfile.TemporaryDirectory(prefix="porch_jit_") as cache:
        porch.set_disk_cache(cache)
        porch.reset_jit_cache()
        step(0)
        porch.synchronize()
        porch.set_disk_cache(None)
        disk_ms = disk_warm_jit_ms(name, cache)

    # Warm-up, untimed: at least `warmup` steps and at least WARM_SECONDS of
    # back-to-back work, synchronising every 8 steps so the queue stays
    # short.  An idle MI355X ramps its clocks over the first tens of
    # milliseconds of load (the 4096^3 matmul runs ~1130 us on the first
    # launches and settles near 975 us after ~25 of them), so fewer steps
    # would time the ramp rather than the kernel.
    warm_start = time.perf_counter()
    done = 0
    while done < warmup or time.perf_counter() - warm_start < WARM_SECONDS:
        for _ in range(8):
            step(done)
            done += 1
        porch.synchronize()

    # Timed region A (whole-job value): K steps back to back.
    porch.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    porch.synchronize()
    elapsed = time.perf_counter() - t0

    # Timed region B (roofline): the same steps, each kernel launched with a
    # HIP event pair attached to its dispatch on porch's stream
    # (hipExtModuleLaunchKernel), so start/stop bracket the kernel itself.
    # Short HBM-bound kernels get at least 200 launches, so that a few slow
    # dispatches do not decide the mean.
    launches = max(steps, 200) if WORK[name][0] == "hbm" else max(steps, 20)
    starts = [synth.Event() for _ in range(launches)]
    stops = [synth.Event() for _ in range(launches)]
    porch.synchronize()
    for i in range(launches):
        step(i, starts[i], stops[i])
    porch.synchronize()
    kernel_ms = [a.elapsed_ms(b) for a, b in zip(starts, stops)]

    # Host latency of a cache-hit materialisation (call to return).
    hit_us = []
    for i in range(min(steps, 50)):
        step(i)
        hit_us.append(porch.jit_stats()["last_hit_us"])
    porch.synchronize()

    bound, work = WORK[name]
    mean_kernel_s = float(np.mean(kernel_ms)) / 1e3
    if bound == "hbm":
        achieved = work / mean_kernel_s / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
        whole_job = work * steps / elapsed / 1e9
    else:
        achieved = work / mean_kernel_s / 1e12
        peak, unit = FP32_MFMA_PEAK_TFLOPS, "TFLOP/s"
        whole_job = work * steps / elapsed / 1e12
    plan = porch.plan(expr)
    return {
        "workload": DESCRIPTION[name],
        "kernels": [k["kind"] for k in plan["kernels"]],
        "value": whole_job,
        "unit": unit,
        "ms_per_step": elapsed / steps * 1e3,
        "kernel_ms_mean": float(np.mean(kernel_ms)),
        "kernel_ms_median": float(np.median(kernel_ms)),
        "roofline": {"bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
                     "frac": achieved / peak, "traffic": profiled_traffic(name),
                     "launch_us": {"mean": float(np.mean(kernel_ms)) * 1e3,
                                   "median": float(np.median(kernel_ms)) * 1e3,
                                   "launches": launches, "frac_uses": "mean"}},
        "jit_ms": {"cold": cold_ms, "cold_codegen": cold_split["codegen_ms"],
                   "cold_hiprtc": cold_split["compile_ms"], "cold_module_load": cold_split["module_load_ms"],
                   "disk": disk_ms, "hit": float(np.median(hit_us)) / 1e3},
        "steps": steps,
    }


def disk_warm_jit_ms(name: str, cache: str):
    """First-materialisation time of workload `name` in a fresh process whose
    persistent code-object cache (`cache`) already holds its kernels."""
    env = dict(os.environ, PORCH_CACHE_DIR=cache)
    try:
        done = subprocess.run([sys.executable, os.path.abspath(__file__), "--jit-probe", name],
                              env=env, capture_output=True, text=True, timeout=300)
        probe = json.loads(done.stdout.strip().splitlines()[-1])
    except (subprocess.SubprocessError, ValueError, IndexError) as error:
        log(f"{name}: disk-warm JIT probe failed: {error}")
        return None
    if not probe.get("disk_hits"):
        log(f"{name}: disk-warm JIT probe compiled instead of reading the cache")
        return None
    return probe["first_ms"]


def jit_probe(name: str) -> int:
    """Child side of disk_warm_jit_ms: one materialisation, timed inside the
    library, then its JIT counters as one JSON line."""
    import porch_amd as porch
    from porch_amd.workloads import config_graph, config_inputs, config_shapes

    if not porch.is_available():
        return 1
    tensors = [porch.tensor(s, v) for s, v in zip(config_shapes(name), config_inputs(name))]
    expr = config_graph(name, tensors)
    porch.synchronize()
    porch.materialize(expr)
    porch.synchronize()
    stats = porch.jit_stats()
    print(json.dumps({"first_ms": stats["last_miss_ms"], "disk_hits": stats["disk_hits"],
                      "compiles": stats["compiles"], "module_load_ms": stats["module_load_ms"]}),
          flush=True)
    return 0


def cpu_baseline(name: str, min_seconds: float = 10.0) -> dict:
    """The host evaluator (the oracle, OpenMP over the host's threads) timed
    on the same workload, repeated until at least `min_seconds` of CPU work
    has run; the median run is reported."""
    from oracle import host
    from porch_amd.workloads import config_graph, config_inputs, config_shapes

    import porch_amd as porch

    shapes = config_shapes(name)
    values = config_inputs(name)
    tensors = []
    for s, v in zip(shapes, values):
        t = porch.tensor.__new__(porch.tensor)
        t._state = porch._State(s, porch.device())
        t._state.storage = porch._Storage(None, v)
        tensors.append(t)
    sample = "the full workload"
    scale = 1.0
    if name == "matmul_epilogue":
        rows = 256  # 1/16 of the rows of A and C; time scaled by 16
        a, b, bias = values
        tensors[0]._state = porch._State([rows, 4096], porch.device())
        tensors[0]._state.storage = porch._Storage(None, a[: rows * 4096])
        expr = porch.relu(porch.matmul(tensors[0], tensors[1]) +
                          porch.broadcast_to(tensors[2], [rows, 4096])) - 0.5
        sample = f"{rows} of the 4096 rows of C per run (time x {4096 // rows})"
        scale = 4096 / rows
    elif name == "batched_matmul":
        entries = 1  # 1 of the 32 batch entries; time scaled by 32
        a, b, bias = values
        for i, (shape, v) in enumerate(((([entries, 1024, 1024]), a), (([entries, 1024, 1024]), b))):
            tensors[i]._state = porch._State(shape, porch.device())
            tensors[i]._state.storage = porch._Storage(None, v[: entries * 1024 * 1024])
        expr = porch.relu(porch.batched_matmul(tensors[0], tensors[1]) +
                          porch.broadcast_to(tensors[2], [entries, 1024, 1024])) - 0.5
        sample = f"{entries} of the 32 batch entries per run (time x {32 // entries})"
        scale = 32 / entries
    elif name == "attention_scores":
        rows = 256  # 256 of the 4096 rows of one of the 16 entries; time scaled by 256
        q, k = values
        tensors[0]._state = porch._State([1, rows, 64], porch.device())
        tensors[0]._state.storage = porch._Storage(None, q[: rows * 64])
        tensors[1]._state = porch._State([1, 64, 4096], porch.device())
        tensors[1]._state.storage = porch._Storage(None, k[: 64 * 4096])
        expr = porch.batched_matmul(tensors[0], tensors[1]) * 0.125
        sample = f"{rows} rows of 1 of the 16 entries per run (time x {16 * 4096 // rows})"
        scale = 16 * 4096 / rows
    else:
        expr = config_graph(name, tensors)
    times = []
    host.evaluate(expr)  # warm-up
    start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - start < min_seconds:
        t0 = time.perf_counter()
        host.evaluate(expr)
        times.append((time.perf_counter() - t0) * scale)
    spent = time.perf_counter() - start
    seconds = float(np.median(times))
    bound, work = WORK[name]
    value = work / seconds / (1e9 if bound == "hbm" else 1e12)
    return {"value": value, "unit": "GB/s" if bound == "hbm" else "TFLOP/s",
            "cores": host.threads(), "cpu_model": cpu_model(), "kind": "port",
            "sample": f"host evaluator on {sample}, median of {len(times)} runs over {spent:.1f} s",
            "seconds": seconds}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# Control kernels at the elementwise workload's launch geometry (1024
# workgroups of 256 lanes, one float4 of each operand per lane), launched
# through porch's raw launch path (the reference's in0, in1, out, count
# parameters): an empty kernel, the reads alone, the writes alone, and a
# copy.  Their rocprofv3 durations set the floor the elementwise kernel is
# compared with.
CONTROL_SOURCE = r"""
typedef float porch_v4f __attribute__((ext_vector_type(4)));
extern "C" __global__ void __launch_bounds__(256) porch_control_empty(
    const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out,
    unsigned long long count) {}
extern "C" __global__ void __launch_bounds__(256) porch_control_read(
    const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out,
    unsigned long long count) {
    const unsigned long long g = blockIdx.x * 256ull + threadIdx.x;
    if (g >= count) return;
    const porch_v4f x = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(a0) + g);
    const porch_v4f y = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(a1) + g);
    const float s = ((x.x + x.y) + (x.z + x.w)) + ((y.x + y.y) + (y.z + y.w));
    if (s == 1234.5f) out[g] = s;  // never true for U[-1,1] inputs: keeps the loads, stores nothing
}
extern "C" __global__ void __launch_bounds__(256) porch_control_write(
    const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out,
    unsigned long long count) {
    const unsigned long long g = blockIdx.x * 256ull + threadIdx.x;
    if (g >= count) return;
    reinterpret_cast<float4*>(out)[g] = make_float4(1.0f, 2.0f, 3.0f, (float)g);
}
extern "C" __global__ void __launch_bounds__(256) porch_control_copy(
    const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out,
    unsigned long long count) {
    const unsigned long long g = blockIdx.x * 256ull + threadIdx.x;
    if (g >= count) return;
    const porch_v4f x = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(a0) + g);
    reinterpret_cast<float4*>(out)[g] = make_float4(x.x, x.y, x.z, x.w);
}
// The view chain's bytes in coalesced order: `count` lanes, each reading 32
// float4 of a0 (8 rounds of 4, strided by the lane count: all of x
// [4096,4096] at count = 131072) and writing two floats of each (out
// [4096,2048]), with the workload's + 1.
extern "C" __global__ void __launch_bounds__(256) porch_control_half(
    const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out,
    unsigned long long count) {
    typedef float porch_v2f __attribute__((ext_vector_type(2)));
    const unsigned long long g = blockIdx.x * 256ull + threadIdx.x;
    if (g >= count) return;
    const porch_v4f* x = reinterpret_cast<const porch_v4f*>(a0);
    porch_v2f* y = reinterpret_cast<porch_v2f*>(out);
    for (int round = 0; round < 8; ++round) {
        porch_v4f v[4];
        for (int r = 0; r < 4; ++r) v[r] = __builtin_nontemporal_load(x + g + (round * 4 + r) * count);
        for (int r = 0; r < 4; ++r) y[g + (round * 4 + r) * count] = (porch_v2f){v[r].y + 1.0f, v[r].w + 1.0f};
    }
}
// Other launch shapes of the elementwise workload's arithmetic, (a + b) * 2 - 1
// over 262144 float4 of each operand: `count` lanes (256 a workgroup), each
// taking 262144 / count float4s, strided by the lane count ("grid") or
// consecutive ("run"); with plain or non-temporal loads and stores.
#define PORCH_EW_STEP(L, S)                                                                  \
    {                                                                                      \
        const porch_v4f x = L(reinterpret_cast<const porch_v4f*>(a0) + i);                 \
        const porch_v4f y = L(reinterpret_cast<const porch_v4f*>(a1) + i);                 \
        const porch_v4f r = (porch_v4f){((x.x + y.x) * 2.0f) - 1.0f, ((x.y + y.y) * 2.0f) - 1.0f, \
                                        ((x.z + y.z) * 2.0f) - 1.0f, ((x.w + y.w) * 2.0f) - 1.0f}; \
        S(r, reinterpret_cast<porch_v4f*>(out) + i);                                       \
    }
#define PORCH_PLAIN_LOAD(p) (*(p))
#define PORCH_PLAIN_STORE(v, p) (*(p) = (v))
#define PORCH_NT_STORE(v, p) __builtin_nontemporal_store((v), (p))
#define PORCH_EW_GRID(name, L, S)                                                            \
    extern "C" __global__ void __launch_bounds__(256) name(                                \
        const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out, \
        unsigned long long count) {                                                        \
        for (unsigned i = blockIdx.x * 256u + threadIdx.x; i < 262144u; i += (unsigned)count) \
            PORCH_EW_STEP(L, S)                                                            \
    }
#define PORCH_EW_RUN(name, per_lane, L, S)                                                   \
    extern "C" __global__ void __launch_bounds__(256) name(                                \
        const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out, \
        unsigned long long count) {                                                        \
        const unsigned g = blockIdx.x * 256u + threadIdx.x;                                \
        _Pragma("unroll") for (unsigned j = 0; j < per_lane; ++j) {                        \
            const unsigned i = (g / 64u) * (64u * per_lane) + j * 64u + (g % 64u);          \
            PORCH_EW_STEP(L, S)                                                            \
        }                                                                                  \
    }
PORCH_EW_GRID(porch_ew_grid_nt_plain, __builtin_nontemporal_load, PORCH_PLAIN_STORE)
PORCH_EW_GRID(porch_ew_grid_plain_plain, PORCH_PLAIN_LOAD, PORCH_PLAIN_STORE)
PORCH_EW_GRID(porch_ew_grid_nt_nt, __builtin_nontemporal_load, PORCH_NT_STORE)
PORCH_EW_RUN(porch_ew_run2_nt_plain, 2u, __builtin_nontemporal_load, PORCH_PLAIN_STORE)
PORCH_EW_RUN(porch_ew_run4_nt_plain, 4u, __builtin_nontemporal_load, PORCH_PLAIN_STORE)
// A plain copy at a large size: `count` lanes, each copying four float4 of
// a0 to out, strided by the lane count (non-temporal loads and stores).
extern "C" __global__ void __launch_bounds__(256) porch_control_stream(
    const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out,
    unsigned long long count) {
    const unsigned long long g = blockIdx.x * 256ull + threadIdx.x;
    if (g >= count) return;
    const porch_v4f* x = reinterpret_cast<const porch_v4f*>(a0);
    porch_v4f* y = reinterpret_cast<porch_v4f*>(out);
    for (int r = 0; r < 4; ++r)
        __builtin_nontemporal_store(__builtin_nontemporal_load(x + g + r * count), y + g + r * count);
}
// The wide product's B [4096, 4096] (a0) read alone, 256 workgroups (count =
// 65536 lanes), nothing stored unless a lane's sum is 1234.5 (never, for the
// workload's inputs): "strips" reads it as the wide product's split kernel
// does (workgroup = 64 columns by a quarter of K; wave w, group g: rows
// k0 + 16 w + 64 g + 4 (lane / 16) + j, 256 B of each), two groups of four
// float4 a lane in flight; "blocks" reads workgroup b's contiguous 256 KB,
// sixteen float4 a lane in flight.
extern "C" __global__ void __launch_bounds__(256) porch_control_strips(
    const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out,
    unsigned long long count) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, lg = lane >> 4;
    const int c0 = (blockIdx.x / 4) * 64, k0 = (blockIdx.x % 4) * 1024;
    porch_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    porch_v4f b[2][4];
    for (int g = 0; g < 2; ++g)
        for (int j = 0; j < 4; ++j)
            b[g][j] = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(
                a0 + (unsigned long long)(k0 + 16 * w + 64 * g + 4 * lg + j) * 4096 + c0 + 4 * li));
#pragma unroll
    for (int g = 0; g < 16; ++g) {
        for (int j = 0; j < 4; ++j) acc += b[g & 1][j];
        if (g + 2 < 16)
            for (int j = 0; j < 4; ++j)
                b[g & 1][j] = __builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(
                    a0 + (unsigned long long)(k0 + 16 * w + 64 * (g + 2) + 4 * lg + j) * 4096 + c0 + 4 * li));
    }
    const float s = (acc.x + acc.y) + (acc.z + acc.w);
    if (s == 1234.5f) out[blockIdx.x * 256 + threadIdx.x] = s;
}
extern "C" __global__ void __launch_bounds__(256) porch_control_blocks(
    const float* __restrict__ a0, const float* __restrict__ a1, float* __restrict__ out,
    unsigned long long count) {
    const porch_v4f* x = reinterpret_cast<const porch_v4f*>(a0) + blockIdx.x * 16384ull;
    porch_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = threadIdx.x; i < 16384; i += 4096) {
        porch_v4f v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = __builtin_nontemporal_load(x + i + 256 * u);
#pragma unroll
        for (int u = 0; u < 16; ++u) acc += v[u];
    }
    const float s = (acc.x + acc.y) + (acc.z + acc.w);
    if (s == 1234.5f) out[blockIdx.x * 256 + threadIdx.x] = s;
}
"""


def controls(launches: int) -> int:
    """Each control kernel, then the elementwise workload's own kernel,
    `launches` times each over rotated (cache-cold) buffers; then the view
    chain's bytes moved in coalesced order and that workload itself; then
    a plain copy of the vocabulary softmax's bytes and that workload; then
    two read-only passes over the wide product's B and that workload,
    `launches` times each; timed by the profiler this runs under
    (rocprofv3 --kernel-trace --stats)."""
    import porch_amd as porch
    from porch_amd import _lib
    from porch_amd.workloads import config_graph, config_inputs, config_shapes

    if not porch.is_available():
        return 1
    n = 1 << 20
    copies = ROTATION["elementwise"]
    host = config_inputs("elementwise")
    sets = [[porch.tensor([n], v) for v in host] for _ in range(copies)]
    outs = [porch.zeros([n]).realize() for _ in range(copies)]
    code = ctypes.c_void_p()
    _lib.check(_lib.lib.porch_compile(CONTROL_SOURCE.encode(), None, 0, ctypes.byref(code)))
    data, size = _lib.lib.porch_code_object_data(code), _lib.lib.porch_code_object_size(code)
    for kernel in ("porch_control_empty", "porch_control_read", "porch_control_write", "porch_control_copy"):
        for i in range(launches):
            a, b = sets[i % copies]
            ins = (ctypes.c_void_p * 2)(a.device_data().handle, b.device_data().handle)
            _lib.check(_lib.lib.porch_launch_fused_elementwise(
                data, size, kernel.encode(), ins, 2, outs[i % copies].device_data().handle, n // 4))
        porch.synchronize()
        log(f"controls: {kernel} x {launches}")
    for i in range(launches):
        porch.materialize(config_graph("elementwise", sets[i % copies]))
    porch.synchronize()
    log(f"controls: elementwise workload x {launches}")
    # other launch shapes of the same arithmetic over the same buffers:
    # (kernel, lanes); the grid is lanes / 256 workgroups
    for kernel, lanes in (("porch_ew_grid_nt_plain", 262144), ("porch_ew_grid_nt_plain", 131072),
                          ("porch_ew_grid_nt_plain", 65536), ("porch_ew_grid_nt_plain", 32768),
                          ("porch_ew_grid_plain_plain", 262144), ("porch_ew_grid_nt_nt", 262144),
                          ("porch_ew_run2_nt_plain", 131072), ("porch_ew_run4_nt_plain", 65536)):
        for i in range(launches):
            a, b = sets[i % copies]
            ins = (ctypes.c_void_p * 2)(a.device_data().handle, b.device_data().handle)
            _lib.check(_lib.lib.porch_launch_fused_elementwise(
                data, size, kernel.encode(), ins, 2, outs[i % copies].device_data().handle, lanes))
        porch.synchronize()
        log(f"controls: {kernel} at {lanes // 256} workgroups x {launches}")
    for i, (a, b) in enumerate(sets[:2]):
        # the variants' values are the workload's bits (read from the device
        # buffer: the kernels wrote it behind the tensor's host copy)
        got = outs[i].device_data().download(n)
        want = ((a.cpu() + b.cpu()) * np.float32(2.0) - np.float32(1.0)).astype(np.float32)
        if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
            raise AssertionError("controls: an elementwise variant differs from the workload's arithmetic")
    del sets, outs

    # The view chain beside a coalesced kernel that moves the same bytes
    # (all of x read, half as many written), both over rotated buffers.
    vc_shape = config_shapes("view_chain")[0]
    (vc_values,) = config_inputs("view_chain")
    copies = ROTATION["view_chain"]
    xs = [porch.tensor(vc_shape, vc_values) for _ in range(copies)]
    halves = [porch.zeros([vc_shape[0] * vc_shape[1] // 2]).realize() for _ in range(copies)]
    lanes = vc_shape[0] * vc_shape[1] // 128  # 32 float4 per lane
    for i in range(launches):
        h = xs[i % copies].device_data().handle
        ins = (ctypes.c_void_p * 2)(h, h)
        _lib.check(_lib.lib.porch_launch_fused_elementwise(
            data, size, b"porch_control_half", ins, 2, halves[i % copies].device_data().handle, lanes))
    porch.synchronize()
    log(f"controls: porch_control_half x {launches}")
    for i in range(launches):
        porch.materialize(config_graph("view_chain", [xs[i % copies]]))
    porch.synchronize()
    log(f"controls: view_chain workload x {launches}")
    del xs, halves

    # The vocabulary softmax beside a plain copy of the same bytes (512 MiB
    # each way: twice the Infinity Cache, so no launch finds its data there).
    shape = config_shapes("vocab_softmax")[0]
    total = shape[0] * shape[1]
    (values,) = config_inputs("vocab_softmax")
    x = porch.tensor(shape, values)
    y = porch.zeros([total]).realize()
    ins = (ctypes.c_void_p * 2)(x.device_data().handle, x.device_data().handle)
    for _ in range(launches):
        _lib.check(_lib.lib.porch_launch_fused_elementwise(
            data, size, b"porch_control_stream", ins, 2, y.device_data().handle, total // 16))
    porch.synchronize()
    log(f"controls: porch_control_stream x {launches}")
    for _ in range(launches):
        porch.materialize(config_graph("vocab_softmax", [x]))
    porch.synchronize()
    log(f"controls: vocab_softmax workload x {launches}")
    del x, y

    # The wide product beside kernels that only read its B, over rotated B
    # copies: its split kernel reads B at the wide product's geometry.
    a_shape, b_shape = config_shapes("wide_product")
    a_values, b_values = config_inputs("wide_product")
    copies = ROTATION["wide_product"]
    a = porch.tensor(a_shape, a_values)
    bs = [porch.tensor(b_shape, b_values) for _ in range(copies)]
    sink = porch.zeros([65536]).realize()
    for kernel in (b"porch_control_strips", b"porch_control_blocks"):
        for i in range(launches):
            h = bs[i % copies].device_data().handle
            ins = (ctypes.c_void_p * 2)(h, h)
            _lib.check(_lib.lib.porch_launch_fused_elementwise(
                data, size, kernel, ins, 2, sink.device_data().handle, 65536))
        porch.synchronize()
        log(f"controls: {kernel.decode()} x {launches}")
    for i in range(launches):
        porch.materialize(config_graph("wide_product", [a, bs[i % copies]]))
    porch.synchronize()
    log(f"controls: wide_product workload x {launches}")
    _lib.lib.porch_code_object_release(code)
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--configs", default="elementwise,view_chain,softmax,logistic_rowsum,matmul_epilogue,"
                                             "batched_transpose,heads_permute,batched_matmul,attention_scores,"
                                             "vocab_softmax,narrow_product,wide_product")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--jit-probe", default=None, help=argparse.SUPPRESS)
    parser.add_argument("--controls", type=int, default=0, metavar="LAUNCHES",
                        help="launch the control kernels beside their workloads (for rocprofv3) and exit")
    args = parser.parse_args()
    if args.jit_probe:
        return jit_probe(args.jit_probe)
    if args.controls:
        return controls(args.controls)
    if args.gpus != 1:
        print("bench.py measures one GPU: porch's fused-graph path runs every graph on "
              "one device and has no multi-GPU execution; run with --gpus 1.",
              file=sys.stderr)
        return 2

    import porch_amd as porch
    from porch_amd import synth

    if not porch.is_available():
        print("porch_amd: the HIP backend is not available", file=sys.stderr)
        return 1
    info = synth.device_info()
    log(f"device: {info}")
    workload_names = [c for c in args.configs.split(",") if c]
    results = {}
    for name in workload_names:
        steps, warmup = args.steps, args.warmup
        log(f"{name}: {DESCRIPTION[name]} ({steps} steps)")
        results[name] = run_config(porch, name, steps, warmup)
        r = results[name]
        log(f"{name}: {r['value']:.1f} {r['unit']} whole-job, kernel {r['kernel_ms_mean']*1e3:.1f} us, "
            f"roofline {r['roofline']['frac']*100:.1f}%, JIT cold {r['jit_ms']['cold']:.1f} ms "
            f"disk {r['jit_ms']['disk'] if r['jit_ms']['disk'] is None else round(r['jit_ms']['disk'], 2)} ms "
            f"hit {r['jit_ms']['hit']*1e3:.1f} us")
        if not args.no_cpu:
            # 10 s of CPU work for the headline workload, 4 s for the others
            results[name]["cpu_baseline"] = cpu_baseline(name, 10.0 if name == "view_chain" else 4.0)
            log(f"{name}: cpu {results[name]['cpu_baseline']['value']:.2f} "
                f"{results[name]['cpu_baseline']['unit']} on {results[name]['cpu_baseline']['cores']} threads")

    head = "view_chain" if "view_chain" in results else workload_names[0]
    h = results[head]
    line = {
        "metric": METRIC,
        "value": h["value"],
        "unit": h["unit"],
        "n_gpus": 1,
        "steps": h["steps"],
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (splitmix64 seeded inputs resident in HBM)",
        "config": {"workload": f"{head}: {h['workload']}", "parallelism": "single GPU",
                   "device": info["arch"], "compute_units": info["compute_units"]},
        "roofline": h["roofline"],
        "cpu_baseline": h.get("cpu_baseline"),
        "jit_ms": h["jit_ms"],
        "configs": results,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
