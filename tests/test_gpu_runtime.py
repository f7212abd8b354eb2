"""Runtime behaviour on the GPU: JIT cache hits, raw launches with the
reference's geometry, buffers, and compile errors."""

import ctypes
import re

import numpy as np
import pytest

from porch_amd import _lib

pytestmark = pytest.mark.gpu


def test_graph_cache_hits_on_structurally_equal_graphs(gpu):
    porch = gpu
    a = porch.tensor([1000], np.ones(1000, dtype=np.float32))
    b = porch.tensor([1000], np.full(1000, 2.0, dtype=np.float32))
    porch.materialize((a + b) * 3.0).cpu()
    before = porch.jit_stats()
    c = porch.tensor([1000], np.full(1000, 5.0, dtype=np.float32))
    d = porch.tensor([1000], np.full(1000, 7.0, dtype=np.float32))
    out = porch.materialize((c + d) * 3.0).cpu()
    after = porch.jit_stats()
    assert (out == 36.0).all()
    assert after["plan_hits"] == before["plan_hits"] + 1
    assert after["compiles"] == before["compiles"]
    # a different scalar is a different kernel
    porch.materialize((c + d) * 4.0).cpu()
    assert porch.jit_stats()["plan_misses"] == after["plan_misses"] + 1


def test_raw_launch_with_reference_geometry(gpu):
    porch = gpu
    src = b"""
    typedef unsigned long long u64;
    extern "C" __global__ void axpy(const float* x, const float* y, float* out, u64 count) {
        const u64 i = blockIdx.x * 256ull + threadIdx.x;
        if (i < count) out[i] = 2.0f * x[i] + y[i];
    }
    extern "C" __global__ void rowsum(const float* x, float* out, u64 count) {
        __shared__ float s[256];
        float t = 0.0f;
        for (int k = threadIdx.x; k < 300; k += 256) t += x[blockIdx.x * 300 + k];
        s[threadIdx.x] = t;
        __syncthreads();
        for (int st = 128; st > 0; st /= 2) {
            if (threadIdx.x < st) s[threadIdx.x] += s[threadIdx.x + st];
            __syncthreads();
        }
        if (threadIdx.x == 0) out[blockIdx.x] = s[0];
    }
    """
    code = ctypes.c_void_p()
    _lib.check(_lib.lib.porch_compile(src, None, 0, ctypes.byref(code)))
    size = _lib.lib.porch_code_object_size(code)
    data = _lib.lib.porch_code_object_data(code)
    n = 1000
    x = porch._Buffer.upload(np.arange(n, dtype=np.float32))
    y = porch._Buffer.upload(np.ones(n, dtype=np.float32))
    out = porch._Buffer.upload(np.zeros(n, dtype=np.float32))
    ins = (ctypes.c_void_p * 2)(x.handle, y.handle)
    _lib.check(_lib.lib.porch_launch_fused_elementwise(data, size, b"axpy", ins, 2, out.handle, n))
    assert np.array_equal(out.download(n), 2.0 * np.arange(n, dtype=np.float32) + 1.0)
    rows = porch._Buffer.upload(np.ones(3 * 300, dtype=np.float32))
    sums = porch._Buffer.upload(np.zeros(3, dtype=np.float32))
    ins = (ctypes.c_void_p * 1)(rows.handle)
    _lib.check(_lib.lib.porch_launch_fused_reduction(data, size, b"rowsum", ins, 1, sums.handle, 3))
    assert sums.download(3).tolist() == [300.0, 300.0, 300.0]
    # the reference's validation: empty input, small output
    empty = porch._Buffer.empty()
    ins = (ctypes.c_void_p * 1)(empty.handle)
    rc = _lib.lib.porch_launch_fused_elementwise(data, size, b"axpy", ins, 1, out.handle, n)
    assert rc == _lib.ERR_INVALID_ARGUMENT
    _lib.lib.porch_code_object_release(code)


def test_undersized_input_buffer_is_rejected(gpu):
    porch = gpu
    import porch_amd
    nodes, dims, n_dims, inputs, _ = porch_amd.serialize(porch.tensor([8], np.ones(8)) + 1.0)
    g = porch_amd._graph(nodes, dims, n_dims)
    small = porch._Buffer.upload(np.ones(4, dtype=np.float32))
    handles = (ctypes.c_void_p * 1)(small.handle)
    out = ctypes.c_void_p()
    rc = _lib.lib.porch_materialize(ctypes.byref(g), handles, 1, ctypes.byref(out), None, 0, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT
    assert "too small" in _lib.lib.porch_last_error().decode()


def test_device_info(gpu):
    from porch_amd import synth
    info = synth.device_info()
    assert info["compute_units"] > 0 and info["arch"].startswith("gfx9")


def test_events_time_the_stream(gpu):
    porch = gpu
    from porch_amd import synth
    x = porch.tensor([1 << 22], np.ones(1 << 22, dtype=np.float32))
    start, stop = synth.Event(), synth.Event()
    start.record()
    y = porch.materialize(x * 2.0)
    stop.record()
    stop.synchronize()
    assert 0.0 < start.elapsed_ms(stop) < 1000.0
    assert y.cpu()[0] == 2.0


@pytest.mark.gpu
def test_staged_uploads_round_trip(gpu):
    """Uploads return before their DMA ends (pinned staging chunks, 32 MiB
    pieces): every buffer must still hold exactly what was uploaded, also
    when chunks are reused while earlier DMAs are pending and the source
    array is overwritten right after the call returns."""
    rng = np.random.default_rng(12)
    sizes = [1, 3, 1 << 18, (1 << 20) + 7, (9 << 20) + 5, 40 << 20, 100 << 20]
    expected, buffers = [], []
    source = np.empty(max(sizes), np.float32)
    for n in sizes * 2:
        values = rng.standard_normal(n).astype(np.float32)
        source[:n] = values
        buffers.append(gpu._Buffer.upload(source[:n]))
        source[:n] = -1.0  # the caller may reuse its memory at once
        expected.append(values)
    for buf, values in zip(buffers, expected):
        got = buf.download(values.size)
        assert np.array_equal(got.view(np.uint32), values.view(np.uint32)), values.size


@pytest.mark.gpu
def test_staged_uploads_from_several_threads(gpu):
    import threading

    results = {}

    def worker(k):
        values = np.full((12 << 20) + k, float(k), np.float32)
        buf = gpu._Buffer.upload(values)
        t = gpu.tensor._realized([values.size], buf, None, gpu.device())
        results[k] = gpu.materialize(t * 2.0).cpu()

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(6)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for k in range(6):
        assert results[k].size == (12 << 20) + k
        assert np.all(results[k] == 2.0 * k)


@pytest.mark.gpu
def test_realised_lazy_tensor_is_read_not_recomputed(gpu):
    """A pending tensor is inlined into later expressions; once realised, its
    buffer is read instead (the reference re-inlines its expression at every
    use, src/tensor.cpp:1323-1325)."""
    x = gpu.tensor([512, 512], np.arange(512 * 512, dtype=np.float32))
    pending = gpu.tensor(gpu.exp(x * 1e-6) + 1.0)
    def body(expr):  # the kernel itself, without the shared helper definitions
        source = gpu.kernel_source(expr)
        return source[source.index('extern "C"'):]

    inlined = gpu.plan(pending * 2.0)
    computes_exp = re.compile(r"\bexpf\(|porch_exp")
    assert computes_exp.search(body(pending * 2.0))  # the exp is recomputed in the consumer
    pending.realize()
    assert not computes_exp.search(body(pending * 2.0))  # the consumer reads the buffer
    nodes, _, _, inputs, _ = gpu.serialize((pending * 2.0)._root)
    assert len(inputs) == 1 and inputs[0] is pending
    assert len(inlined["kernels"]) == 1
    out = gpu.materialize(pending * 2.0).cpu()
    assert np.array_equal(out.view(np.uint32), (pending.cpu() * np.float32(2)).view(np.uint32))
