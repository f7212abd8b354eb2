"""Realised tensors over strided storage: tensor(layout, storage) (an
extension; the reference rejects non-contiguous storage,
src/tensor.cpp:1193-1197).

A strided tensor enters a graph as its raw storage (the flat span its layout
reaches) read through a slice node, so every kernel class reads it in place.
The oracle is pinned against numpy's as_strided view of the same storage
(transposed, offset, zero-stride and overlapping layouts); the GPU tests check
expressions over strided tensors bit-exact against the oracle and data()'s
gather against numpy.
"""

import numpy as np
import pytest
from numpy.lib.stride_tricks import as_strided

import porch_amd as porch
from oracle import host
from tests.helpers import placeholder, strided_placeholder

# (shape, strides, offset) over a storage of STORAGE floats
STORAGE = 600
LAYOUTS = [
    ([12, 10], [1, 12], 0),        # a transposed [10, 12] matrix
    ([5, 7], [20, 2], 13),         # offset, every other column
    ([4, 6], [0, 3], 5),           # a broadcast row (zero stride)
    ([6, 4], [1, 1], 2),           # overlapping sliding windows
    ([3, 1, 5], [100, 7, 1], 40),  # a size-1 dimension with its own stride
    ([2, 3, 4], [1, 2, 6], 0),     # fully permuted strides
]


def storage_values(seed=0):
    rng = np.random.default_rng(seed)
    return (rng.integers(-512, 512, size=STORAGE).astype(np.float32) / np.float32(8))


def numpy_view(values, shape, strides, offset):
    return as_strided(values[offset:], shape=shape, strides=[4 * s for s in strides]).copy()


@pytest.mark.parametrize("shape, strides, offset", LAYOUTS)
def test_oracle_reads_strided_storage_like_numpy(shape, strides, offset):
    v = storage_values()
    t = strided_placeholder(porch.tensor_layout(shape, strides, offset), v)
    assert not t.is_contiguous()
    assert t.strides() == tuple(strides) and t.storage_offset() == offset
    expected = numpy_view(v, shape, strides, offset)
    assert np.array_equal(host.evaluate(porch.tensor_expr(t)), expected)
    assert np.array_equal(host.evaluate(t * 2.0 + 1.0), expected * 2 + 1)


def test_slicing_a_strided_tensor_composes_with_its_layout():
    v = storage_values(1)
    shape, strides, offset = [12, 10], [1, 12], 3
    t = strided_placeholder(porch.tensor_layout(shape, strides, offset), v)
    view = numpy_view(v, shape, strides, offset)
    cases = [
        (t[porch.slice(1, 12, 2), porch.all], view[1:12:2, :]),
        (t[4], view[4]),
        (t[porch.slice(-5, 100), porch.slice(2, 9, 3)], view[-5:, 2:9:3]),
    ]
    for expr, expected in cases:
        assert np.array_equal(host.evaluate(expr), expected)


def test_node_table_holds_the_storage_span_and_a_slice():
    layout = porch.tensor_layout([5, 7], [20, 2], 13)
    t = strided_placeholder(layout, storage_values())
    nodes, dims, _, inputs, _ = porch.serialize(porch.tensor_expr(t))
    assert [nodes[i].op for i in range(len(nodes))] == [porch._lib.OP["input"], porch._lib.OP["slice"]]
    assert layout.span() == 13 + 4 * 20 + 6 * 2 + 1
    assert dims[nodes[0].dims] == layout.span()
    assert len(inputs) == 1


@pytest.mark.parametrize("shape, strides, offset, message", [
    ([2, 3], [1], 0, "tensor layout rank mismatch"),
    ([2, 3], [3, 1], -1, "tensor layout offset must be non-negative"),
    ([2, 3], [3, -1], 0, "tensor layout strides must be non-negative"),
])
def test_layout_validation_uses_reference_messages(shape, strides, offset, message):
    with pytest.raises(porch.InvalidArgument, match=message):
        porch.tensor_layout(shape, strides, offset)


def test_storage_must_cover_the_layout():
    with pytest.raises(porch.InvalidArgument, match="tensor device storage is too small"):
        porch.tensor(porch.tensor_layout([4, 4], [1, 4], 0), porch._Buffer.empty())


def test_kernels_read_strided_storage_in_place():
    # a transposed layout: the tiled (LDS transpose) kernel, no copy first
    t = strided_placeholder(porch.tensor_layout([64, 48], [1, 64], 0), np.zeros(64 * 48, np.float32))
    kinds = [k["kind"] for k in porch.plan(t * 2.0 + porch.tensor_expr(placeholder([64, 48])))["kernels"]]
    assert kinds == ["pointwise.tiled"]
    # a transposed operand of a product: read in place by the gemm
    a = strided_placeholder(porch.tensor_layout([96, 64], [1, 96], 0), np.zeros(96 * 64, np.float32))
    kinds = [k["kind"] for k in porch.plan(porch.matmul(a, placeholder([64, 80])))["kernels"]]
    assert kinds == ["gemm.mfma"]


@pytest.mark.gpu
def test_strided_tensors_on_the_gpu(gpu):
    v = storage_values(2)
    base = gpu.tensor([STORAGE], v)
    storage = base.device_data()
    for shape, strides, offset in LAYOUTS:
        print("strided layout", shape, strides, offset, flush=True)
        t = gpu.tensor(gpu.tensor_layout(shape, strides, offset), storage)
        expected = numpy_view(v, shape, strides, offset)
        # data() gathers in row-major order
        assert np.array_equal(t.cpu().reshape(shape), expected)
        # (sums of multiples of 1/8 are exact in any order)
        for expr, exact in ((t * 2.0 + 1.0, True), (gpu.sum(t, len(shape) - 1), True),
                            (gpu.exp(t * 0.125) - t, False)):
            ref = host.evaluate(expr)
            out = gpu.materialize(expr).cpu().reshape(ref.shape)
            if exact:
                assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
            else:  # exp within a few ulp of the oracle's std::exp
                np.testing.assert_allclose(out, ref, rtol=2e-6, atol=1e-6)


@pytest.mark.gpu
def test_strided_operands_bit_exact(gpu):
    rng = np.random.default_rng(3)
    # a [256, 192] matrix stored transposed, inside a larger buffer at an offset
    rows, cols, pad = 256, 192, 37
    storage_host = rng.integers(-3, 4, size=pad + rows * cols + 11).astype(np.float32)
    storage = gpu.tensor([storage_host.size], storage_host).device_data()
    at = gpu.tensor(gpu.tensor_layout([rows, cols], [1, rows], pad), storage)
    b = gpu.tensor([cols, 160], rng.integers(-3, 4, size=cols * 160).astype(np.float32))
    dense = numpy_view(storage_host, [rows, cols], [1, rows], pad)
    cases = [
        at + 1.0,                                         # tiled transpose
        gpu.matmul(at, b),                                # gemm operand in place
        gpu.relu(gpu.matmul(at, b) - 2.0),                # with an epilogue
        gpu.sum(at, 0),                                   # column reduction
        at[gpu.slice(1, rows, 3), gpu.slice(0, cols, 2)] * 2.0,  # sliced view
    ]
    for i, expr in enumerate(cases):
        print("strided case", i, flush=True)
        ref = host.evaluate(expr)
        out = gpu.materialize(expr).cpu().reshape(ref.shape)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), i
    assert np.array_equal(gpu.materialize(gpu.matmul(at, b)).cpu().reshape(rows, 160),
                          (dense.astype(np.float64) @ b.cpu().reshape(cols, 160)).astype(np.float32))


@pytest.mark.gpu
def test_empty_strided_tensor(gpu):
    storage = gpu.tensor([8], np.arange(8, dtype=np.float32)).device_data()
    t = gpu.tensor(gpu.tensor_layout([4, 0], [2, 1], 3), storage)
    assert t.numel() == 0 and t.cpu().size == 0
    assert gpu.materialize(t + 1.0).cpu().size == 0
