"""Tensors past 2^31 elements: every kernel class switches to 64-bit index
arithmetic when a tensor it touches holds 2^30 elements or more.

The CPU tests pin that switch in the generated source.  The GPU tests run
each kernel class on tensors of 2^31 + 2^16 elements (8 GiB of fp32) built
on the device, and check the results against closed forms computed on the
host: small-integer data keeps every sum exact in any order, and the data
at index i and at i - 2^31 differ, so a 32-bit index that wraps reads a
wrong value and fails the check.
"""

import numpy as np
import pytest

import porch_amd as porch
from tests.helpers import placeholder

R, C = (1 << 15) + 1, 1 << 16          # R * C = 2^31 + 2^16 elements


def wide_kernels(expr):
    plan = porch.plan(expr, compile=True)
    return [(k["kind"], porch.kernel_source(expr, i)) for i, k in enumerate(plan["kernels"])]


@pytest.mark.parametrize("build", [
    lambda x: x * 2.0 + 1.0,
    lambda x: porch.transpose(x) + 1.0,
    lambda x: porch.sum(x, 1),
    lambda x: porch.sum(x, 0),
    lambda x: porch.softmax(x, 1),
])
def test_large_tensors_use_64_bit_indices(build):
    for kind, source in wide_kernels(build(placeholder([R, C]))):
        assert "typedef long long idx_t;" in source, kind


def test_small_tensors_keep_32_bit_indices():
    (kind, source), = wide_kernels(placeholder([1024, 1024]) * 2.0)
    assert "typedef int idx_t;" in source


def test_large_product_operand_uses_64_bit_indices():
    expr = porch.matmul(placeholder([C, R]), placeholder([R, 64]))
    for kind, source in wide_kernels(expr):
        assert "typedef long long idx_t;" in source, kind


def test_large_band_product_uses_64_bit_indices():
    # [33, 8192, 8] @ [33, 8, 8192]: 33 x 8192^2 = 2^31 + 2^26 outputs
    expr = porch.batched_matmul(placeholder([33, 8192, 8]), placeholder([33, 8, 8192]))
    (kind, source), = wide_kernels(expr)
    assert kind == "gemm.band"
    assert "typedef long long idx_t;" in source


def device_data(gpu, rows, cols):
    """x[i, j] = (i % 7) + (j % 5), made on the device from two small
    vectors (a broadcast sum, materialised)."""
    a = gpu.tensor([rows, 1], (np.arange(rows) % 7).astype(np.float32))
    b = gpu.tensor([1, cols], (np.arange(cols) % 5).astype(np.float32))
    return gpu.materialize(gpu.broadcast_to(a, [rows, cols]) + gpu.broadcast_to(b, [rows, cols]))


def expected_rows(lo, hi, cols):
    """Rows lo..hi-1 of the device data, as computed on the host."""
    return (np.arange(lo, hi, dtype=np.float32) % 7)[:, None] + (np.arange(cols, dtype=np.float32) % 5)[None, :]


def check_blocks(got, rows, cols, expect, block=2048):
    """got [rows, cols] against expect(lo, hi) block by block (bounded host memory)."""
    for lo in range(0, rows, block):
        hi = min(rows, lo + block)
        assert np.array_equal(got[lo:hi], expect(lo, hi)), (lo, hi)


@pytest.mark.gpu
def test_wide_pointwise_and_transpose(gpu):
    x = device_data(gpu, R, C)
    print("wide: flat", flush=True)
    y = gpu.materialize(x * 2.0 + 1.0).cpu().reshape(R, C)
    check_blocks(y, R, C, lambda lo, hi: expected_rows(lo, hi, C) * 2 + 1)
    del y
    print("wide: tiled transpose", flush=True)
    t = gpu.materialize(gpu.transpose(x) - 1.0).cpu().reshape(C, R)
    # t[j, i] = x[i, j] - 1 = (i % 7) + (j % 5) - 1
    check_blocks(t, C, R, lambda lo, hi: (np.arange(lo, hi, dtype=np.float32) % 5)[:, None]
                 + (np.arange(R, dtype=np.float32) % 7)[None, :] - 1, block=4096)


@pytest.mark.gpu
def test_wide_reductions(gpu):
    x = device_data(gpu, R, C)
    i = np.arange(R)
    j = np.arange(C)
    print("wide: row sums", flush=True)
    rows = gpu.materialize(gpu.sum(x, 1)).cpu()
    assert np.array_equal(rows, (C * (i % 7) + (j % 5).sum()).astype(np.float32))
    print("wide: column sums", flush=True)
    cols = gpu.materialize(gpu.sum(x, 0)).cpu()
    assert np.array_equal(cols, ((i % 7).sum() + R * (j % 5)).astype(np.float32))
    print("wide: row max with broadcast", flush=True)
    shifted = gpu.materialize(x - gpu.broadcast_to(gpu.max(x, 1, True), [R, C])).cpu().reshape(R, C)
    # every row's max is (i % 7) + 4
    check_blocks(shifted, R, C, lambda lo, hi: np.broadcast_to((j % 5 - 4).astype(np.float32), (hi - lo, C)))


@pytest.mark.gpu
def test_wide_matmul_operand(gpu):
    # A [65536, 32769] holds 2^31 + 2^16 elements; products of small
    # integers sum exactly (below 2^24) in any order
    a = device_data(gpu, C, R)
    b_host = (np.arange(R * 64) % 3).astype(np.float32)
    b = gpu.tensor([R, 64], b_host)
    print("wide: matmul", flush=True)
    out = gpu.materialize(gpu.matmul(a, b)).cpu().reshape(C, 64)
    rows = [0, 1, 2, 12345, 32767, 32768, 40000, C - 1]
    a_rows = np.concatenate([expected_rows(r, r + 1, R) for r in rows]).astype(np.float64)
    assert np.array_equal(out[rows], (a_rows @ b_host.reshape(R, 64).astype(np.float64)).astype(np.float32))


@pytest.mark.gpu
def test_wide_band_product(gpu):
    # 33 entries of [8192, 8] @ [8, 8192]: entry 32 starts at output 2^31;
    # small integers sum exactly in any order
    nb, n, k = 33, 8192, 8
    bi, ii, kk = np.meshgrid(np.arange(nb), np.arange(n), np.arange(k), indexing="ij")
    a_host = ((bi + ii + kk) % 5).astype(np.float32)
    bb, kb, jb = np.meshgrid(np.arange(nb), np.arange(k), np.arange(n), indexing="ij")
    b_host = ((3 * bb + kb + jb) % 7).astype(np.float32)
    a = gpu.tensor([nb, n, k], a_host.reshape(-1))
    b = gpu.tensor([nb, k, n], b_host.reshape(-1))
    expr = gpu.batched_matmul(a, b) - 1.0
    assert [x["kind"] for x in gpu.plan(expr)["kernels"]] == ["gemm.band"]
    print("wide: band product", flush=True)
    out = gpu.materialize(expr).cpu().reshape(nb, n, n)
    for e in (0, 31, 32):
        for r in (0, 1, 4097, n - 1):
            want = a_host[e, r].astype(np.float64) @ b_host[e].astype(np.float64) - 1.0
            assert np.array_equal(out[e, r], want.astype(np.float32)), (e, r)

