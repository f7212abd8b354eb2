"""Every access of the generated kernels stays inside its buffers, checked
on the CPU: each kernel of a plan is compiled as host C++ and run over its
whole grid with its buffers, sized exactly as on the device, placed against
inaccessible guard regions (tests/kernel_emu).  An out-of-bounds read or
write faults the emulation process instead of a GPU.

Covers the benchmark graphs at small sizes, the tiled, permute, batched and
strided cases of the other tests, the persistent short-K products (on a
subset of their workgroups), seeded random graphs (views, concat,
reductions, products, strided leaves), and a regression: a transposed leaf
in one branch of a concat is staged by the LDS-transpose kernel ahead of the
select, and must be loaded only where the select takes its branch.
"""

import re
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import porch_amd as porch
from tests.helpers import config_graph, config_shapes, placeholder, strided_placeholder
from tests.kernel_emu import emulate as emu
from tests.test_batched_matmul import PERSISTENT
from tests.test_gpu_fuzz import random_graph, random_product
from tests.test_permute import CASES as PERMUTE_CASES
from tests.test_tiled import CASES as TILED_CASES, build_case

pytestmark = pytest.mark.skipif(not emu.available(), reason="host clang++ from ROCm is required")


def in_bounds(expr):
    results = emu.emulate(expr)
    assert all(r["ok"] for r in results), results
    return results


def test_emulation_catches_an_out_of_bounds_read():
    # a planted mistake: one element before the start of a0
    source = ('extern "C" __global__ void __launch_bounds__(256) k(const float* __restrict__ a0, '
              'float* __restrict__ out) { out[threadIdx.x] = a0[(int)threadIdx.x - 1]; }')
    ok, detail = emu.run_kernel(source, "k", [256, 256], (1, 1, 1))
    assert not ok and "placement 0" in detail
    fixed = source.replace("(int)threadIdx.x - 1", "threadIdx.x")
    assert emu.run_kernel(fixed, "k", [256, 256], (1, 1, 1)) == (True, "")


def test_emulation_catches_a_read_past_the_end():
    source = ('extern "C" __global__ void __launch_bounds__(256) k(const float* __restrict__ a0, '
              'float* __restrict__ out) { out[threadIdx.x] = a0[threadIdx.x + 8]; }')
    ok, detail = emu.run_kernel(source, "k", [256, 256], (1, 1, 1))
    assert not ok and "placement 1" in detail


def test_staged_leaf_under_a_concat_branch_is_guarded():
    n = 300
    x1 = placeholder([n, 4], np.zeros(n * 4, np.float32))
    x2 = placeholder([4, n], np.zeros(4 * n, np.float32))
    expr = porch.concat(x1, porch.transpose(x2), 1) + 1.0
    assert [k["kind"] for k in porch.plan(expr)["kernels"]] == ["pointwise.tiled"]
    phase1 = porch.kernel_source(expr).split("__syncthreads();")[0]
    assert "if (!((q1) < 4)) {" in phase1
    in_bounds(expr)


@pytest.mark.parametrize("name, size", [
    ("elementwise", {"n": 1000}),
    ("view_chain", {"n": 130}),
    ("softmax", {"rows": 7, "cols": 2100}),
    ("softmax", {"rows": 33, "cols": 100}),
    ("softmax", {"rows": 1001, "cols": 3}),
    ("softmax", {"rows": 77, "cols": 32}),
    ("logistic_rowsum", {"rows": 999, "cols": 1}),
    ("logistic_rowsum", {"rows": 35, "cols": 40}),
    ("softmax", {"rows": 3, "cols": 65536}),
    ("softmax", {"rows": 2, "cols": 262148}),  # beyond the register cache: one online pass
    ("logistic_rowsum", {"rows": 9, "cols": 2052}),
    ("matmul_epilogue", {"m": 200, "k": 70, "n": 136}),
])
def test_benchmark_graphs(name, size):
    tensors = [placeholder(s) for s in config_shapes(name, size)]
    in_bounds(config_graph(name, tensors, size))


@pytest.mark.parametrize("widths", [(64, 128), (8, 12), (4, 4)])
def test_concat_along_the_last_axis_values(widths):
    # the flat kernel with one branch per group of 4: every access in
    # bounds and the values the oracle gives, on rows whose split falls at
    # a multiple of 4
    from oracle import host
    a, b = widths
    rng = np.random.default_rng(a * 100 + b)
    xa = rng.standard_normal(37 * a).astype(np.float32)
    xb = rng.standard_normal(37 * b).astype(np.float32)
    expr = porch.concat(placeholder([37, a], xa), placeholder([37, b], xb), 1) * 2.0
    assert [k["kind"] for k in porch.plan(expr)["kernels"]] == ["pointwise.flat"]
    in_bounds(expr)
    got = emu.evaluate(expr, [xa, xb])
    want = host.evaluate(expr)
    assert np.array_equal(got.reshape(-1).view(np.uint32), want.reshape(-1).view(np.uint32))


def test_tiled_and_permute_cases():
    exprs = [build_case(name, placeholder) for name in sorted(TILED_CASES) if name != "transpose_3000x4100"]
    exprs += [fn(placeholder) for fn, _ in PERMUTE_CASES.values()]
    with ThreadPoolExecutor(6) as pool:
        for results in pool.map(emu.emulate, exprs):
            assert all(r["ok"] for r in results), results


def test_persistent_products_on_a_subset_of_workgroups():
    # each persistent workgroup walks several tiles; the first and last
    # workgroups (by index) reach the first tiles and the ragged last ones
    # through the XCD mapping, and the loop's hand-over between tiles
    exprs = [build(placeholder) for build in PERSISTENT]
    for expr in exprs:
        assert porch.plan(expr)["kernels"][-1]["grid"][0] == 512
    with ThreadPoolExecutor(5) as pool:
        for i, results in enumerate(pool.map(lambda e: emu.emulate(e, only=[0, 1, 7, 256, 505, 510, 511]), exprs)):
            assert all(r["ok"] for r in results), (i, results)


def test_subset_emulation_catches_a_planted_overrun():
    # the last tile's prefetch of "the next tile" without its clamp reads
    # past the operands, in the last workgroup only
    expr = porch.tensor_expr(PERSISTENT[0](placeholder))
    plan = porch.plan(expr)
    kernel = plan["kernels"][0]
    source = porch.kernel_source(expr, 0)
    planted = re.sub(r"const idx_t rn = rr \+ gridDim\.x < \d+ \? rr \+ gridDim\.x : rr;",
                     "const idx_t rn = rr + gridDim.x;", source)
    assert planted != source
    _, _, _, inputs, _ = porch.serialize(expr._root)
    sizes = [int(np.prod(t.shape())) for t in inputs] + [int(np.prod(plan["out_shape"]))]
    ok, _ = emu.run_kernel(planted, kernel["name"], sizes, kernel["grid"], kernel["block"], only=[511])
    assert not ok
    ok, detail = emu.run_kernel(source, kernel["name"], sizes, kernel["grid"], kernel["block"], only=[511])
    assert ok, detail


def strided_or_dense(shape, rng):
    n = int(np.prod(shape))
    if n and rng.integers(0, 4) == 0:
        strides = [int(s) for s in rng.integers(0, 5, size=len(shape))]
        offset = int(rng.integers(0, 7))
        span = offset + sum((e - 1) * s for e, s in zip(shape, strides)) + 1
        return strided_placeholder(porch.tensor_layout(list(shape), strides, offset), np.zeros(span, np.float32))
    return placeholder(list(shape), np.zeros(n, np.float32))


def test_random_graphs():
    rng = np.random.default_rng(20261203)
    exprs = []
    while len(exprs) < 40:
        expr = random_graph(rng, strided_or_dense) if len(exprs) % 4 else random_product(rng, strided_or_dense)
        exprs.append(expr)
    with ThreadPoolExecutor(6) as pool:
        for i, results in enumerate(pool.map(emu.emulate, exprs)):
            assert all(r["ok"] for r in results), (i, results)
