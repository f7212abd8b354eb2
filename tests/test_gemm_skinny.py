"""Matmuls with one short side (kernel kinds gemm.rows, gemm.combine,
gemm.cols, gemm.narrow, gemm.narrow_rows, gemm.wide): a few rows (a vector
times a matrix, a small batch of rows; 8 to 64 rows over 256 columns or more
on 16x16x4 MFMA blocks, split over K) or a few columns (a matrix times a
vector; up to 8 columns over many rows, one wave holding 1, 2 or 4 rows; 7
to 32 columns over 128 rows or more on 16x16x4 MFMA blocks, split over K;
7 to 16 columns over 4096 rows or more and K >= 2048, one workgroup per 16
rows over all of K, A's rows staged through LDS); and matmuls whose tiles leave
most of the machine idle over a long K (gemm.mfma split over K, then
gemm.combine).

Bars: bit for bit on integer data (every partial sum exact, whatever the
order); on real data within the accumulation bound (K - 1) u sum |a b| per
output of a float64 product (u = 2^-24), any summation order meeting it;
the epilogue on top as in the matmul tests.  CPU: the planner's choice and
the kernels run on the CPU (bounds, and values on integer data).  GPU: the
same shapes and layouts against the oracle and float64.
"""

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import CONFIG_SIZES, config_graph, config_inputs, placeholder
from tests.kernel_emu import emulate as emu

needs_clang = pytest.mark.skipif(not emu.available(), reason="host clang++ from ROCm is required")


def _kinds(expr):
    return [k["kind"] for k in porch.plan(expr)["kernels"]]


def _ints(shape, seed):
    return np.random.default_rng(seed).integers(-3, 4, size=shape).astype(np.float32)


def _reals(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


# name: (operand shapes (storage), graph over the two tensors, the product
# of two arrays as the graph takes it, the epilogue on that product,
# expected kernels)
CASES = {
    "vector times matrix": (
        ([1, 4096], [4096, 4096]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.wide", "gemm.combine"]),
    "eight rows, relu epilogue": (
        ([8, 2048], [2048, 1024]), lambda a, b: porch.relu(porch.matmul(a, b) - 1.0), lambda a, b: a @ b,
        lambda p: np.maximum(p - 1.0, 0.0), ["gemm.wide", "gemm.combine"]),
    "seven rows, relu epilogue": (
        ([7, 2048], [2048, 1024]), lambda a, b: porch.relu(porch.matmul(a, b) - 1.0), lambda a, b: a @ b,
        lambda p: np.maximum(p - 1.0, 0.0), ["gemm.wide", "gemm.combine"]),
    "seven rows, columns not a multiple of four, relu epilogue": (
        ([7, 2048], [2048, 1022]), lambda a, b: porch.relu(porch.matmul(a, b) - 1.0), lambda a, b: a @ b,
        lambda p: np.maximum(p - 1.0, 0.0), ["gemm.rows", "gemm.combine"]),
    "wide, thirty-two rows": (
        ([32, 1024], [1024, 4096]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.wide", "gemm.combine"]),
    "wide, ragged rows and columns, K tail, relu": (
        ([20, 203], [203, 300]), lambda a, b: porch.relu(porch.matmul(a, b) + 1.0), lambda a, b: a @ b,
        lambda p: np.maximum(p + 1.0, 0.0), ["gemm.wide", "gemm.combine"]),
    "wide, one chunk, epilogue in the kernel": (
        ([32, 100], [100, 256]), lambda a, b: porch.matmul(a, b) * 0.5 - 1.0, lambda a, b: a @ b,
        lambda p: p * 0.5 - 1.0, ["gemm.wide"]),
    "wide, two groups a wave, written out": (
        ([32, 512], [512, 1024]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.wide", "gemm.combine"]),
    "wide, four groups a wave, written out, relu": (
        ([32, 2048], [2048, 2048]), lambda a, b: porch.relu(porch.matmul(a, b) - 2.0), lambda a, b: a @ b,
        lambda p: np.maximum(p - 2.0, 0.0), ["gemm.wide", "gemm.combine"]),
    "wide, forty-eight rows": (
        ([48, 4096], [4096, 2048]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.wide", "gemm.combine"]),
    "wide, sixty-four rows, relu": (
        ([64, 4096], [4096, 4096]), lambda a, b: porch.relu(porch.matmul(a, b) + 0.5), lambda a, b: a @ b,
        lambda p: np.maximum(p + 0.5, 0.0), ["gemm.wide", "gemm.combine"]),
    "wide, batched": (
        ([2, 24, 516], [2, 516, 512]), lambda a, b: porch.batched_matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.wide", "gemm.combine"]),
    "wide, transposed A": (
        ([300, 32], [300, 1024]), lambda a, b: porch.matmul(porch.transpose(a), b), lambda a, b: a.T @ b,
        lambda p: p, ["gemm.wide", "gemm.combine"]),
    "rows, ragged columns": (
        ([3, 777], [777, 1003]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.rows", "gemm.combine"]),
    "rows, transposed B, K not a multiple of 16": (
        ([2, 1000], [3000, 1000]), lambda a, b: porch.matmul(a, porch.transpose(b)), lambda a, b: a @ b.T,
        lambda p: p, ["gemm.rows", "gemm.combine"]),
    "wide, transposed B, two rows": (
        ([2, 1024], [3000, 1024]), lambda a, b: porch.matmul(a, porch.transpose(b)), lambda a, b: a @ b.T,
        lambda p: p, ["gemm.wide", "gemm.combine"]),
    "wide, transposed B (x @ W^T)": (
        ([32, 4096], [4096, 4096]), lambda a, b: porch.matmul(a, porch.transpose(b)), lambda a, b: a @ b.T,
        lambda p: p, ["gemm.wide", "gemm.combine"]),
    "wide, transposed B, ragged columns, relu": (
        ([20, 512], [1000, 512]), lambda a, b: porch.relu(porch.matmul(a, porch.transpose(b)) + 1.0),
        lambda a, b: a @ b.T, lambda p: np.maximum(p + 1.0, 0.0), ["gemm.wide", "gemm.combine"]),
    "wide, transposed B, one chunk, epilogue in the kernel": (
        ([32, 64], [300, 64]), lambda a, b: porch.matmul(a, porch.transpose(b)) * 0.5 - 1.0,
        lambda a, b: a @ b.T, lambda p: p * 0.5 - 1.0, ["gemm.wide"]),
    "wide, transposed B, batched": (
        ([2, 24, 512], [2, 520, 512]), lambda a, b: porch.batched_matmul(a, porch.permute(b, [0, 2, 1])),
        lambda a, b: a @ np.swapaxes(b, -1, -2), lambda p: p, ["gemm.wide", "gemm.combine"]),
    "rows, batched": (
        ([4, 3, 512], [4, 512, 1022]), lambda a, b: porch.batched_matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.rows", "gemm.combine"]),
    "wide, three rows, batched": (
        ([4, 3, 512], [4, 512, 1024]), lambda a, b: porch.batched_matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.wide", "gemm.combine"]),
    "rows, one chunk": (
        ([2, 64], [64, 4094]), lambda a, b: porch.matmul(a, b) * 0.5, lambda a, b: a @ b, lambda p: p * 0.5,
        ["gemm.rows"]),
    "wide, two rows, one chunk": (
        ([2, 64], [64, 4096]), lambda a, b: porch.matmul(a, b) * 0.5, lambda a, b: a @ b, lambda p: p * 0.5,
        ["gemm.wide"]),
    "matrix times vector": (
        ([4096, 4096], [4096, 1]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.cols"]),
    "three columns, odd K, bias": (
        ([5000, 701], [701, 3]), lambda a, b: porch.matmul(a, b) + 2.0, lambda a, b: a @ b, lambda p: p + 2.0,
        ["gemm.cols"]),
    "eight columns over many rows": (
        ([2048, 700], [700, 8]), lambda a, b: porch.matmul(a, b) * 0.5 + 1.0, lambda a, b: a @ b,
        lambda p: p * 0.5 + 1.0, ["gemm.narrow", "gemm.combine"]),
    "seven columns over many rows, A transposed": (
        ([700, 2048], [700, 7]), lambda a, b: porch.matmul(porch.transpose(a), b), lambda a, b: a.T @ b,
        lambda p: p, ["gemm.cols"]),
    "narrow, sixteen columns": (
        ([4096, 1024], [1024, 16]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.narrow", "gemm.combine"]),
    "narrow, ragged rows and columns, K tail, relu": (
        ([1100, 1036], [1036, 20]), lambda a, b: porch.relu(porch.matmul(a, b) - 2.0), lambda a, b: a @ b,
        lambda p: np.maximum(p - 2.0, 0.0), ["gemm.narrow", "gemm.combine"]),
    "narrow, one chunk, epilogue in the kernel": (
        ([2048, 120], [120, 32]), lambda a, b: porch.matmul(a, b) * 0.5 + 1.0, lambda a, b: a @ b,
        lambda p: p * 0.5 + 1.0, ["gemm.narrow"]),
    "narrow, batched, ragged row tiles": (
        ([3, 700, 96], [3, 96, 24]), lambda a, b: porch.batched_matmul(a, b) + 1.0, lambda a, b: a @ b,
        lambda p: p + 1.0, ["gemm.narrow"]),
    "narrow, batched, split K": (
        ([2, 600, 2048], [2, 2048, 24]), lambda a, b: porch.batched_matmul(a, b), lambda a, b: a @ b,
        lambda p: p, ["gemm.narrow", "gemm.combine"]),
    "narrow, transposed B": (
        ([2048, 516], [12, 516]), lambda a, b: porch.matmul(a, porch.transpose(b)), lambda a, b: a @ b.T,
        lambda p: p, ["gemm.narrow", "gemm.combine"]),
    "narrow, two groups a wave, written out": (
        ([1024, 1024], [1024, 24]), lambda a, b: porch.matmul(a, b) - 1.0, lambda a, b: a @ b, lambda p: p - 1.0,
        ["gemm.narrow", "gemm.combine"]),
    "narrow rows, sixteen columns": (
        ([4096, 2048], [2048, 16]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.narrow_rows"]),
    "narrow rows, ragged rows and columns, K tail, relu": (
        ([4090, 2100], [2100, 13]), lambda a, b: porch.relu(porch.matmul(a, b) - 2.0), lambda a, b: a @ b,
        lambda p: np.maximum(p - 2.0, 0.0), ["gemm.narrow_rows"]),
    "narrow rows, batched": (
        ([2, 2048, 2048], [2, 2048, 16]), lambda a, b: porch.batched_matmul(a, b) + 1.0, lambda a, b: a @ b,
        lambda p: p + 1.0, ["gemm.narrow_rows"]),
    "narrow rows, four waves, K tail": (
        ([4096, 4104], [4104, 9]), lambda a, b: porch.matmul(a, b) * 0.5, lambda a, b: a @ b, lambda p: p * 0.5,
        ["gemm.narrow_rows"]),
    "narrow rows, four waves, eight rounds, relu": (
        ([4096, 8196], [8196, 11]), lambda a, b: porch.relu(porch.matmul(a, b) + 1.0), lambda a, b: a @ b,
        lambda p: np.maximum(p + 1.0, 0.0), ["gemm.narrow_rows"]),
    "narrow rows, transposed B": (
        ([4096, 3000], [9, 3000]), lambda a, b: porch.matmul(a, porch.transpose(b)), lambda a, b: a @ b.T,
        lambda p: p, ["gemm.narrow_rows"]),
    # every wave's range whole rounds of 256 (the next round's values of B
    # loaded during this round's MFMAs)
    "narrow rows, whole rounds, ragged rows and columns, relu": (
        ([4090, 4096], [4096, 13]), lambda a, b: porch.relu(porch.matmul(a, b) - 2.0), lambda a, b: a @ b,
        lambda p: np.maximum(p - 2.0, 0.0), ["gemm.narrow_rows"]),
    "narrow rows, whole rounds, transposed B": (
        ([4096, 4096], [11, 4096]), lambda a, b: porch.matmul(a, porch.transpose(b)), lambda a, b: a @ b.T,
        lambda p: p, ["gemm.narrow_rows"]),
    "narrow rows, four waves, whole rounds, batched": (
        ([2, 2048, 6144], [2, 6144, 16]), lambda a, b: porch.batched_matmul(a, b) * 0.5, lambda a, b: a @ b,
        lambda p: p * 0.5, ["gemm.narrow_rows"]),
    "six columns, batched, ragged row groups": (
        ([2, 1101, 512], [2, 512, 6]), lambda a, b: porch.batched_matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.cols"]),
    "three columns, ragged row pairs, transposed B": (
        ([1001, 300], [3, 300]), lambda a, b: porch.matmul(a, porch.transpose(b)), lambda a, b: a @ b.T,
        lambda p: p, ["gemm.cols"]),
    "columns, transposed A": (
        ([1024, 2000], [1024, 2]), lambda a, b: porch.matmul(porch.transpose(a), b), lambda a, b: a.T @ b,
        lambda p: p, ["gemm.cols"]),
    "split K": (
        ([96, 4096], [4096, 4096]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.mfma", "gemm.combine"]),
    "split K, ragged K, relu epilogue": (
        ([40, 1030], [1030, 200]), lambda a, b: porch.relu(porch.matmul(a, b) + 1.0), lambda a, b: a @ b,
        lambda p: np.maximum(p + 1.0, 0.0), ["gemm.mfma", "gemm.combine"]),
    "split K, transposed A": (
        ([2048, 96], [2048, 160]), lambda a, b: porch.matmul(porch.transpose(a), b), lambda a, b: a.T @ b,
        lambda p: p, ["gemm.mfma", "gemm.combine"]),
    "split K, five rows": (
        ([5, 1030], [1030, 200]), lambda a, b: porch.matmul(a, b) * 2.0, lambda a, b: a @ b, lambda p: p * 2.0,
        ["gemm.mfma", "gemm.combine"]),
    "split K, eight columns": (
        ([100, 1024], [1024, 8]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.mfma", "gemm.combine"]),
    "vector times a narrow matrix": (
        ([1, 4096], [4096, 100]), lambda a, b: porch.matmul(a, b), lambda a, b: a @ b, lambda p: p,
        ["gemm.mfma", "gemm.combine"]),
    "split K, batched": (
        ([2, 100, 1024], [2, 1024, 300]), lambda a, b: porch.batched_matmul(a, b), lambda a, b: a @ b,
        lambda p: p, ["gemm.mfma", "gemm.combine"]),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_short_sided_products_take_the_skinny_kernels(name):
    shapes, build, _, _, kinds = CASES[name]
    expr = build(*[placeholder(s) for s in shapes])
    assert _kinds(expr) == kinds
    porch.plan(expr, compile=True)


def test_wide_products_keep_mfma():
    assert _kinds(porch.matmul(placeholder([96, 512]), placeholder([512, 1024]))) == ["gemm.mfma"]  # short K
    assert _kinds(porch.matmul(placeholder([1024, 4096]), placeholder([4096, 2048]))) == ["gemm.mfma"]  # many tiles
    assert _kinds(porch.matmul(placeholder([8, 64]), placeholder([64, 64]))) == ["gemm.scalar"]


@pytest.mark.parametrize("shape, chunks", [
    ((96, 4096, 4096), 16),  # 32 tiles: 16 chunks of 256 give 512 workgroups
    ((40, 1030, 200), 5),    # 65 K-steps, 2 tiles: the largest divisor with 8 steps a chunk
    ((512, 1024, 512), 8),   # 16 tiles: 64 K-steps in 8 chunks
])
def test_split_k_chunks(shape, chunks):
    m, k, n = shape
    plan = porch.plan(porch.matmul(placeholder([m, k]), placeholder([k, n])))
    assert [x["kind"] for x in plan["kernels"]] == ["gemm.mfma", "gemm.combine"]
    tiles = -(-m // 128) * -(-n // 128)
    assert plan["kernels"][0]["grid"][0] == tiles * chunks
    assert plan["temps"] == [chunks * m * n]


# Epilogues that read another input (a bias row): the kernel that applies
# the epilogue (the combine where there is one) loads it at the output's
# coordinates.
BIAS_SHAPES = {
    (4096, 2048, 16): ["gemm.narrow_rows"],
    (8, 2048, 1024): ["gemm.wide", "gemm.combine"],
    (4, 2048, 1024): ["gemm.wide", "gemm.combine"],
    (4, 2048, 1022): ["gemm.rows", "gemm.combine"],
    (40, 1030, 200): ["gemm.mfma", "gemm.combine"],
    (3000, 300, 2): ["gemm.cols"],
}


def _bias_graph(a, b, bias, m, n):
    return porch.relu(porch.matmul(a, b) + porch.broadcast_to(bias, [m, n]))


@pytest.mark.parametrize("shape", sorted(BIAS_SHAPES))
def test_epilogues_reading_an_input(shape):
    m, k, n = shape
    expr = _bias_graph(placeholder([m, k]), placeholder([k, n]), placeholder([1, n]), m, n)
    assert _kinds(expr) == BIAS_SHAPES[shape]
    porch.plan(expr, compile=True)


@needs_clang
def test_emulated_split_k_with_a_bias_is_exact():
    m, k, n = 40, 1030, 200
    xs = [_ints([m, k], 1), _ints([k, n], 2), _ints([1, n], 3)]
    expr = _bias_graph(*[placeholder(x.shape, x) for x in xs], m, n)
    assert all(r["ok"] for r in emu.emulate(expr, timeout=600))
    got = emu.evaluate(expr, xs, timeout=600)
    want = np.maximum(xs[0].astype(np.float64) @ xs[1] + xs[2], 0.0).astype(np.float32)
    assert np.array_equal(got.reshape(want.shape), want)


@needs_clang
@pytest.mark.parametrize("name", ["rows, ragged columns", "rows, transposed B, K not a multiple of 16", "rows, batched",
                                  "rows, one chunk", "three columns, odd K, bias", "columns, transposed A",
                                  "split K, ragged K, relu epilogue", "split K, transposed A",
                                  "split K, five rows", "split K, eight columns",
                                  "eight columns over many rows", "six columns, batched, ragged row groups",
                                  "three columns, ragged row pairs, transposed B",
                                  "seven columns over many rows, A transposed",
                                  "narrow, ragged rows and columns, K tail, relu",
                                  "narrow, one chunk, epilogue in the kernel", "narrow, batched, ragged row tiles",
                                  "narrow, transposed B", "narrow rows, ragged rows and columns, K tail, relu",
                                  "narrow rows, four waves, K tail", "narrow, two groups a wave, written out",
                                  "wide, ragged rows and columns, K tail, relu",
                                  "wide, one chunk, epilogue in the kernel", "wide, batched", "wide, transposed A",
                                  "wide, two groups a wave, written out", "wide, transposed B, ragged columns, relu",
                                  "wide, transposed B, one chunk, epilogue in the kernel",
                                  "wide, transposed B, batched", "narrow rows, transposed B",
                                  "narrow rows, whole rounds, ragged rows and columns, relu",
                                  "narrow rows, whole rounds, transposed B",
                                  "narrow rows, four waves, whole rounds, batched"])
def test_emulated_integer_products_are_exact(name):
    shapes, build, prod, epi, _ = CASES[name]
    xs = [_ints(s, i + 1) for i, s in enumerate(shapes)]
    expr = build(*[placeholder(s, x) for s, x in zip(shapes, xs)])
    want = epi(prod(*[x.astype(np.float64) for x in xs])).astype(np.float32)
    kernels = porch.plan(expr)["kernels"]
    if len(kernels) == 1 and kernels[0]["grid"][0] >= 64:
        # a single kernel over many workgroups: its first two and last two
        # (the first rows or columns and the ragged last ones); every
        # output is compared with the oracle on the GPU
        assert emu.check_edges(expr, xs, want) > 0
        return
    assert all(r["ok"] for r in emu.emulate(expr, timeout=600))
    got = emu.evaluate(expr, xs, timeout=600)
    assert np.array_equal(got.reshape(want.shape), want)


# -- GPU -----------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_integer_products_bit_exact(gpu, name):
    shapes, build, _, _, kinds = CASES[name]
    xs = [_ints(s, i + 7) for i, s in enumerate(shapes)]
    expr = build(*[gpu.tensor(s, x) for s, x in zip(shapes, xs)])
    assert _kinds(expr) == kinds
    out = gpu.materialize(expr).cpu().reshape(expr.shape())
    ref = host.evaluate(expr)
    assert np.array_equal(out, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_real_products_within_the_accumulation_bound(gpu, name):
    shapes, build, prod, epi, _ = CASES[name]
    xs = [_reals(s, i + 11) for i, s in enumerate(shapes)]
    expr = build(*[gpu.tensor(s, x) for s, x in zip(shapes, xs)])
    out = gpu.materialize(expr).cpu().reshape(expr.shape()).astype(np.float64)
    x64 = [x.astype(np.float64) for x in xs]
    product = prod(*x64)
    k = x64[0].shape[-1] if "transposed A" not in name else x64[0].shape[0]
    bound = (k - 1) * 2.0 ** -24 * prod(*[np.abs(x) for x in x64])
    want = epi(product)
    # the product within its bound, then one rounding of the epilogue
    assert np.all(np.abs(out - want) <= bound + 2.0 ** -24 * np.abs(want) + 1e-37), \
        np.max(np.abs(out - want) - bound)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", sorted(BIAS_SHAPES))
def test_epilogue_reading_an_input_bit_exact(gpu, shape):
    m, k, n = shape
    xs = [_ints([m, k], 21), _ints([k, n], 22), _ints([1, n], 23)]
    expr = _bias_graph(*[gpu.tensor(list(x.shape), x) for x in xs], m, n)
    assert _kinds(expr) == BIAS_SHAPES[shape]
    out = gpu.materialize(expr).cpu().reshape(m, n)
    assert np.array_equal(out, host.evaluate(expr).reshape(m, n))


@pytest.mark.parametrize("shape, chunks", [
    ((4096, 1024, 16), 2),   # 128 row tiles of 32: 2 chunks of 512 for a workgroup a CU
    ((1100, 1036, 20), 6),   # 35 row tiles: 8 chunks for the CUs (12 for partials at most 1/4
                             # of A), of 130 -> 192 values of K (a multiple of 64): 6 chunks
    ((2048, 256, 32), 2),    # partials at most 1/4 of A: 256 / (4 x 32) chunks
    ((512, 4096, 16), 16),   # 16 row tiles: 16 chunks of 256 for the CUs
    ((256, 8192, 8), 32),    # 8 row tiles: 32 chunks for the CUs, at most 32
    ((2048, 120, 32), 1),    # too short a K to split: the epilogue in the kernel
])
def test_narrow_chunks(shape, chunks):
    m, k, n = shape
    plan = porch.plan(porch.matmul(placeholder([m, k]), placeholder([k, n])))
    kinds = [x["kind"] for x in plan["kernels"]]
    assert kinds == (["gemm.narrow", "gemm.combine"] if chunks > 1 else ["gemm.narrow"])
    # one workgroup of four waves per 32-row tile and chunk
    assert plan["kernels"][0]["grid"][0] == -(-m // 32) * chunks
    assert plan["kernels"][0]["block"] == 256
    assert plan["temps"] == ([chunks * m * n] if chunks > 1 else [])


@pytest.mark.parametrize("shape, batch", [((4096, 4096, 16), 1), ((4090, 2100, 13), 1), ((2048, 2048, 16), 2),
                                          ((4096, 8192, 16), 1), ((4096, 16384, 7), 1)])
def test_narrow_rows_plan(shape, batch):
    # one workgroup per 16 rows (over all batch entries), no partial
    # products: 8 waves while each takes at most two rounds of 256 values
    # of K, else 4
    m, k, n = shape
    a, b = placeholder([batch, m, k] if batch > 1 else [m, k]), placeholder([batch, k, n] if batch > 1 else [k, n])
    plan = porch.plan(porch.batched_matmul(a, b) if batch > 1 else porch.matmul(a, b))
    assert [x["kind"] for x in plan["kernels"]] == ["gemm.narrow_rows"]
    assert plan["kernels"][0]["grid"][0] == batch * -(-m // 16)
    assert plan["kernels"][0]["block"] == (512 if k <= 4096 else 256)
    assert plan["temps"] == []


def test_narrow_bounds():
    # below 7 columns gemm.cols, above 32 or below 128 rows the MFMA tiles
    assert _kinds(porch.matmul(placeholder([4096, 4096]), placeholder([4096, 6]))) == ["gemm.cols"]
    assert _kinds(porch.matmul(placeholder([4096, 4096]), placeholder([4096, 7])))[0] == "gemm.narrow_rows"
    # gemm.narrow_rows: up to 16 columns, at least one workgroup of 16 rows
    # per compute unit, K of 2048 or more
    assert _kinds(porch.matmul(placeholder([4096, 4096]), placeholder([4096, 16])))[0] == "gemm.narrow_rows"
    assert _kinds(porch.matmul(placeholder([4096, 4096]), placeholder([4096, 17])))[0] == "gemm.narrow"
    assert _kinds(porch.matmul(placeholder([4080, 4096]), placeholder([4096, 16])))[0] == "gemm.narrow"
    assert _kinds(porch.matmul(placeholder([4081, 4096]), placeholder([4096, 16])))[0] == "gemm.narrow_rows"
    assert _kinds(porch.matmul(placeholder([4096, 2044]), placeholder([2044, 16])))[0] == "gemm.narrow"
    assert _kinds(porch.matmul(placeholder([4096, 2048]), placeholder([2048, 16])))[0] == "gemm.narrow_rows"
    # at most 16 rounds of 256 values a wave (four waves): K up to 16384
    assert _kinds(porch.matmul(placeholder([4096, 16384]), placeholder([16384, 16])))[0] == "gemm.narrow_rows"
    assert _kinds(porch.matmul(placeholder([4096, 16388]), placeholder([16388, 16])))[0] == "gemm.narrow"
    assert _kinds(porch.matmul(placeholder([4096, 4096]), placeholder([4096, 32])))[0] == "gemm.narrow"
    assert _kinds(porch.matmul(placeholder([4096, 4096]), placeholder([4096, 33])))[0] == "gemm.mfma"
    assert _kinds(porch.matmul(placeholder([128, 4096]), placeholder([4096, 16])))[0] == "gemm.narrow"
    assert _kinds(porch.matmul(placeholder([127, 4096]), placeholder([4096, 16])))[0] == "gemm.mfma"
    # K not a multiple of 4: A's rows cannot be read as float4s
    assert _kinds(porch.matmul(placeholder([4096, 1030]), placeholder([1030, 16])))[0] == "gemm.mfma"


@pytest.mark.gpu
def test_narrow_infinities_in_the_k_tail(gpu):
    """Infinities in the last rows of B (K = 1036: a partial last step of 16,
    whose lanes past K read the last 4 values and zero both operands): the
    outputs are inf or NaN exactly where the oracle's are, in any summation
    order (integer data, zeros in A giving 0 x inf)."""
    m, k, n = 1100, 1036, 20
    a, b = _ints([m, k], 31), _ints([k, n], 32)
    b[k - 1, :] = np.inf
    b[k - 2, 3] = -np.inf
    b[k - 5, 7] = np.inf
    expr = porch.matmul(gpu.tensor([m, k], a), gpu.tensor([k, n], b))
    assert _kinds(expr) == ["gemm.narrow", "gemm.combine"]
    out = gpu.materialize(expr).cpu().reshape(m, n)
    ref = np.asarray(host.evaluate(expr), np.float32).reshape(m, n)
    assert np.isinf(ref).any() and np.isnan(ref).any()
    assert np.array_equal(out, ref, equal_nan=True)


@pytest.mark.parametrize("shape, chunks", [
    ((32, 4096, 4096), 4),   # 64 column tiles: 4 chunks for a workgroup a CU
    ((20, 203, 300), 2),     # partials at most 1/4 of B: 203 / (4 x 20) chunks
    ((8, 8192, 256), 32),    # 4 column tiles: 64 chunks for the CUs, at most 32
    ((32, 100, 256), 1),     # too short a K to split: the epilogue in the kernel
])
def test_wide_chunks(shape, chunks):
    m, k, n = shape
    plan = porch.plan(porch.matmul(placeholder([m, k]), placeholder([k, n])))
    kinds = [x["kind"] for x in plan["kernels"]]
    assert kinds == (["gemm.wide", "gemm.combine"] if chunks > 1 else ["gemm.wide"])
    # one workgroup of four waves per 64-column tile and chunk
    assert plan["kernels"][0]["grid"][0] == -(-n // 64) * chunks
    assert plan["kernels"][0]["block"] == 256
    assert plan["temps"] == ([chunks * m * n] if chunks > 1 else [])


def test_wide_bounds():
    # from 1 to 32 rows over 256 columns or more (64 with enough
    # workgroups), B's rows read as float4s
    assert _kinds(porch.matmul(placeholder([1, 4096]), placeholder([4096, 4096])))[0] == "gemm.wide"
    assert _kinds(porch.matmul(placeholder([7, 4096]), placeholder([4096, 4096])))[0] == "gemm.wide"
    assert _kinds(porch.matmul(placeholder([7, 4096]), placeholder([4096, 4094])))[0] == "gemm.rows"
    assert _kinds(porch.matmul(placeholder([8, 4096]), placeholder([4096, 4096])))[0] == "gemm.wide"
    assert _kinds(porch.matmul(placeholder([64, 4096]), placeholder([4096, 4096])))[0] == "gemm.wide"
    assert _kinds(porch.matmul(placeholder([65, 4096]), placeholder([4096, 4096])))[0] == "gemm.mfma"
    # over 32 rows only with a workgroup for every CU (64 tiles x 4 chunks,
    # 32 x 8, then 16 x 2 below)
    assert _kinds(porch.matmul(placeholder([48, 4096]), placeholder([4096, 4096])))[0] == "gemm.wide"
    assert _kinds(porch.matmul(placeholder([48, 2048]), placeholder([2048, 2048])))[0] == "gemm.wide"
    assert _kinds(porch.matmul(placeholder([64, 512]), placeholder([512, 1024])))[0] == "gemm.mfma"
    assert _kinds(porch.matmul(placeholder([32, 4096]), placeholder([4096, 252])))[0] == "gemm.mfma"
    assert _kinds(porch.matmul(placeholder([16, 4096]), placeholder([4096, 254])))[0] == "gemm.mfma"
    # B stored transposed (x @ W^T): its columns read along K, in whole
    # groups of 32 values of K
    assert _kinds(porch.matmul(placeholder([32, 4096]), porch.transpose(placeholder([4096, 4096]))))[0] == "gemm.wide"
    assert _kinds(porch.matmul(placeholder([32, 4064]), porch.transpose(placeholder([4096, 4064]))))[0] == "gemm.wide"
    assert _kinds(porch.matmul(placeholder([32, 4080]), porch.transpose(placeholder([4096, 4080]))))[0] == "gemm.mfma"
    assert _kinds(porch.matmul(placeholder([32, 4092]), porch.transpose(placeholder([4096, 4092]))))[0] == "gemm.mfma"
    assert _kinds(porch.matmul(placeholder([8, 4092]), porch.transpose(placeholder([4096, 4092]))))[0] == "gemm.rows"


@pytest.mark.gpu
def test_wide_infinities_in_the_k_tail(gpu):
    """Infinities in the last rows of B (K = 203: a partial last step of 4,
    whose lanes past K read the last value and zero both operands): inf or
    NaN exactly where the oracle has them, in any summation order."""
    m, k, n = 20, 203, 300
    a, b = _ints([m, k], 41), _ints([k, n], 42)
    b[k - 1, :] = np.inf
    b[k - 2, 5] = -np.inf
    b[k - 3, 9] = np.inf
    expr = porch.matmul(gpu.tensor([m, k], a), gpu.tensor([k, n], b))
    assert _kinds(expr) == ["gemm.wide", "gemm.combine"]
    out = gpu.materialize(expr).cpu().reshape(m, n)
    ref = np.asarray(host.evaluate(expr), np.float32).reshape(m, n)
    assert np.isinf(ref).any() and np.isnan(ref).any()
    assert np.array_equal(out, ref, equal_nan=True)


@pytest.mark.gpu
def test_narrow_rows_infinities_at_the_waves_ends(gpu):
    """Infinities in B's rows at the ends of the waves' ranges of K (K = 2100:
    264 values a wave, the last wave 252, its second round empty; lanes
    past a wave's end read column 0 and zero both operands): inf or NaN
    exactly where the oracle has them."""
    m, k, n = 4090, 2100, 13
    a, b = _ints([m, k], 33), _ints([k, n], 34)
    b[k - 1, :] = np.inf
    b[263, 3] = -np.inf     # the first wave's last value
    b[264, 4] = np.inf      # the second wave's first
    b[k - 252, 7] = np.inf  # the last wave's first
    expr = porch.matmul(gpu.tensor([m, k], a), gpu.tensor([k, n], b))
    assert _kinds(expr) == ["gemm.narrow_rows"]
    out = gpu.materialize(expr).cpu().reshape(m, n)
    ref = np.asarray(host.evaluate(expr), np.float32).reshape(m, n)
    assert np.isinf(ref).any() and np.isnan(ref).any()
    assert np.array_equal(out, ref, equal_nan=True)


@pytest.mark.gpu
def test_narrow_rows_infinities_at_whole_round_edges(gpu):
    """Infinities in B's rows at the edges of whole rounds (K = 4096: 512
    values a wave in two rounds of 256, the second round's values of B
    loaded during the first round's MFMAs): inf or NaN exactly where the
    oracle has them."""
    m, k, n = 4096, 4096, 16
    a, b = _ints([m, k], 35), _ints([k, n], 36)
    b[255, :] = np.inf      # the first wave's first round, its last value
    b[256, 3] = -np.inf     # its second round's first
    b[767, 5] = np.inf      # the second wave's first round, its last value
    b[768, 2] = -np.inf     # its second round's first
    b[k - 1, 7] = np.inf    # the last wave's last value
    expr = porch.matmul(gpu.tensor([m, k], a), gpu.tensor([k, n], b))
    assert _kinds(expr) == ["gemm.narrow_rows"]
    out = gpu.materialize(expr).cpu().reshape(m, n)
    ref = np.asarray(host.evaluate(expr), np.float32).reshape(m, n)
    assert np.isinf(ref).any() and np.isnan(ref).any()
    assert np.array_equal(out, ref, equal_nan=True)


@pytest.mark.gpu
@pytest.mark.parametrize("kind, m, k, n", [("gemm.narrow", 1100, 1036, 20), ("gemm.narrow_rows", 4090, 2100, 13),
                                           ("gemm.wide", 20, 203, 300)])
def test_clamped_edge_rows_and_columns(gpu, kind, m, k, n):
    """Rows past m and columns past n of the last tiles are read at the last
    row (column) and feed only outputs that are not stored: a NaN in A's
    last row and an infinity in B's last column reach exactly the outputs
    the oracle gives them (integer data, zeros in A giving 0 x inf = NaN)."""
    a, b = _ints([m, k], 51), _ints([k, n], 52)
    a[m - 1, 3] = np.nan
    b[7, n - 1] = np.inf
    expr = porch.matmul(gpu.tensor([m, k], a), gpu.tensor([k, n], b))
    assert _kinds(expr)[0] == kind
    out = gpu.materialize(expr).cpu().reshape(m, n)
    ref = np.asarray(host.evaluate(expr), np.float32).reshape(m, n)
    assert np.isnan(ref[m - 1]).all() and not np.isnan(ref[: m - 1, : n - 1]).any()
    assert np.array_equal(out, ref, equal_nan=True)


@pytest.mark.gpu
@pytest.mark.parametrize("name, kinds", [("narrow_product", ["gemm.narrow_rows"]),
                                         ("wide_product", ["gemm.wide", "gemm.combine"])])
def test_benchmark_products_every_output(gpu, name, kinds):
    """The benchmark's two products with one short side, at their size, on
    its seeded inputs: every output against a float64 product of the same
    float32 operands, within the accumulation bound (K - 1) 2^-24 sum |a||b|
    (the reference computes every output through its K loop,
    src/tensor.cpp:684-721)."""
    size = CONFIG_SIZES[name]
    m, k, n = size["m"], size["k"], size["n"]
    a, b = config_inputs(name)
    expr = config_graph(name, [gpu.tensor([m, k], a), gpu.tensor([k, n], b)])
    assert _kinds(expr) == kinds
    out = gpu.materialize(expr).cpu().reshape(m, n).astype(np.float64)
    a64 = np.asarray(a, np.float32).reshape(m, k).astype(np.float64)
    b64 = np.asarray(b, np.float32).reshape(k, n).astype(np.float64)
    bound = (k - 1) * 2.0 ** -24 * (np.abs(a64) @ np.abs(b64))
    frac = np.abs(out - a64 @ b64) / bound
    assert np.all(frac <= 1.0), (float(frac.max()), np.unravel_index(frac.argmax(), frac.shape))

