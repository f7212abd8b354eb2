"""Seeded random graphs mixing every kind of region the planner forms:
views (permutes included), concat, broadcasts, elementwise arithmetic, sum/max reductions over
any axis (fused into row programs, column reductions, or materialised
temporaries), and matmuls and batched matmuls whose operands are expressions
and whose results feed further ops.

Leaves hold small integers and the graphs are sized so every intermediate
stays far below 2^24: sums, maxima and matmul accumulations are then exact in
binary32 whatever the order, so every result must equal the oracle's bit for
bit, although the GPU sums in a different order.  The CPU test checks the
generator itself: every graph plans and compiles offline.
"""

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import placeholder

TRIALS = 120
LIMIT = float(1 << 20)


def random_graph(rng, make):
    """A random expression over leaves built by make(shape, rng)."""
    matmuls = 0

    def leaf(shape):
        return porch.tensor_expr(make(list(shape), rng))

    rank = int(rng.integers(1, 4))
    shape = [int(rng.integers(1, 40)) for _ in range(rank)]
    expr = leaf(shape)
    for _ in range(int(rng.integers(2, 8))):
        shape = list(expr.shape())
        rank = len(shape)
        kind = int(rng.integers(0, 12))
        if kind == 0:
            expr = expr * float(rng.choice([2.0, -1.0, 0.5])) + float(rng.integers(-3, 4))
        elif kind == 1:
            other = leaf(shape)
            expr = porch.maximum(expr, other) - porch.minimum(other, 1.0)
        elif kind == 2 and rank >= 1:
            axis = int(rng.integers(0, rank))
            keep = bool(rng.integers(0, 2))
            reduced = porch.sum(expr, axis, keep) if rng.integers(0, 2) else porch.max(expr, axis, keep)
            if keep and rng.integers(0, 2):
                # consume the reduction through a broadcast (row programs,
                # or a materialised temporary for non-last axes)
                expr = expr - porch.broadcast_to(reduced, shape)
            else:
                expr = reduced
        elif kind == 3 and rank >= 2:
            if rank == 2 and rng.integers(0, 2):
                expr = porch.transpose(expr)
            else:
                expr = porch.permute(expr, [int(a) for a in rng.permutation(rank)])
        elif kind == 4:
            lazy = porch.tensor(expr)
            items = [porch.slice(int(rng.integers(0, e)), e, int(rng.integers(1, 3))) for e in shape]
            expr = lazy[tuple(items)]
        elif kind == 5:
            n = int(np.prod(shape))
            factors = [f for f in range(1, n + 1) if n % f == 0]
            f = int(rng.choice(factors))
            expr = porch.reshape(expr, [f, n // f])
        elif kind == 6 and rank < 3:
            expr = porch.unsqueeze(expr, int(rng.integers(0, rank + 1)))
        elif kind == 7:
            target = [int(rng.integers(1, 4))] + [e if e != 1 else int(rng.integers(1, 5)) for e in shape]
            expr = porch.broadcast_to(expr, target)
        elif kind == 8:
            axis = int(rng.integers(0, rank))
            other_shape = list(shape)
            other_shape[axis] = int(rng.integers(1, 6))
            other = leaf(other_shape)
            expr = porch.concat(expr, other, axis) if rng.integers(0, 2) else porch.concat(other, expr, axis)
        elif kind == 9 and rank == 2 and matmuls < 2:
            matmuls += 1
            # wide products now and then, so the MFMA kernel and its tails run
            n = int(rng.integers(130, 300)) if rng.integers(0, 3) == 0 else int(rng.integers(1, 50))
            if rng.integers(0, 2):
                expr = porch.matmul(expr, leaf([shape[1], n]))
            else:
                expr = porch.matmul(leaf([n, shape[0]]), expr)
            if rng.integers(0, 2):  # an epilogue over the product
                expr = porch.relu(expr + porch.broadcast_to(leaf([1, expr.shape()[1]]), expr.shape())) - 1.0
        elif kind == 9 and rank == 3 and matmuls < 2:
            matmuls += 1
            n = int(rng.integers(1, 70))
            other = leaf([shape[0], shape[2], n])
            if rng.integers(0, 2):  # a weight shared by every entry
                other = porch.broadcast_to(leaf([shape[2], n]), [shape[0], shape[2], n])
            expr = porch.batched_matmul(expr, other)
        elif kind == 10:
            expr = expr + leaf(shape) * 2.0
        else:
            expr = porch.relu(expr) - porch.maximum(expr, -2.0)
        if int(np.prod(expr.shape())) > 40000 or int(np.prod(expr.shape())) == 0:
            break
    return expr


def integer_leaf(shape, rng):
    values = rng.integers(-3, 4, size=int(np.prod(shape))).astype(np.float32)
    return placeholder(shape, values)


def test_fuzz_graphs_plan_and_compile():
    rng = np.random.default_rng(424242)
    kinds = set()
    for _ in range(30):
        expr = random_graph(rng, integer_leaf)
        plan = porch.plan(expr, compile=True)
        kinds.update(k["kind"].split(".")[0] for k in plan["kernels"])
    # the generator reaches the planner's region kinds
    assert {"pointwise", "row", "gemm"} <= kinds


@pytest.mark.gpu
def test_fuzz_graphs_bit_exact(gpu):
    rng = np.random.default_rng(20261202)

    def device_leaf(shape, rng):
        values = rng.integers(-3, 4, size=int(np.prod(shape))).astype(np.float32)
        return gpu.tensor(shape, values)

    checked = 0
    kinds = set()
    for trial in range(TRIALS):
        expr = random_graph(rng, device_leaf)
        ref = host.evaluate(expr)
        if ref.size and np.max(np.abs(ref)) > LIMIT:
            continue  # too large to be exact in binary32 in every order
        plan = gpu.plan(expr)
        kinds.update(k["kind"] for k in plan["kernels"])
        out = gpu.materialize(expr).cpu().reshape(expr.shape())
        assert out.shape == ref.shape, trial
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (trial, plan)
        checked += 1
    assert checked >= TRIALS * 3 // 4
    print("kernel kinds exercised:", sorted(kinds))


def random_product(rng, make):
    """A matmul at MFMA sizes whose operands are views or expressions of
    leaves (ragged m, n, k), with a random epilogue."""
    m, k, n = (int(rng.integers(32, 300)), int(rng.integers(1, 300)), int(rng.integers(32, 300)))

    def operand(rows, cols):
        form = int(rng.integers(0, 4))
        if form == 0:
            return porch.tensor_expr(make([rows, cols], rng))
        if form == 1:  # transposed storage
            return porch.transpose(porch.tensor_expr(make([cols, rows], rng)))
        if form == 2:  # a strided window of a larger leaf
            big = make([rows + 3, 2 * cols], rng)
            return big[porch.slice(3, rows + 3), porch.slice(0, 2 * cols, 2)]
        return porch.tensor_expr(make([rows, cols], rng)) * 2.0 - 1.0  # an expression: materialised first

    expr = porch.matmul(operand(m, k), operand(k, n))
    form = int(rng.integers(0, 3))
    if form == 1:
        expr = porch.relu(expr + porch.broadcast_to(porch.tensor_expr(make([1, n], rng)), [m, n])) - 0.5
    elif form == 2:
        expr = porch.maximum(expr, porch.tensor_expr(make([m, n], rng))) * 2.0
    return expr


def test_fuzz_products_reach_the_mfma_kernel():
    rng = np.random.default_rng(7)
    kinds = [porch.plan(random_product(rng, integer_leaf))["kernels"][-1]["kind"] for _ in range(20)]
    assert kinds.count("gemm.mfma") >= 15


@pytest.mark.gpu
def test_fuzz_products_bit_exact(gpu):
    rng = np.random.default_rng(99)

    def device_leaf(shape, rng):
        values = rng.integers(-3, 4, size=int(np.prod(shape))).astype(np.float32)
        return gpu.tensor(shape, values)

    for trial in range(30):
        expr = random_product(rng, device_leaf)
        ref = host.evaluate(expr)
        assert np.max(np.abs(ref)) < LIMIT
        out = gpu.materialize(expr).cpu().reshape(expr.shape())
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (trial, gpu.plan(expr))


def random_lopsided_product(rng, make):
    """A matmul with one short side or few tiles over a long K (the
    few-row, few-column, narrow, wide and split-K kernels), operands as in
    random_product, with a random epilogue (a bias row among them)."""
    form = int(rng.integers(0, 5))
    if form == 0:    # a few rows: gemm.rows or gemm.wide (+ gemm.combine)
        m, k, n = int(rng.integers(1, 17)), int(rng.integers(64, 3000)), int(rng.integers(256, 1200))
    elif form == 1:  # a few columns: gemm.cols
        m, k, n = int(rng.integers(64, 3000)), int(rng.integers(1, 1500)), int(rng.integers(1, 5))
    elif form == 2:  # few 128 x 128 tiles over K >= 1024: split over K
        m, k, n = int(rng.integers(17, 260)), int(rng.integers(1024, 3000)), int(rng.integers(32, 300))
    elif form == 3:  # 7 to 32 columns, K a multiple of 4: gemm.narrow where A's rows are contiguous
        m, k, n = int(rng.integers(128, 3000)), 4 * int(rng.integers(1, 700)), int(rng.integers(7, 33))
    else:            # 8 to 32 rows, N a multiple of 4: gemm.wide where B's rows are contiguous
        m, k, n = int(rng.integers(8, 33)), int(rng.integers(16, 3000)), 4 * int(rng.integers(64, 300))

    def operand(rows, cols):
        f = int(rng.integers(0, 3))
        if f == 0:
            return porch.tensor_expr(make([rows, cols], rng))
        if f == 1:
            return porch.transpose(porch.tensor_expr(make([cols, rows], rng)))
        return porch.tensor_expr(make([rows, cols], rng)) * 2.0 - 1.0

    expr = porch.matmul(operand(m, k), operand(k, n))
    epi = int(rng.integers(0, 3))
    if epi == 1:
        expr = porch.relu(expr + porch.broadcast_to(porch.tensor_expr(make([1, n], rng)), [m, n])) - 0.5
    elif epi == 2:
        expr = porch.maximum(expr, porch.tensor_expr(make([m, n], rng))) * 2.0
    return expr


def test_lopsided_products_reach_their_kernels():
    rng = np.random.default_rng(17)
    kinds = set()
    for _ in range(40):
        plan = porch.plan(random_lopsided_product(rng, integer_leaf), compile=True)
        kinds.update(k["kind"] for k in plan["kernels"])
    assert {"gemm.rows", "gemm.cols", "gemm.narrow", "gemm.wide", "gemm.combine", "gemm.mfma"} <= kinds


@pytest.mark.gpu
def test_fuzz_lopsided_products_bit_exact(gpu):
    # integer leaves in [-3, 3]: |sums| <= 9 * 3000 < 2^24, exact in any order
    rng = np.random.default_rng(123)

    def device_leaf(shape, rng):
        values = rng.integers(-3, 4, size=int(np.prod(shape))).astype(np.float32)
        return gpu.tensor(shape, values)

    kinds = set()
    for trial in range(40):
        expr = random_lopsided_product(rng, device_leaf)
        plan = gpu.plan(expr)
        kinds.update(k["kind"] for k in plan["kernels"])
        print("lopsided product", trial, expr.shape(), [k["kind"] for k in plan["kernels"]], flush=True)
        ref = host.evaluate(expr)
        assert np.max(np.abs(ref)) < LIMIT
        out = gpu.materialize(expr).cpu().reshape(expr.shape())
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (trial, plan)
    assert {"gemm.rows", "gemm.cols", "gemm.narrow", "gemm.wide", "gemm.combine", "gemm.mfma"} <= kinds
