"""Division on general operands, bit for bit against the oracle.

The reference emits `(l / r)` for divide and `(1.0f / x)` for reciprocal
(src/tensor.cpp:659-667,864) under NVRTC's default IEEE division; the
oracle's DIVIDE and RECIPROCAL are pinned to numpy's correctly rounded
binary32 division in tests/test_oracle.py.  Here the kernels' quotients
are compared with the oracle's bit for bit (NaN as NaN) over the same edge
and random operands (signed zeros, infinities, NaN, denormals, overflowing
and underflowing quotients, random operands over the whole binary32
range), in each kernel class that evaluates a quotient: the flat
pointwise kernel, the LDS-tiled transpose kernel, the row program (the
quotient and its row max in one pass) and the column reduction.
"""

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import assert_bits_or_both_nan, division_operands

pytestmark = pytest.mark.gpu

ROWS, COLS = 256, 1024


def _kinds(expr):
    return [k["kind"] for k in porch.plan(expr)["kernels"]]


@pytest.fixture(scope="module")
def operands():
    lhs, rhs = division_operands(ROWS * COLS, 11)
    return lhs.reshape(ROWS, COLS), rhs.reshape(ROWS, COLS)


def _check(gpu, expr, kind):
    assert kind in _kinds(expr), _kinds(expr)
    print("divide:", kind, expr.shape(), flush=True)
    out = gpu.materialize(expr).cpu()
    assert_bits_or_both_nan(out, host.evaluate(expr))


def test_tensor_by_tensor_flat(gpu, operands):
    lhs, rhs = operands
    tl, tr = gpu.tensor([ROWS, COLS], lhs), gpu.tensor([ROWS, COLS], rhs)
    _check(gpu, tl / tr, "pointwise.flat")
    _check(gpu, gpu.reciprocal(tr), "pointwise.flat")
    # against numpy as well: the oracle's quotient is numpy's
    with np.errstate(all="ignore"):
        assert_bits_or_both_nan(gpu.materialize(tl / tr).cpu(), np.divide(lhs, rhs, dtype=np.float32))


def test_tensor_by_broadcast_row(gpu, operands):
    lhs, rhs = operands
    tl = gpu.tensor([ROWS, COLS], lhs)
    row = gpu.tensor([1, COLS], rhs[:1])
    _check(gpu, tl / gpu.broadcast_to(row, [ROWS, COLS]), "pointwise.flat")
    _check(gpu, gpu.broadcast_to(row, [ROWS, COLS]) / tl, "pointwise.flat")


def test_transposed_operand_tiled(gpu, operands):
    lhs, rhs = operands
    tt = gpu.tensor([COLS, ROWS], np.ascontiguousarray(lhs.reshape(-1).reshape(COLS, ROWS)))
    tr = gpu.tensor([ROWS, COLS], rhs)
    _check(gpu, gpu.transpose(tt) / tr, "pointwise.tiled")
    _check(gpu, tr / gpu.transpose(tt), "pointwise.tiled")


def test_quotient_in_the_row_program(gpu, operands):
    # q - max(q) per row: the row program evaluates each quotient once for
    # its max and again for the output; subtraction and max are exact, so
    # the result's bits are the quotient's
    lhs, rhs = operands
    tl, tr = gpu.tensor([ROWS, COLS], lhs), gpu.tensor([ROWS, COLS], rhs)
    q = tl / tr
    _check(gpu, q - gpu.broadcast_to(gpu.max(q, 1, True), [ROWS, COLS]), "row")


def test_quotient_in_a_column_reduction(gpu, operands):
    lhs, rhs = operands
    tl = gpu.tensor([ROWS, COLS], lhs)
    row = gpu.tensor([1, COLS], rhs[:1])
    _check(gpu, gpu.max(tl / gpu.broadcast_to(row, [ROWS, COLS]), 0, True), "reduce.column")
