"""Reductions over the last axis into few outputs (kernel kinds row.partial
and row.combine): a full sum of a long vector, a max over a few long rows.

Each row is split into pieces; one kernel folds every (row, piece) into a
partial, a second folds each row's partials.  Sums: exact where every
partial sum is exact (integer data), otherwise within 1e-6 of the sum of
absolute values of a float64 sum.  Max: bit for bit the oracle's, NaN and
signed zeros included (the reference's block order is recomputed where the
order-free max may differ).  CPU: the planner's choice, bounds and values of
the kernels run on the CPU.  GPU: the same against the oracle at full size.
"""

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import placeholder
from tests.kernel_emu import emulate as emu
from tests.test_max_order import mismatches, same_or_both_nan, special_rows

needs_clang = pytest.mark.skipif(not emu.available(), reason="host clang++ from ROCm is required")


def _kinds(expr):
    return [k["kind"] for k in porch.plan(expr)["kernels"]]


def full_sum(t, n):
    return porch.sum(porch.reshape(t, [n]), 0)


@pytest.mark.parametrize("build, temps", [
    (lambda: full_sum(placeholder([8192, 8192]), 8192 * 8192), [1024]),
    (lambda: porch.max(placeholder([3, 1000000]), 1), [3 * 123]),
    (lambda: porch.sum(porch.exp(placeholder([2, 3, 100000])), 2), [6 * 13]),
    (lambda: porch.sum(placeholder([5, 100003]), 1, True), [5 * 13]),  # odd length: scalar reads
])
def test_few_long_rows_are_split(build, temps):
    expr = build()
    plan = porch.plan(expr, compile=True)
    assert _kinds(expr) == ["row.partial", "row.combine"]
    assert plan["temps"] == temps
    assert plan["kernels"][0]["dest"] == "temp0" and plan["kernels"][1]["dest"] == "output"


@pytest.mark.parametrize("build", [
    lambda: porch.sum(placeholder([512, 131072]), 1),   # rows fill the machine
    lambda: porch.sum(placeholder([4, 20000]), 1),      # short rows
    lambda: porch.softmax(placeholder([2, 262144]), 1),  # not a single fold
])
def test_other_reductions_are_not_split(build):
    assert not {"row.partial", "row.combine"} & set(_kinds(build()))


@needs_clang
@pytest.mark.parametrize("shape", [[2, 65536], [3, 40003]])
def test_emulated_sums_are_exact_on_integer_data(shape):
    x = np.random.default_rng(shape[1]).integers(-4, 5, size=shape).astype(np.float32)
    expr = porch.sum(placeholder(shape, x), 1)
    assert _kinds(expr) == ["row.partial", "row.combine"]
    assert all(r["ok"] for r in emu.emulate(expr))
    got = emu.evaluate(expr, [x])
    assert np.array_equal(got, x.astype(np.float64).sum(axis=1).astype(np.float32))


@needs_clang
def test_emulated_max_takes_the_reference_order():
    shape = [10, 40000]
    x = special_rows(*shape, seed=4)
    expr = porch.max(placeholder(shape, x), 1)
    assert _kinds(expr) == ["row.partial", "row.combine"]
    ref = host.evaluate(expr)
    assert same_or_both_nan(emu.evaluate(expr, [x]), ref), mismatches(emu.evaluate(expr, [x]), ref)
    assert same_or_both_nan(emu.evaluate(expr, [x], force_exact=True), ref)


# -- GPU -----------------------------------------------------------------------


@pytest.mark.gpu
def test_full_sum_of_a_long_vector(gpu):
    n = 8192 * 8192
    rng = np.random.default_rng(3)
    # {0, 1} with density 1/8: every partial sum and the total (< 2^24)
    # are exact, whatever the order
    ones = (rng.random(n) < 0.125).astype(np.float32)
    expr = full_sum(gpu.tensor([n], ones), n)
    assert _kinds(expr) == ["row.partial", "row.combine"]
    out = gpu.materialize(expr).cpu()
    assert out.reshape(-1)[0] == np.float32(ones.sum(dtype=np.float64))
    assert np.array_equal(out, host.evaluate(expr))
    # normal data: within 1e-6 of sum |x| of the float64 sum
    x = rng.standard_normal(n).astype(np.float32)
    out = gpu.materialize(full_sum(gpu.tensor([n], x), n)).cpu().reshape(-1)[0]
    exact = x.astype(np.float64).sum()
    assert abs(float(out) - exact) <= 1e-6 * np.abs(x.astype(np.float64)).sum()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [[3, 1000000], [10, 300001]])
def test_max_over_few_long_rows(gpu, shape):
    x = special_rows(*shape, seed=shape[1] % 97)
    expr = gpu.max(gpu.tensor(shape, x), 1)
    assert _kinds(expr) == ["row.partial", "row.combine"]
    out = gpu.materialize(expr).cpu().reshape(-1)
    ref = host.evaluate(expr)
    assert same_or_both_nan(out, ref), mismatches(out, ref)


@pytest.mark.gpu
def test_sum_of_an_expression_over_few_rows(gpu):
    shape = [2, 3, 100000]
    x = (np.random.default_rng(5).standard_normal(shape)).astype(np.float32)
    expr = gpu.sum(gpu.exp(gpu.tensor(shape, x) * 0.5), 2)
    assert _kinds(expr) == ["row.partial", "row.combine"]
    out = gpu.materialize(expr).cpu().reshape(-1).astype(np.float64)
    exact = np.exp(x.astype(np.float64) * 0.5).sum(axis=2).reshape(-1)
    assert np.all(np.abs(out - exact) <= 2e-6 * exact), np.abs(out - exact) / exact
