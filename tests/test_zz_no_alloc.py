"""porch_materialize_noalloc (libporch_amd_noalloc.so) against
porch_materialize and against the oracle, through the C ABI.

The allocation-free entry point runs the same kernels, with the graph's
temporaries in a fixed per-GPU device array instead of fresh allocations.
Checked on two calls in a row for each graph, the second with a smaller
input (the array keeps the first call's contents, so a temporary read
before it is written would show):

* no allocation: across a call made after one warm-up call for the same
  graph structure, the runtime's counts of hipMallocAsync, hipFreeAsync,
  hipHostMalloc, hipHostFree and hipModuleLoadData calls do not change;
* the results equal porch_materialize's bit for bit (NaN as NaN), except
  for split softmax rows, whose sums depend on which parts finish their
  bounded wait in time: those are held to 1e-6 relative;
* the results meet the oracle's bars: bit-exact for the elementwise graph
  and the column max, 1e-6 for the softmaxes (with the float64 check of
  assert_softmax_close for the split rows), 1e-5 for the nested reduction,
  and for the product (whose results pass through zero) the accumulation
  bound against a float64 product.

Graphs with temporaries of every kind: split column reductions (partials),
memoised reductions, a materialised product operand, split softmax rows
(exchange words that a fill kernel must zero before each launch); and one
without.  Sizes past the array's limit, and an output buffer too small,
are rejected before any launch.
"""

import ctypes

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from porch_amd import _lib
from tests.helpers import assert_softmax_close

pytestmark = pytest.mark.gpu

LIMIT = 64 << 20  # PORCH_NOALLOC_SCRATCH_BYTES


ALLOCATION_CALLS = ("device_allocs", "device_frees", "host_allocs", "host_frees", "module_loads")


def allocation_calls():
    stats = porch.jit_stats()
    return {name: stats[name] for name in ALLOCATION_CALLS}


def call_noalloc(expr, out_floats=None, calls=None):
    """(status, error message, output values, shape written) of
    porch_materialize_noalloc into a NaN-filled buffer of `out_floats`
    (default: the result's size).  With `calls` a dict, stores there how
    many allocation calls the runtime made during the call and the stream
    synchronisation after it."""
    nodes, dims, n_dims, inputs, _ = porch.serialize(expr._root)
    g = porch._graph(nodes, dims, n_dims)
    handles = (ctypes.c_void_p * max(len(inputs), 1))(
        *[t._state.realized().buffer.handle for t in inputs])
    count = int(np.prod(expr.shape()))
    size = count if out_floats is None else out_floats
    out = porch._Buffer.upload(np.full(size, np.nan, np.float32))
    shape = (ctypes.c_int64 * 64)()
    rank = ctypes.c_int32()
    porch.synchronize()
    before = allocation_calls()
    status = _lib.noalloc_lib().porch_materialize_noalloc(
        ctypes.byref(g), handles, len(inputs), out.handle, shape, 64, ctypes.byref(rank))
    message = porch.lib.porch_last_error().decode()  # before later calls clear it
    porch.synchronize()
    if calls is not None:
        after = allocation_calls()
        calls.update({name: after[name] - before[name] for name in ALLOCATION_CALLS})
    return status, message, out.download(size), [shape[i] for i in range(rank.value)]


def noalloc(expr, calls=None):
    status, message, values, shape = call_noalloc(expr, calls=calls)
    assert status == _lib.OK, message
    assert shape == list(expr.shape())
    return values.reshape(expr.shape())


def assert_same(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    same = (np.isnan(a) & np.isnan(b)) | (a.view(np.uint32) == b.view(np.uint32))
    assert same.all(), (np.flatnonzero(~same)[:8], a[~same][:8], b[~same][:8])


def rand(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(int(np.prod(shape))) * scale).astype(np.float32)


def softmax_first_axis(shape, seed):
    return porch.softmax(porch.tensor(shape, rand(shape, seed, 3.0)), 0)


def split_softmax_rows(shape, seed):
    # rows split over workgroups: a zeroed exchange temporary, then the rows
    return porch.softmax(porch.tensor(shape, rand(shape, seed, 3.0)), 1)


def split_column_max(shape, seed):
    return porch.max(porch.tensor(shape, rand(shape, seed)), 0, False)


def product_of_expression(m, k, n, seed):
    a = porch.tensor([m, k], rand([m, k], seed))
    b = porch.tensor([k, n], rand([k, n], seed + 1))
    return porch.relu(porch.matmul(porch.relu(a), b) + 1.0)


def nested_reduction(shape, seed):
    x = porch.tensor(shape, rand(shape, seed))
    return porch.sum(x - porch.broadcast_to(porch.max(x, 0, True), shape), 1, False)


def elementwise(n, seed):
    a = porch.tensor([n], rand([n], seed))
    return (a + 1.0) * 2.0 - 1.0


def check_against_oracle(name, expr, out, args, seed):
    if name == "product of an expression":
        # relu(relu(a) @ b + 1) against float64, within the accumulation
        # bound (the result passes through zero, so no relative bar)
        m, k, n = args
        a = np.maximum(rand([m, k], seed), 0).reshape(m, k).astype(np.float64)
        b = rand([k, n], seed + 1).reshape(k, n).astype(np.float64)
        v = a @ b + 1.0
        eps = float(np.finfo(np.float32).eps)
        bound = k * eps * (a @ np.abs(b)) + eps * (np.abs(v) + 1.0)
        assert np.all(np.abs(out.reshape(m, n) - np.maximum(v, 0.0)) <= bound)
        ref = np.asarray(host.evaluate(expr), np.float32).reshape(m, n)
        assert np.all(np.abs(ref - np.maximum(v, 0.0)) <= bound)
        return
    if name == "split softmax rows":
        (t,) = [n.input for n in _inputs(expr)]
        assert_softmax_close(out.reshape(expr.shape()), t, t.cpu())
        return
    ref = np.asarray(host.evaluate(expr), np.float32).reshape(-1)
    out = np.asarray(out, np.float32).reshape(-1)
    bar = BARS[name]
    if bar == 0:
        assert_same(out, ref)
        return
    err = np.abs(out.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)), 1e-30)
    assert err.max() <= bar, (name, err.max())


def _inputs(expr):
    nodes, seen, stack = [], set(), [expr._root]
    while stack:
        n = stack.pop()
        if n is None or id(n) in seen:
            continue
        seen.add(id(n))
        if n.kind == "input":
            nodes.append(n)
        stack += [n.lhs, n.rhs]
    return nodes


CASES = {
    # name: (graph builder, first call's arguments, second call's (smaller)
    # arguments, kernels of each call)
    "softmax over the first axis": (softmax_first_axis, ([6000, 200],), ([3000, 100],), (3, 2)),
    "split column max": (split_column_max, ([262144, 8],), ([131072, 8],), (2, 2)),
    "split softmax rows": (split_softmax_rows, ([40, 131072],), ([9, 65540],), (2, 2)),
    "product of an expression": (product_of_expression, (512, 256, 384), (200, 96, 136), (2, 2)),
    "nested reduction": (nested_reduction, ([300, 500],), ([70, 30],), (2, 2)),
    "no temporaries": (elementwise, (1 << 20,), (1000,), (1, 1)),
}

# the oracle's bar for each graph (0: bit for bit)
BARS = {
    "softmax over the first axis": 1e-6,
    "split column max": 0,
    "split softmax rows": 1e-6,
    "product of an expression": None,  # the accumulation bound instead
    "nested reduction": 1e-5,
    "no temporaries": 0,
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_matches_materialize_on_two_calls(gpu, name):
    build, first, second, kernels = CASES[name]
    for seed, args, count in ((11, first, kernels[0]), (12, second, kernels[1])):
        expr = build(*args, seed)
        plan = porch.plan(expr)
        assert len(plan["kernels"]) == count, plan
        assert (count > 1) == bool(plan["temps"])
        expected = porch.materialize(expr).cpu().reshape(expr.shape())
        warm = noalloc(expr)
        # and again on the same array contents, with no allocation at all
        calls = {}
        again = noalloc(expr, calls)
        assert all(v == 0 for v in calls.values()), (name, args, calls)
        for out in (warm, again):
            if name == "split softmax rows":
                np.testing.assert_allclose(out, expected, rtol=1e-6, atol=0)
            else:
                assert_same(out, expected)
        check_against_oracle(name, expr, again, args, seed)


def test_counts_see_allocations(gpu):
    """The counters the test above relies on move when the runtime
    allocates: with the allocator's cache emptied (which frees its blocks),
    porch_materialize of a large result allocates its output, and a plan
    compiled for the first time loads a module."""
    x = porch.tensor([3, 1 << 22], rand([3, 1 << 22], 51))
    porch.synchronize()
    cached = porch.release_cached_memory()
    before = allocation_calls()
    r = porch.materialize(x * 3.0 + 7.25)
    r.synchronize()
    after = allocation_calls()
    assert after["device_allocs"] > before["device_allocs"], (before, after)
    assert after["module_loads"] > before["module_loads"], (before, after)
    # releasing the result caches its block; emptying the cache frees it
    del r
    porch.synchronize()
    assert porch.release_cached_memory() >= 3 * 4 * (1 << 22)
    assert allocation_calls()["device_frees"] > after["device_frees"]
    assert cached >= 0


def test_uses_the_fixed_array_for_temporaries(gpu):
    """Two different graphs in turn on the same array: the second's
    temporaries overwrite the first's, and both stay exact."""
    a = split_column_max([262144, 8], 21)
    b = softmax_first_axis([4000, 64], 22)
    ra, rb = porch.materialize(a).cpu(), porch.materialize(b).cpu()
    for _ in range(2):
        assert_same(noalloc(a), ra)
        assert_same(noalloc(b), rb)


def test_rejects_temporaries_beyond_the_limit(gpu):
    expr = product_of_expression(4200, 4096, 64, 31)  # relu(a) is a 68.8 MB temporary
    need = sum(max(t, 1) * 4 for t in porch.plan(expr)["temps"])
    assert need > LIMIT
    status, message, values, _ = call_noalloc(expr)
    assert status == _lib.ERR_INVALID_ARGUMENT
    assert "PORCH_NOALLOC_SCRATCH_BYTES" in message and str(need) in message, message
    assert np.isnan(values).all()  # nothing ran


def test_rejects_a_short_output_buffer(gpu):
    expr = elementwise(4096, 41)
    status, message, values, _ = call_noalloc(expr, out_floats=4095)
    assert status == _lib.ERR_INVALID_ARGUMENT
    assert "too small" in message, message
    assert np.isnan(values).all()
