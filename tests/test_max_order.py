"""Max reductions give the reference's result on rows holding NaN, signed
zeros and -inf, where the order of the reduction decides the result.

The reference reduces each output with one 256-thread block
(src/tensor.cpp:896-962): thread t folds axis positions t, t + 256, ... with
`t = t > v ? t : v` from -FLT_MAX (849-851), then a shared-memory tree with
strides 128, 64, ..., 1 combines the partials the same way.  That step keeps
a NaN only as its right operand and gives a +0/-0 tie to the right operand,
so which NaN survives, and the sign of a zero maximum, depend on positions.

The kernels fold with an order-free maximum (NaN-propagating, -0 < +0) and
recompute, in the reference's order, every output whose order-free result is
NaN or +0, the only values for which the order can matter.

* CPU: the oracle's max is pinned against a closed form of the reference's
  order stated independently (below); the generated kernels, run on the CPU
  by tests/kernel_emu, match the oracle bit for bit on such rows, with and
  without the order-free result forcing the exact path.
* GPU: every kernel form that reduces with max (wave, segment and workgroup
  rows, rows beyond the register cache, column and split-column reductions)
  matches the oracle bit for bit on such rows; NaN payloads are not compared
  (they are not part of the reference's semantics, and the reference's own
  NaN bits come from NVIDIA hardware).
"""

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import assert_softmax_close, placeholder
from tests.kernel_emu import emulate as emu

FLT_MAX = np.float32(3.4028234663852886e38)


# -- a closed form of the reference's block max ------------------------------

def _rightmost_maximum(values):
    """The last element among those equal to the largest (NaN-free)."""
    values = np.asarray(values, np.float32)
    top = values.max()
    return values[np.flatnonzero(values == top)[-1]]


def closed_form_block_max(row) -> np.float32:
    """The reference's block max, stated without its loops.

    A fold left-to-right with `t > v ? t : v` keeps NaN only from its last
    step, and a NaN accumulator is replaced by the next value: a thread's
    partial is NaN if its last value is, and otherwise the rightmost maximum
    of what follows its last NaN (of -FLT_MAX and all its values if it has
    none).  In the tree, thread t sits at in-order position k = bitrev8(t)
    (the root splits on bit 0, the leaves pair on bit 7); a subtree is NaN
    exactly when its rightmost leaf is, a NaN subtree that is a left child
    is discarded, so a NaN leaf at position k discards the 2^j positions
    ending at k, j being the number of trailing one bits of k.  The result
    is NaN if position 255 is, else the rightmost maximum of the leaves
    left."""
    row = np.asarray(row, np.float32)
    partial = np.empty(256, np.float32)
    for t in range(256):
        seq = row[t::256]
        if seq.size and np.isnan(seq[-1]):
            partial[t] = np.nan
            continue
        nans = np.flatnonzero(np.isnan(seq))
        rest = seq[nans[-1] + 1:] if nans.size else np.concatenate([[-FLT_MAX], seq])
        partial[t] = _rightmost_maximum(rest)
    leaves = np.array([partial[int(f"{k:08b}"[::-1], 2)] for k in range(256)], np.float32)
    if np.isnan(leaves[255]):
        return np.float32(np.nan)
    keep = np.ones(256, bool)
    for k in np.flatnonzero(np.isnan(leaves)):
        ones = 0
        while (k >> ones) & 1:
            ones += 1
        keep[k - (1 << ones) + 1: k + 1] = False
    return _rightmost_maximum(leaves[keep])


def special_rows(rows: int, cols: int, seed: int) -> np.ndarray:
    """Rows whose block max depends on the reduction order, mixed with
    plain ones: NaN at random positions, at the end, at a virtual thread's
    last element; +0/-0 ties below negative values; all -inf; all zeros."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    for r in range(rows):
        kind = r % 10
        if kind == 0:
            x[r, rng.integers(cols)] = np.nan
        elif kind == 1:
            x[r] = -np.abs(x[r])
            x[r, rng.integers(cols, size=3)] = 0.0
            x[r, rng.integers(cols, size=3)] = -0.0
        elif kind == 2:
            x[r] = -np.inf
        elif kind == 3:
            x[r, rng.integers(cols, size=min(cols, 7))] = np.nan
        elif kind == 4:
            x[r, cols - 1] = np.nan
        elif kind == 5:
            x[r] = np.where(rng.random(cols) < 0.5, np.float32(0.0), np.float32(-0.0))
        elif kind == 6:
            # NaN as the last element of virtual thread 255, then of thread 254
            x[r, max(cols - 1 - (cols - 1) % 256 + 255, 0) % cols] = np.nan
            x[r, rng.integers(cols)] = -0.0
        elif kind == 7:
            x[r] = -np.abs(x[r])
            x[r, rng.integers(cols)] = np.nan
            x[r, rng.integers(cols, size=2)] = 0.0
        elif kind == 8:
            x[r, rng.integers(cols, size=min(cols, 40))] = np.nan
    return x


def same_or_both_nan(a, b) -> bool:
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    return a.shape == b.shape and bool(np.all((np.isnan(a) & np.isnan(b)) |
                                              (a.view(np.uint32) == b.view(np.uint32))))


def mismatches(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    bad = np.flatnonzero(~((np.isnan(a) & np.isnan(b)) | (a.view(np.uint32) == b.view(np.uint32))))
    return bad[:8], a[bad[:8]], b[bad[:8]]


@pytest.mark.parametrize("cols", [1, 3, 255, 256, 257, 700, 4096])
def test_oracle_max_matches_the_closed_form(cols):
    x = special_rows(40, cols, seed=cols)
    ref = host.evaluate(porch.max(placeholder(x.shape, x), 1, False))
    for r in range(x.shape[0]):
        assert same_or_both_nan(ref[r], closed_form_block_max(x[r])), (r, ref[r], closed_form_block_max(x[r]))


def test_position_decides_the_reference_max():
    """The rows above do exercise the order: an order-free NaN-propagating
    max (or one that ignores NaN) disagrees with the oracle on some."""
    x = special_rows(60, 700, seed=5)
    ref = host.evaluate(porch.max(placeholder(x.shape, x), 1, False))
    propagating = np.where(np.isnan(x).any(axis=1), np.nan, np.nanmax(np.where(np.isnan(x), -np.inf, x), axis=1))
    ignoring = np.nanmax(np.where(np.isnan(x), -np.inf, x), axis=1)
    assert not same_or_both_nan(ref, propagating.astype(np.float32))
    assert not same_or_both_nan(ref, ignoring.astype(np.float32))
    # and the sign of a zero maximum follows the positions of the zeros: a
    # tie goes to the thread at the later in-order position of the tree,
    # bitrev8(t): thread 3 (position 192) beats thread 200 (position 19)
    row = np.full(300, -1.0, np.float32)
    row[[3, 200]] = [0.0, -0.0]
    assert not np.signbit(closed_form_block_max(row))
    assert not np.signbit(host.evaluate(porch.max(placeholder([1, 300], row), 1, False))[0])
    row[[3, 200]] = [-0.0, 0.0]
    assert np.signbit(closed_form_block_max(row))
    assert np.signbit(host.evaluate(porch.max(placeholder([1, 300], row), 1, False))[0])
    # within a thread the later value wins: positions 3 and 259 are both thread 3
    row[[3, 200, 259]] = [0.0, -1.0, -0.0]
    assert np.signbit(closed_form_block_max(row))
    assert np.signbit(host.evaluate(porch.max(placeholder([1, 300], row), 1, False))[0])


# -- the graphs: every kernel form that reduces with max -------------------

def _row_max(x):
    return porch.max(x, len(x.shape()) - 1, False)


def _minus_row_max(x):
    shape = list(x.shape())
    return x - porch.broadcast_to(porch.max(x, len(shape) - 1, True), shape)


CASES = [
    # (shape of the rows [rows, cols], graph, kernel form)
    ([20, 4096], _row_max, "workgroup row"),
    ([10, 2048], _minus_row_max, "workgroup row, cached"),
    ([20, 1000], _minus_row_max, "wave row"),
    ([20, 1999], _row_max, "wave row, ragged"),
    ([40, 64], _minus_row_max, "16-lane segments"),
    ([40, 3], _row_max, "1-lane segments"),
    ([30, 17], _minus_row_max, "8-lane segments, scalar"),
    ([4, 33000], _row_max, "8-wave workgroup row"),
    ([3, 65536], _minus_row_max, "16-wave workgroup row"),
    ([2, 262148], _row_max, "row beyond the register cache"),
]

COLUMN_CASES = [
    # (shape, axis) of a max over a non-last axis
    ([300, 12], 0),
    ([3, 500, 7], 1),
    ([1000, 3], 0),
    ([262144, 8], 0),  # split over the axis: partials, then a second pass
]


def _column_input(shape, axis, seed):
    """special_rows laid along `axis`."""
    extent = shape[axis]
    others = int(np.prod(shape)) // extent
    rows = special_rows(others, extent, seed)
    moved = [s for d, s in enumerate(shape) if d != axis] + [extent]
    return np.ascontiguousarray(np.moveaxis(rows.reshape(moved), -1, axis))


def _kernels(expr):
    return [k["kind"] + (" split" if k["grid"][1] > 1 else "") for k in porch.plan(expr)["kernels"]]


@pytest.mark.skipif(not emu.available(), reason="host clang++ from ROCm is required")
@pytest.mark.parametrize("shape, graph, form", [c for c in CASES if c[0][1] <= 4096])
def test_emulated_kernels_match_the_oracle(shape, graph, form):
    x = special_rows(*shape, seed=shape[1])
    expr = graph(placeholder(shape, x))
    ref = host.evaluate(expr)
    assert same_or_both_nan(emu.evaluate(expr, [x]), ref), (form, mismatches(emu.evaluate(expr, [x]), ref))
    # the path in the reference's order alone gives the same result
    assert same_or_both_nan(emu.evaluate(expr, [x], force_exact=True), ref), form


@pytest.mark.skipif(not emu.available(), reason="host clang++ from ROCm is required")
@pytest.mark.parametrize("shape, axis", COLUMN_CASES[:3])
def test_emulated_column_kernels_match_the_oracle(shape, axis):
    x = _column_input(shape, axis, seed=shape[axis])
    expr = porch.max(placeholder(shape, x), axis, False)
    ref = host.evaluate(expr)
    assert same_or_both_nan(emu.evaluate(expr, [x]), ref)
    assert same_or_both_nan(emu.evaluate(expr, [x], force_exact=True), ref)


@pytest.mark.gpu
@pytest.mark.parametrize("shape, graph, form", CASES)
def test_row_max_matches_the_oracle_on_gpu(gpu, shape, graph, form):
    x = special_rows(*shape, seed=shape[1] + 1)
    expr = graph(gpu.tensor(shape, x))
    out = gpu.materialize(expr).cpu().reshape(expr.shape())
    ref = host.evaluate(expr)
    assert same_or_both_nan(out, ref), (form, mismatches(out, ref))


@pytest.mark.gpu
@pytest.mark.parametrize("shape, axis", COLUMN_CASES)
@pytest.mark.parametrize("keepdim", [False, True])
def test_column_max_matches_the_oracle_on_gpu(gpu, shape, axis, keepdim):
    x = _column_input(shape, axis, seed=shape[axis] + 2)
    expr = gpu.max(gpu.tensor(shape, x), axis, keepdim)
    if shape[axis] == 262144:
        assert _kernels(expr) == ["reduce.column split", "reduce.column"]
    out = gpu.materialize(expr).cpu().reshape(expr.shape())
    ref = host.evaluate(expr)
    assert same_or_both_nan(out, ref), mismatches(out, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [[40, 64], [20, 1000], [20, 4096], [2, 262148]])
def test_softmax_of_special_rows_matches_the_oracle_on_gpu(gpu, shape):
    """Softmax over the same rows: NaN exactly where the oracle has NaN,
    elsewhere within 1e-6 relative (beyond the oracle's own row-sum drift:
    assert_softmax_close)."""
    x = special_rows(*shape, seed=shape[1] + 3)
    t = gpu.tensor(shape, x)
    out = gpu.materialize(gpu.softmax(t, 1)).cpu().reshape(shape)
    assert_softmax_close(out, t, x)


@pytest.mark.gpu
def test_two_element_rows_on_gpu(gpu):
    """Rows of two: element i is thread i's only value, and thread 1 sits at
    position 128 of the tree.  [nan, 1] and [1, nan] both give 1 (thread
    1's NaN is a left child where it meets positions 129-255), [0, -0]
    gives -0 and [-0, 0] gives +0 (the tie goes to position 128); a NaN
    survives only from position 255, thread 255."""
    porch = gpu
    rows = np.array([[np.nan, 1.0], [1.0, np.nan], [0.0, -0.0], [-0.0, 0.0]], np.float32)
    out = porch.materialize(porch.max(porch.tensor([4, 2], rows), 1)).cpu()
    for r in range(4):
        assert same_or_both_nan(out[r], closed_form_block_max(rows[r])), (r, out[r])
    assert out[0] == 1.0 and out[1] == 1.0
    assert out[2] == 0.0 and np.signbit(out[2]) and out[3] == 0.0 and not np.signbit(out[3])
    last = np.zeros((2, 256), np.float32)
    last[0, 255] = np.nan
    last[1, 254] = np.nan
    out = porch.materialize(porch.max(porch.tensor([2, 256], last), 1)).cpu()
    assert np.isnan(out[0]) and out[1] == 0.0
