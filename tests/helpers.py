"""Shared test helpers: the KAT expression notation, host-only placeholder
tensors (graphs for the oracle and the planner without a GPU), and the five
benchmark graphs at any size."""

from __future__ import annotations

import json
import os

import numpy as np

import porch_amd as porch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def placeholder(shape, values=None) -> porch.tensor:
    """A tensor with host values and no device buffer (CPU-only graphs)."""
    t = porch.tensor.__new__(porch.tensor)
    t._state = porch._State(list(shape), porch.device())
    host = None
    if values is not None:
        host = np.ascontiguousarray(np.asarray(values, dtype=np.float32).reshape(-1))
    t._state.storage = porch._Storage(None, host)
    return t


def strided_placeholder(layout, storage_values) -> porch.tensor:
    """A host-only tensor over strided storage (the raw storage values)."""
    t = porch.tensor.__new__(porch.tensor)
    t._state = porch._State(list(layout.shape()), porch.device())
    host = np.ascontiguousarray(np.asarray(storage_values, dtype=np.float32).reshape(-1))
    t._state.storage = porch._Storage(None, host)
    if not layout.is_contiguous():
        t._state.layout = layout
    return t


def kat_cases():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        data = json.load(f)
    return data["cases"], data["errors"]


def kat_input_values(spec) -> np.ndarray:
    count = int(np.prod(spec["shape"]))
    if "values" in spec:
        values = np.asarray(spec["values"], dtype=np.float32)
    else:
        values = np.arange(spec["iota_from"], spec["iota_from"] + count, dtype=np.float32)
    for position, value in spec.get("set", []):
        values[position] = value
    return values


_BINARY = {"add": "__add__", "sub": "__sub__", "mul": "__mul__", "div": "__truediv__"}


def build(expr, inputs):
    """porch expression from the prefix notation over `inputs` (tensors)."""
    if isinstance(expr, (int, float)):
        return porch.tensor_expr(float(expr))
    op, *args = expr
    if op == "in":
        return porch.tensor_expr(inputs[args[0]])
    if op == "idx":
        items = []
        for item in args[1]:
            if item == "all":
                items.append(porch.all)
            elif isinstance(item, list):
                items.append(porch.slice(*item))
            else:
                items.append(item)
        return inputs[args[0]][tuple(items)]
    if op in _BINARY:
        lhs = build(args[0], inputs)
        rhs = build(args[1], inputs)
        return getattr(porch.tensor_expr(lhs), _BINARY[op])(rhs)
    if op in ("matmul", "maximum", "minimum"):
        return getattr(porch, op)(build(args[0], inputs), build(args[1], inputs))
    if op in ("exp", "reciprocal", "transpose", "relu", "logistic"):
        return getattr(porch, op)(build(args[0], inputs))
    if op == "reshape":
        return porch.reshape(build(args[0], inputs), args[1])
    if op == "broadcast":
        return porch.broadcast_to(build(args[0], inputs), args[1])
    if op == "unsqueeze":
        return porch.unsqueeze(build(args[0], inputs), args[1])
    if op == "concat":
        return porch.concat(build(args[0], inputs), build(args[1], inputs), args[2])
    if op in ("sum", "max"):
        return getattr(porch, op)(build(args[0], inputs), args[1], args[2])
    if op == "softmax":
        return porch.softmax(build(args[0], inputs), args[1])
    raise ValueError(f"unknown op {op}")


def check_kat(case, values: np.ndarray) -> None:
    values = np.asarray(values, dtype=np.float32).reshape(-1)
    if "exact" in case:
        expected = np.asarray(case["exact"], dtype=np.float32)
        assert values.shape == expected.shape, (values, expected)
        assert np.array_equal(values.view(np.uint32), expected.view(np.uint32)), (values, expected)
    for i, interval in enumerate(case.get("open", [])):
        if interval is None:
            continue
        lo, hi = interval
        assert lo < values[i] < hi, (case["name"], i, values[i])
    for position, value in case.get("eq", []):
        assert values[position] == np.float32(value), (case["name"], position, values[position])


from porch_amd.workloads import CONFIG_SIZES, config_graph, config_inputs, config_shapes  # noqa: E402,F401


def _ulps(a, b):
    ai = np.asarray(a, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi).reshape(np.shape(a))


def assert_softmax_close(out, t, values, rel=1e-6):
    """Softmax over the last axis of 2-D tensor `t` holding `values`, `out`
    computed by the kernels, against two references:

    1. the softmax of the same float32 differences x - max(x) with exp, sum
       and division in float64 (rows of finite values): within `rel`, or
       2 ulp where the result is far below the row max (tiny or denormal);
    2. the oracle: NaN exactly where it has NaN, elsewhere within `rel`
       plus the oracle's own row-sum drift.  The oracle sums in the
       reference's order, 256 float32 chains of L/256 terms each, so on long
       rows its sum drifts from the exact one (about 1.1e-6 relative at
       L = 262144, one part in 10^8 at L = 4096); a result summed more
       exactly differs from it by that much before any error of its own.
       The drift is measured per row: the oracle's sum of exp(x - max)
       against the float64 sum of the same terms."""
    from oracle import host

    shape = list(out.shape)
    rows, cols = shape
    ref = np.asarray(host.evaluate(porch.softmax(t, 1)), np.float32).reshape(shape)
    out = np.asarray(out, np.float32).reshape(shape)
    values = np.asarray(values, np.float32).reshape(shape)
    m = porch.broadcast_to(porch.max(t, 1, True), shape)
    oracle_sums = np.asarray(host.evaluate(porch.sum(porch.exp(t - m), 1)), np.float64).reshape(rows)

    finite_rows = np.isfinite(values).all(axis=1)
    with np.errstate(all="ignore"):
        d = (values - values.max(axis=1, keepdims=True)).astype(np.float32).astype(np.float64)
        e = np.exp(d)
        s = e.sum(axis=1, keepdims=True)
        truth = e / s
        drift = np.where(finite_rows, np.abs(oracle_sums / s[:, 0] - 1.0), 0.0)

    def rel_err(a, b):
        return np.abs(a.astype(np.float64) - b) / np.maximum(np.abs(b.astype(np.float64)), 1e-300)

    tr = truth[finite_rows]
    o = out[finite_rows]
    ok = (rel_err(o, tr) <= rel) | (_ulps(o, tr.astype(np.float32)) <= 2)
    assert ok.all(), ("vs float64", np.argwhere(~ok)[:5], o[~ok][:5], tr[~ok][:5])

    assert np.array_equal(np.isnan(out), np.isnan(ref))
    finite = ~np.isnan(ref)
    bar = np.broadcast_to((rel + drift)[:, None], shape)
    ok = (rel_err(out[finite], ref[finite]) <= bar[finite]) | (_ulps(out[finite], ref[finite]) <= 2)
    assert ok.all(), ("vs oracle", float(drift.max()), rel_err(out[finite], ref[finite]).max())


def check_matmul_epilogue_every_output(out, a, b, bias, m, k, n):
    """`out` = relu(A @ B + bias) - 0.5 over every one of its m x n outputs,
    against a float64 GEMM of the same float32 operands (the reference
    computes every output through its K loop, src/tensor.cpp:684-721):

    1. the product before the epilogue, recovered from the output where
       relu passed it (out + 0.5 is exact in float64): within the
       accumulation bound K * eps * sum_k |a_ik| |b_kj| plus the rounding of
       the final subtraction (half an ulp of 0.5); where relu clamped it
       (out == -0.5), the exact value is at most that bound above zero;
    2. the final result within 1e-4 relative, and 5e-6 absolute.

    Returns (max |delta| of the product, max |delta| / bound)."""
    am = np.asarray(a, np.float32).reshape(m, k).astype(np.float64)
    bm = np.asarray(b, np.float32).reshape(k, n).astype(np.float64)
    bias64 = np.asarray(bias, np.float32).reshape(1, n).astype(np.float64)
    out = np.asarray(out, np.float32).reshape(m, n)
    assert np.isfinite(out).all()
    exact_v = am @ bm + bias64
    bound = k * float(np.finfo(np.float32).eps) * (np.abs(am) @ np.abs(bm)) + np.abs(bias64) * 2.0 ** -23
    half_ulp = 2.0 ** -25
    o64 = out.astype(np.float64)
    passed = o64 > -0.5
    v = o64 + 0.5
    delta = np.where(passed, np.abs(v - exact_v), np.maximum(exact_v, 0.0))
    frac = delta / (bound + half_ulp)
    assert np.all(frac <= 1.0), (float(frac.max()), np.unravel_index(frac.argmax(), frac.shape))
    assert np.all(o64 >= -0.5)
    exact = np.maximum(exact_v, 0.0) - 0.5
    err = np.abs(o64 - exact)
    rel = err / np.maximum(np.abs(exact), 1e-30)
    assert rel.max() <= 1e-4, (float(rel.max()), np.unravel_index(rel.argmax(), rel.shape))
    assert err.max() < 5e-6, float(err.max())
    return float(delta.max()), float(frac.max())


def division_operands(count, seed):
    """float32 pairs (l, r) for division: edge operands first (signed
    zeros, infinities, NaN, the smallest and largest denormals and normals,
    FLT_MAX, quotients that overflow to infinity or underflow into the
    denormals or to zero, exact quotients), every pairing of a set of
    specials, then random values of log-uniform magnitude over the whole
    binary32 range with random signs."""
    f = np.float32
    tiny, dmax = f(np.finfo(np.float32).smallest_subnormal), f(np.finfo(np.float32).tiny) - f(np.finfo(np.float32).smallest_subnormal)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 3.0, tiny, -tiny, dmax,
                         np.finfo(np.float32).tiny, np.finfo(np.float32).max, -np.finfo(np.float32).max,
                         1e-30, 7e37], np.float32)
    pl, pr = np.meshgrid(specials, specials, indexing="ij")
    fixed_l = [f(1e38), f(1e-38), f(3e-39), f(6.0), f(1.0), f(1.0), f(2.0), f(1e-45), f(5e-39)]
    fixed_r = [f(1e-5), f(1e5), f(7.0), f(3.0), f(3.0), f(0.1), f(3.0 ** 10), f(2.0), f(0.5)]
    rng = np.random.default_rng(seed)
    n = max(count - pl.size - len(fixed_l), 0)

    def random_values(k):
        bits = rng.integers(0, 0xFF, k, dtype=np.uint32) << np.uint32(23)
        bits |= rng.integers(0, 1 << 23, k, dtype=np.uint32)
        bits |= rng.integers(0, 2, k, dtype=np.uint32) << np.uint32(31)
        return bits.view(np.float32)

    lhs = np.concatenate([pl.reshape(-1), np.array(fixed_l, np.float32), random_values(n)])
    rhs = np.concatenate([pr.reshape(-1), np.array(fixed_r, np.float32), random_values(n)])
    return lhs[:count].astype(np.float32), rhs[:count].astype(np.float32)


def assert_bits_or_both_nan(got, expected):
    """Bit-for-bit equality, except that any NaN matches any NaN."""
    got = np.asarray(got, np.float32).reshape(-1)
    expected = np.asarray(expected, np.float32).reshape(-1)
    assert got.shape == expected.shape
    both_nan = np.isnan(got) & np.isnan(expected)
    bad = (got.view(np.uint32) != expected.view(np.uint32)) & ~both_nan
    idx = np.flatnonzero(bad)
    assert idx.size == 0, (idx.size, idx[:6], got[idx[:6]], expected[idx[:6]])
