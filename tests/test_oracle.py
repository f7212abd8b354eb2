"""Pins the host evaluator (the oracle) before results are compared against it.

Checks: every known-answer vector of the reference's tests, and — where
those leave room — independent statements of the result (numpy slicing for
view chains, float64 evaluations for the arithmetic), invariants (softmax
rows sum to 1, order-free exact integer sums), and planted mistakes that the
same checks must reject.  CPU only.
"""

import math

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import (assert_bits_or_both_nan, build, check_kat, config_graph, config_inputs, config_shapes,
                           division_operands, kat_cases, kat_input_values, placeholder)

CASES, ERRORS = kat_cases()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_reference_kats(case):
    tensors = [placeholder(spec["shape"], kat_input_values(spec)) for spec in case["inputs"]]
    expr = build(case["expr"], tensors)
    assert expr.shape() == case["shape"]
    values = host.evaluate(expr)
    check_kat(case, values)


def oracle_of(name, size, inputs=None):
    shapes = config_shapes(name, size)
    inputs = inputs if inputs is not None else config_inputs(name, size)
    tensors = [placeholder(s, v) for s, v in zip(shapes, inputs)]
    return host.evaluate(config_graph(name, tensors, size)), inputs


def test_elementwise_chain_is_ieee_binary32():
    out, (a, b) = oracle_of("elementwise", {"n": 4099})
    expected = (a + b) * np.float32(2.0) - np.float32(1.0)  # numpy binary32, same order
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))


def c2_closed_form(x, n):
    xm = x.reshape(n, n)
    # y[i, j] = x[2j, 2i+1] + 1 for i < n/2; x[2j+1, 2(i-n/2)] + 1 otherwise
    top = xm[0::2, 1::2].T
    bottom = xm[1::2, 0::2].T
    return np.concatenate([top, bottom], axis=0) + np.float32(1.0)


@pytest.mark.parametrize("n", [2, 6, 64, 130])
def test_view_chain_matches_closed_form(n):
    out, (x,) = oracle_of("view_chain", {"n": n})
    assert out.shape == (n, n // 2)
    assert np.array_equal(out, c2_closed_form(x, n))


def test_view_chain_planted_mistake_is_caught():
    """Swapping the concat operands must fail the closed-form check."""
    n = 8
    x = config_inputs("view_chain", {"n": n})[0]
    t = placeholder([n, n], x)
    wrong = porch.concat(porch.transpose(t[porch.slice(1, n, 2), porch.slice(0, n, 2)]),
                         porch.transpose(t[porch.slice(0, n, 2), porch.slice(1, n, 2)]), 0) + 1.0
    assert not np.array_equal(host.evaluate(wrong), c2_closed_form(x, n))
    transposed_slice = porch.concat(t[porch.slice(0, n, 2), porch.slice(1, n, 2)],
                                    porch.transpose(t[porch.slice(1, n, 2), porch.slice(0, n, 2)]),
                                    0) + 1.0
    assert not np.array_equal(host.evaluate(transposed_slice), c2_closed_form(x, n))


def test_softmax_against_float64():
    size = {"rows": 64, "cols": 1000}
    out, (x,) = oracle_of("softmax", size)
    xm = x.reshape(64, 1000)
    # porch's graph subtracts the row max in binary32 (exact IEEE, so numpy
    # reproduces it); the rest is taken in float64 as the exact value.
    shifted = (xm - xm.max(axis=1, keepdims=True)).astype(np.float64)
    e = np.exp(shifted)
    truth = e / e.sum(axis=1, keepdims=True)
    rel = np.abs(out - truth) / truth
    assert rel.max() < 1e-6
    # against the unrounded shift the binary32 subtraction alone costs up to
    # half an ulp of |x - max| (~35 here): about 2e-6 relative
    e64 = np.exp(xm.astype(np.float64) - xm.max(axis=1, keepdims=True))
    assert (np.abs(out - e64 / e64.sum(axis=1, keepdims=True)) / out).max() < 4e-6
    assert np.allclose(out.sum(axis=1), 1.0, atol=1e-5)
    # the +20 outliers are present and dominate their rows
    assert (x == 20.0).any()


def test_softmax_planted_mistake_is_caught():
    """Dropping the max shift changes nothing mathematically but a wrong
    axis does: softmax over axis 0 must not pass the axis-1 check."""
    x = config_inputs("softmax", {"rows": 16, "cols": 32})[0]
    t = placeholder([16, 32], x)
    wrong = host.evaluate(porch.softmax(t, 0))
    xm = x.reshape(16, 32).astype(np.float64)
    e = np.exp(xm - xm.max(axis=1, keepdims=True))
    truth = e / e.sum(axis=1, keepdims=True)
    assert np.abs(wrong - truth).max() > 1e-3


def test_softmax_without_the_max_shift_is_caught():
    """A softmax built without its max shift, exp(x) / sum(exp(x)), equals
    softmax mathematically but overflows once a row holds values above 88:
    the float64 check passes the oracle's softmax and fails the unshifted
    one on such rows (N(0, 3) scaled by 10, so values reach ~150)."""
    x = config_inputs("softmax", {"rows": 16, "cols": 64})[0] * np.float32(10.0)
    t = placeholder([16, 64], x)
    xm = x.reshape(16, 64)
    # the shift in binary32, as porch's graph takes it; the rest in float64
    e = np.exp((xm - xm.max(axis=1, keepdims=True)).astype(np.float64))
    truth = e / e.sum(axis=1, keepdims=True)
    assert xm.max() > 88.0

    def passes(out):
        with np.errstate(invalid="ignore"):
            return bool(np.all(np.abs(out - truth) <= 1e-6 * truth + 1e-30))

    assert passes(host.evaluate(porch.softmax(t, 1)))
    unshifted = porch.exp(t) / porch.broadcast_to(porch.sum(porch.exp(t), 1, True), [16, 64])
    assert not passes(host.evaluate(unshifted))


def test_logistic_row_sums_against_float64():
    size = {"rows": 40, "cols": 2048}
    out, (x, w, b) = oracle_of("logistic_rowsum", size)
    z = (x.reshape(40, 2048) * w + b).astype(np.float64)  # binary32 product and sum as in porch
    z = np.maximum(z, 0.0)
    truth = (1.0 / (1.0 + np.exp(-z))).sum(axis=1)
    assert out.shape == (40,)
    assert (np.abs(out - truth) / np.abs(truth)).max() < 1e-5


def test_matmul_epilogue_against_float64():
    size = {"m": 48, "k": 4096, "n": 40}
    out, (a, b, bias) = oracle_of("matmul_epilogue", size)
    c = a.reshape(48, 4096).astype(np.float64) @ b.reshape(4096, 40).astype(np.float64)
    truth = np.maximum(c + bias.astype(np.float64), 0.0) - 0.5
    assert (np.abs(out - truth) / np.abs(truth)).max() < 1e-4
    # pre-epilogue product
    ta = placeholder([48, 4096], a)
    tb = placeholder([4096, 40], b)
    product = host.evaluate(porch.matmul(ta, tb))
    assert np.abs(product - c).max() < 1e-6
    # planted mistake: a transposed operand
    wrong = host.evaluate(porch.matmul(ta, porch.transpose(porch.transpose(tb))))
    assert np.array_equal(wrong, product)  # transpose twice is the identity
    sq = placeholder([40, 40], b[: 40 * 40])
    left = placeholder([48, 40], a[: 48 * 40])
    assert not np.allclose(host.evaluate(porch.matmul(left, porch.transpose(sq))),
                           host.evaluate(porch.matmul(left, sq)))


def test_reductions_exact_on_integers_and_order_free():
    rng = np.random.default_rng(7)
    values = rng.integers(-1000, 1000, size=(7, 1300)).astype(np.float32)
    t = placeholder([7, 1300], values)
    assert np.array_equal(host.evaluate(porch.sum(t, 1)), values.sum(axis=1))
    assert np.array_equal(host.evaluate(porch.sum(t, 0)), values.sum(axis=0))
    assert np.array_equal(host.evaluate(porch.max(t, 1, True)), values.max(axis=1, keepdims=True))
    assert np.array_equal(host.evaluate(porch.max(t, 0)), values.max(axis=0))


def test_max_reduction_of_all_minus_infinity_is_minus_flt_max():
    t = placeholder([1, 5], [-np.inf] * 5)
    out = host.evaluate(porch.max(t, 1))
    assert out[0] == np.float32(-3.4028234663852886e38)


def test_views_against_numpy_by_coordinates():
    rng = np.random.default_rng(3)
    x = rng.integers(0, 100, size=(5, 6, 7)).astype(np.float32)
    t = placeholder([5, 6, 7], x)
    cases = [
        (t[porch.slice(1, 5, 2), porch.all, porch.slice(-3, 100)], x[1:5:2, :, -3:]),
        (t[2, porch.slice(0, 6, 3)], x[2, 0:6:3]),
        (porch.reshape(t, [30, 7]), x.reshape(30, 7)),
        (porch.transpose(porch.reshape(t, [30, 7])), x.reshape(30, 7).T),
        (porch.unsqueeze(t, 1), x[:, None]),
        (porch.broadcast_to(placeholder([6, 1], x[0, :, :1]), [4, 6, 3]),
         np.broadcast_to(x[0, :, :1], (4, 6, 3))),
        (porch.concat(t, t[porch.slice(0, 2)], 0), np.concatenate([x, x[0:2]], 0)),
        (porch.concat(t, t[porch.all, porch.all, porch.slice(0, 2)], 2),
         np.concatenate([x, x[:, :, 0:2]], 2)),
        (porch.reshape(porch.transpose(porch.reshape(t[porch.slice(1, 4)], [18, 7])), [7, 3, 6]),
         x[1:4].reshape(18, 7).T.reshape(7, 3, 6)),
    ]
    for expr, expected in cases:
        out = host.evaluate(expr)
        assert out.shape == expected.shape
        assert np.array_equal(out, expected)


def test_exp_within_one_ulp_of_correct_rounding():
    xs = np.linspace(-80.0, 80.0, 20001).astype(np.float32)
    t = placeholder([xs.size], xs)
    out = host.evaluate(porch.exp(t))
    truth = np.array([math.exp(float(v)) for v in xs])
    ulp = np.spacing(truth.astype(np.float32))
    assert (np.abs(out.astype(np.float64) - truth) <= ulp).all()


def test_maximum_minimum_follow_the_reference_ternary_on_nan():
    lhs = placeholder([3], [np.nan, 1.0, -0.0])
    rhs = placeholder([3], [2.0, np.nan, 0.0])
    hi = host.evaluate(porch.maximum(lhs, rhs))
    lo = host.evaluate(porch.minimum(lhs, rhs))
    # l > r ? l : r  -> any comparison with NaN is false -> r
    assert hi[0] == 2.0 and np.isnan(hi[1]) and hi[2] == 0.0 and not np.signbit(hi[2])
    assert lo[0] == 2.0 and np.isnan(lo[1]) and lo[2] == 0.0 and not np.signbit(lo[2])


def _quotients(lhs, rhs):
    with np.errstate(all="ignore"):
        return np.divide(lhs, rhs, dtype=np.float32), np.divide(np.float32(1.0), rhs, dtype=np.float32)


def test_divide_and_reciprocal_are_ieee_binary32():
    """l / r and reciprocal(r) = 1.0f / r (src/tensor.cpp:659-667,864)
    against numpy's correctly rounded binary32 division, bit for bit (NaN
    as NaN): every pairing of signed zeros, infinities, NaN, denormals,
    FLT_MAX and FLT_MIN, quotients that overflow and underflow, and random
    operands over the whole range."""
    lhs, rhs = division_operands(1 << 16, 5)
    tl, tr = placeholder([lhs.size], lhs), placeholder([rhs.size], rhs)
    q, inv = _quotients(lhs, rhs)
    assert_bits_or_both_nan(host.evaluate(tl / tr), q)
    assert_bits_or_both_nan(host.evaluate(porch.reciprocal(tr)), inv)
    # the underflowing and overflowing cases are among them
    assert np.isinf(q).sum() > 50 and ((q != 0) & (np.abs(q) < np.finfo(np.float32).tiny)).sum() > 50
    # a divisor broadcast along rows
    rows = 37
    l2 = lhs[: rows * 256].reshape(rows, 256)
    r2 = rhs[-256:].reshape(1, 256)
    t2 = host.evaluate(placeholder([rows, 256], l2) / porch.broadcast_to(placeholder([1, 256], r2), [rows, 256]))
    assert_bits_or_both_nan(t2, _quotients(l2, np.broadcast_to(r2, l2.shape))[0])


def test_divide_planted_reciprocal_product_is_caught():
    """The check above rejects a division written as l * (1.0f / r): that
    differs from l / r in the last bit on many operands."""
    lhs, rhs = division_operands(1 << 16, 5)
    q, inv = _quotients(lhs, rhs)
    with np.errstate(all="ignore"):
        planted = (lhs * inv).astype(np.float32)
    with pytest.raises(AssertionError):
        assert_bits_or_both_nan(planted, q)
    # and a division that flushes denormal results to zero
    flushed = np.where(np.abs(q) < np.finfo(np.float32).tiny, np.float32(0.0) * np.sign(q), q).astype(np.float32)
    with pytest.raises(AssertionError):
        assert_bits_or_both_nan(flushed, q)
