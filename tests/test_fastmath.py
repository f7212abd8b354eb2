"""Range-driven instruction choices for reciprocal and exp.

Where the value-range analysis proves a reciprocal's operand lies in
[2^-125, 2^125] (in magnitude), kernels use the hardware reciprocal plus one
Newton step (porch_rcp), which must equal IEEE 1.0f / x bit for bit; where it
proves an exp argument is <= 88, kernels use porch_exp / porch_exp_finite,
which must stay within 2 ulp of the host's exp.  The CPU tests pin where the
analysis allows each form (and where it must not); the GPU tests check the
results against the oracle, exhaustively over whole binades for the
reciprocal.
"""

import re

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import placeholder


def source_of(expr):
    return porch.kernel_source(expr, 0)


def body(expr):
    s = source_of(expr)
    return s[s.index('extern "C"'):]


# -- where the fast forms apply (no GPU) ---------------------------------------

def test_logistic_of_relu_takes_both_fast_forms():
    x = placeholder([64, 128])
    b = body(porch.logistic(porch.relu(x)))
    # exp's only consumer is 1 + e, which absorbs denormals: the flushing form
    assert "porch_rcp(" in b and "porch_exp_flush_finite(-" in b
    assert "1.0f /" not in b and not re.search(r"\bexpf\(", b)


EXP_FORMS = r"\b(porch_exp_flush_finite|porch_exp_flush|porch_exp_finite|porch_exp|expf)\("


@pytest.mark.parametrize("make,fn", [
    (lambda e: e, "porch_exp_finite"),                    # stored: denormals visible
    (lambda e: 1.0 + e, "porch_exp_flush_finite"),
    (lambda e: 2.0 - e, "porch_exp_flush_finite"),
    (lambda e: e - 0.5, "porch_exp_flush_finite"),
    (lambda e: 1e-38 + e, "porch_exp_finite"),            # constant below 2^-100
    (lambda e: (1.0 + e) * e, "porch_exp_finite"),        # a multiply sees e itself
    (lambda e: porch.sum(1.0 + e, 1), "porch_exp_flush_finite"),
    (lambda e: porch.sum(e, 1), "porch_exp_finite"),      # reduced directly
])
def test_flushing_exp_only_where_consumers_absorb_denormals(make, fn):
    x = placeholder([64, 256])
    b = body(make(porch.exp(porch.minimum(x, 88.0))))
    assert set(re.findall(EXP_FORMS, b)) == {fn}


def test_unknown_operands_keep_ieee_division_and_expf():
    x = placeholder([64, 128])
    b = body(porch.reciprocal(x) + porch.exp(x))
    assert "1.0f / " in b and "expf(" in b and "porch_rcp(" not in b and "porch_exp" not in b


@pytest.mark.parametrize("make,fast", [
    (lambda x: porch.reciprocal(porch.minimum(porch.maximum(x, 1.0), 2.0)), True),
    (lambda x: porch.reciprocal(porch.maximum(x, 0.0)), False),          # 0 is in range
    (lambda x: porch.reciprocal(porch.maximum(x, 1e-38)), False),        # below 2^-125
    (lambda x: porch.reciprocal(porch.maximum(x, 2.0 ** -125)), False),  # unbounded above
    (lambda x: porch.reciprocal(porch.minimum(porch.maximum(x, 2.0 ** -125), 2.0 ** 125)), True),
    (lambda x: porch.reciprocal(porch.minimum(porch.maximum(x, -3.0), -0.5)), True),
    (lambda x: porch.reciprocal(x * x + 1.0), False),  # >= 1, but intervals cannot see a square
])
def test_reciprocal_fast_form_only_when_tame(make, fast):
    b = body(make(placeholder([256])))
    assert ("porch_rcp(" in b) == fast
    assert ("1.0f / " in b) == (not fast)


@pytest.mark.parametrize("make,fn", [
    (lambda x: porch.exp(porch.minimum(x, 88.0)), "porch_exp_finite("),  # NaN becomes 88
    (lambda x: porch.exp(porch.minimum(88.0, x)), "porch_exp("),        # NaN stays NaN
    (lambda x: porch.exp(porch.minimum(x, 89.0)), "expf("),              # may overflow
    (lambda x: porch.exp(x), "expf("),
    (lambda x: porch.exp(0.0 - porch.relu(x)), "porch_exp_finite(-"),
])
def test_exp_form_follows_the_argument_range(make, fn):
    b = body(make(placeholder([256])))
    called = set(re.findall(EXP_FORMS, b))
    assert called == {fn.split("(")[0]}, called
    assert fn in b


RELAXED = ("porch_exp_relaxed(", "__builtin_amdgcn_rcpf(")


def logistic_relu(x):
    return porch.logistic(porch.relu(x))


@pytest.mark.parametrize("make,relaxed", [
    (lambda x: porch.sum(logistic_relu(x), 1), True),                 # result is the sum
    (lambda x: porch.sum(logistic_relu(x), 1, True), True),
    (lambda x: porch.max(logistic_relu(x), 1), False),                # a max selects values
    (lambda x: logistic_relu(x), False),                              # stored elementwise
    (lambda x: porch.softmax(x, 1), False),
    # the logistic also feeds a max reduction: not only the final sum
    (lambda x: porch.sum(logistic_relu(x) - porch.broadcast_to(
        porch.max(logistic_relu(x), 1, True), [64, 2048]), 1), False),
    (lambda x: porch.sum(porch.exp(x), 1), False),                    # exp argument unbounded
])
def test_relaxed_forms_only_inside_a_final_sum(make, relaxed):
    b = body(make(placeholder([64, 2048])))
    for form in RELAXED:
        assert (form in b) == relaxed, form


def test_products_fuse_into_fma_only_inside_a_final_sum():
    x = placeholder([64, 2048])
    w = porch.broadcast_to(placeholder([1, 2048]), [64, 2048])
    b = porch.broadcast_to(placeholder([1, 2048]), [64, 2048])
    affine = x * w + b
    assert "__builtin_fmaf(" in body(porch.sum(porch.logistic(porch.relu(affine)), 1))
    assert "__builtin_fmaf(" in body(porch.sum(b - x * w, 1))
    # stored, or selected by a max: each product rounds on its own
    assert "__builtin_fmaf(" not in body(affine)
    assert "__builtin_fmaf(" not in body(porch.max(affine, 1))
    # a product used twice is computed once, not fused into either use
    assert "__builtin_fmaf(" not in body(porch.sum((x * w + b) * (x * w), 1))


def test_reciprocals_share_one_rcp_only_when_their_operands_are_bounded():
    x = placeholder([64, 2048])
    # the logistic's 1 + exp(-relu(x)) lies in [1, 2]: four terms, one rcp
    paired = body(porch.sum(porch.logistic(porch.relu(x)), 1))
    assert paired.count("__builtin_amdgcn_rcpf(") == 1 and "__builtin_amdgcn_rcpf(xp" in paired
    # 1/x for an unbounded x: one reciprocal per term
    assert "__builtin_amdgcn_rcpf(xp" not in body(porch.sum(porch.reciprocal(x), 1))
    # exp(-x) is unbounded above without the relu
    assert "__builtin_amdgcn_rcpf(xp" not in body(porch.sum(porch.logistic(x), 1))
    # not a final sum
    assert "rcpf(xp" not in body(porch.logistic(porch.relu(x)))


@pytest.mark.parametrize("op, constant, hardware", [
    ("maximum", 0.0, True), ("maximum", -0.0, False), ("maximum", 1.5, True), ("maximum", -2.0, True),
    ("minimum", -0.0, True), ("minimum", 0.0, False), ("minimum", 1.5, True), ("minimum", -2.0, True),
])
def test_max_and_min_against_a_constant_use_one_instruction(op, constant, hardware):
    x = placeholder([1024])
    fn = "__builtin_fmaxf(" if op == "maximum" else "__builtin_fminf("
    assert (fn in body(getattr(porch, op)(x, constant))) == hardware
    # a constant on the left keeps the ternary: a NaN x must pass through
    assert fn not in body(getattr(porch, op)(constant, x))


def test_negation_folds_into_exp_only_for_positive_zero():
    x = placeholder([256])
    assert "expf(-" in body(porch.exp(0.0 - x))
    assert "expf(-" not in body(porch.exp(-0.0 - x))


# -- results (GPU) ---------------------------------------------------------------

def binades(first, count):
    """Every float of the binades [2^first, 2^(first + count)), in order."""
    m = np.arange(1 << 23, dtype=np.uint32)
    exponents = (np.arange(first, first + count, dtype=np.int64) + 127).astype(np.uint32) << np.uint32(23)
    return (exponents[:, None] | m[None, :]).reshape(-1).view(np.float32)


# porch_rcp is chosen wherever range analysis proves |x| in [2^-125, 2^125]:
# every float there (250 binades, both signs, and 2^125 itself), in chunks
# of 25 binades, against numpy's correctly rounded binary32 division.
@pytest.mark.gpu
@pytest.mark.parametrize("sign", [1, -1])
@pytest.mark.parametrize("first", list(range(-125, 125, 25)))
def test_fast_reciprocal_is_ieee_on_every_binade(gpu, first, sign):
    x = binades(first, 25) * np.float32(sign)
    if first + 25 == 125:
        x = np.append(x, np.float32(sign * 2.0 ** 125))
    lo, hi = sorted([float(sign * 2.0 ** first), float(sign * 2.0 ** (first + 25))])
    t = gpu.tensor([x.size], x)
    expr = gpu.reciprocal(gpu.minimum(gpu.maximum(t, lo), hi))
    assert "porch_rcp(" in gpu.kernel_source(expr, 0)
    out = gpu.materialize(expr).cpu()
    ref = np.float32(1.0) / x
    bad = np.flatnonzero(out.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, (bad.size, x[bad[:4]], out[bad[:4]], ref[bad[:4]])


@pytest.mark.gpu
def test_fast_reciprocal_keeps_nan_and_signs(gpu):
    x = np.array([1.0, -1.0, 1.5, -1.75, np.nan, 3.0, -2.5], dtype=np.float32)
    t = gpu.tensor([x.size], x)
    # constants on the left: a NaN x passes through maximum and minimum
    expr = gpu.reciprocal(gpu.minimum(4.0, gpu.maximum(1.0, t)))
    assert "porch_rcp(" in gpu.kernel_source(expr, 0)
    out = gpu.materialize(expr).cpu()
    ref = host.evaluate(expr)
    # NaN where the oracle has NaN (IEEE leaves a NaN result's sign and
    # payload open), every other value bit for bit.
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    keep = ~np.isnan(ref)
    assert np.array_equal(out[keep].view(np.uint32), ref[keep].view(np.uint32))


def ulp_distance(a, b):
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, np.int64(-(1 << 31)) - ia, ia)
    ib = np.where(ib < 0, np.int64(-(1 << 31)) - ib, ib)
    return np.abs(ia - ib)


@pytest.mark.gpu
def test_fast_exp_within_2_ulp(gpu):
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) <= 110.0)]
    x = np.concatenate([x, rng.uniform(-110, 88, size=1 << 20).astype(np.float32),
                        np.array([-np.inf, -1e30, -104.0, -103.9, -87.4, -87.3, -0.0, 0.0,
                                  1e-30, 88.0, 87.99], dtype=np.float32)])
    t = gpu.tensor([x.size], x)
    for make, fn in [(lambda v: gpu.exp(gpu.minimum(v, 88.0)), "porch_exp_finite("),
                     (lambda v: gpu.exp(gpu.minimum(88.0, v)), "porch_exp(")]:
        expr = make(t)
        assert fn in gpu.kernel_source(expr, 0)
        out = gpu.materialize(expr).cpu()
        ref = host.evaluate(expr)
        assert ulp_distance(out, ref).max() <= 2


@pytest.mark.gpu
def test_flushing_exp_consumers_within_2_ulp(gpu):
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-120, 90, size=1 << 20),
                        rng.uniform(-105, -80, size=1 << 18),
                        [-np.inf, np.inf, np.nan, -104.0, -87.5, 0.0]]).astype(np.float32)
    t = gpu.tensor([x.size], x)
    for make in (lambda v: gpu.logistic(gpu.relu(v)),
                 lambda v: 2.0 - gpu.exp(gpu.minimum(v, 0.0)),  # e <= 1: no cancellation
                 lambda v: gpu.exp(gpu.minimum(88.0, v)) + 0.25):
        expr = make(t)
        assert "porch_exp_flush" in gpu.kernel_source(expr, 0)
        out = gpu.materialize(expr).cpu()
        ref = host.evaluate(expr)
        assert np.array_equal(np.isnan(out), np.isnan(ref))
        keep = ~np.isnan(ref)
        assert ulp_distance(out[keep], ref[keep]).max() <= 2


@pytest.mark.gpu
def test_relaxed_logistic_row_sums_within_1e5(gpu):
    rng = np.random.default_rng(9)
    rows, cols = 257, 2048
    x = (rng.standard_normal(rows * cols) * 30).astype(np.float32)
    x[::97] = np.inf
    x[::89] = -np.inf
    x[::83] = np.nan
    x[::79] = -1e30
    t = gpu.tensor([rows, cols], x)
    expr = gpu.sum(gpu.logistic(gpu.relu(t)), 1)
    assert "porch_exp_relaxed(" in gpu.kernel_source(expr, 0)
    out = gpu.materialize(expr).cpu()
    ref = host.evaluate(expr)
    assert np.all(np.abs(out - ref) <= 1e-5 * np.abs(ref))


@pytest.mark.gpu
def test_fast_exp_propagates_nan(gpu):
    x = np.array([np.nan, 0.0, -1.0, -np.inf, 88.0], dtype=np.float32)
    t = gpu.tensor([x.size], x)
    expr = gpu.exp(gpu.minimum(88.0, t))
    out = gpu.materialize(expr).cpu()
    assert np.isnan(out[0]) and out[1] == 1.0 and out[3] == 0.0
    assert ulp_distance(out[1:], host.evaluate(expr)[1:]).max() <= 2


@pytest.mark.gpu
def test_max_and_min_against_constants_match_the_ternaries(gpu):
    """maximum(x, c) and minimum(x, c) as v_max_f32 / v_min_f32 give the
    reference's ternary bits (src/tensor.cpp:677-682) on signed zeros, NaN
    of either sign, infinities and denormals, for every constant form; the
    forms the emitter keeps as ternaries are checked alongside."""
    nan = np.float32(np.nan)
    specials = np.array([-0.0, 0.0, nan, -nan, np.inf, -np.inf, 1e-45, -1e-45, 1.0, -1.0, 1.5, -2.0, 3.0],
                        dtype=np.float32)
    x = np.concatenate([specials, np.random.default_rng(4).standard_normal(4096).astype(np.float32)])
    t = gpu.tensor([x.size], x)
    for c in (0.0, -0.0, 1.5, -2.0, 1e-45):
        for op in (gpu.maximum, gpu.minimum):
            expr = op(t, c)
            out = gpu.materialize(expr).cpu()
            ref = host.evaluate(expr)
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (op.__name__, c)


# porch_div (the split softmax's output division): RN(q + (a - b q) r) with
# r = porch_rcp(b) and q = RN(a r) against the GPU's IEEE division a / b,
# for every significand of a (one binade: the rounding depends on the
# significands, the exponents only shift it while the quotient stays
# normal) against 256 divisors, at three exponent pairs spanning the range
# the kernel uses it in (a in [e^-60, 1], b in [1, 2^31]).
_DIV_KERNEL = r"""
extern "C" __global__ void divcheck(const float* b, const float* abits, float* out, unsigned long long count) {
    const unsigned long long t = blockIdx.x * 256ull + threadIdx.x;
    if (t >= count) return;
    const float d = b[t / 4096];
    const float r = porch_rcp(d);
    const unsigned first = (unsigned)(t % 4096) * 2048u;
    const unsigned base = __float_as_uint(abits[0]);
    float bad = 0.0f;
    for (unsigned i = 0; i < 2048u; ++i) {
        const float a = __uint_as_float(base | (first + i));
        const float q = a / d;
        const float m = porch_div(a, r, d);
        bad += __float_as_uint(q) != __float_as_uint(m) ? 1.0f : 0.0f;
    }
    out[t] = bad;
}
"""


def _split_softmax_helpers():
    source = porch.kernel_source(porch.softmax(placeholder([4, 262144]), 1), 1)
    found = [re.search(r"__device__ __forceinline__ float %s\(.*?\n}\n" % name, source, re.S)
             for name in ("porch_rcp", "porch_div")]
    assert all(found)
    return "".join(m.group(0) for m in found)


def test_split_softmax_uses_the_checked_division():
    helpers = _split_softmax_helpers()
    assert "__builtin_amdgcn_rcpf(d)" in helpers
    assert "__builtin_fmaf(__builtin_fmaf(-b, q, a), r, q)" in helpers


@pytest.mark.gpu
@pytest.mark.parametrize("a_exp, b_exp", [(0, 0), (-60, 30), (-1, 20)])
def test_reciprocal_division_is_ieee(gpu, a_exp, b_exp):
    import ctypes

    from porch_amd import _lib

    rng = np.random.default_rng((a_exp + 100) * 100 + b_exp)
    significands = [0, 1, (1 << 23) - 1, 1 << 22, 1 << 21, 3 << 21, 0x3504F3, (1 << 22) - 1, (1 << 22) + 1]
    significands += [int(v) for v in rng.integers(0, 1 << 23, size=256 - len(significands))]
    b = (np.array(significands, np.uint32) | np.uint32((127 + b_exp) << 23)).view(np.float32)
    abits = np.array([(127 + a_exp) << 23], np.uint32).view(np.float32)
    code = ctypes.c_void_p()
    _lib.check(_lib.lib.porch_compile((_split_softmax_helpers() + _DIV_KERNEL).encode(), None, 0, ctypes.byref(code)))
    try:
        size = _lib.lib.porch_code_object_size(code)
        data = _lib.lib.porch_code_object_data(code)
        bb = gpu._Buffer.upload(b)
        ab = gpu._Buffer.upload(abits)
        count = b.size * 4096
        out = gpu._Buffer.upload(np.zeros(count, np.float32))
        ins = (ctypes.c_void_p * 2)(bb.handle, ab.handle)
        _lib.check(_lib.lib.porch_launch_fused_elementwise(data, size, b"divcheck", ins, 2, out.handle, count))
        bad = out.download(count)
    finally:
        _lib.lib.porch_code_object_release(code)
    assert bad.sum() == 0, (bad.sum(), b[np.flatnonzero(bad.reshape(b.size, 4096).sum(axis=1))[:4]])
