"""Softmax rows split over workgroups (kernel kind row.split).

Rows of more than 32768 values, in a softmax-shaped row program over one
leaf, are split into parts of at most 16384 values (as even as whole chunks
of 1024 allow), one part per workgroup held in registers; the parts of a row exchange (max, sum of
exp(f - max)) words through a zeroed temporary, combine them as M = max m_p,
S = sum s_p exp(m_p - M), and write their outputs from registers, so the row
is read from memory once.  A part whose partners do not publish within a
bounded wait computes the row's max and sum itself from memory.

CPU: the planner's choice and the temporary, bounds and values of the
kernels run on the CPU (blocks run one after another there, so a row's last
part takes the exchange path and the others their own fallback), and a
planted mistake in each path.  GPU: parity with the oracle at the workload's
size and at ragged sizes and row counts, and the fallback alone, forced from
the host with a spin limit of zero.  Bar (assert_softmax_close, on the CPU
and the GPU): 1e-6 relative per element against the float64 softmax of the
same float32 differences, and against the oracle 1e-6 plus the oracle's own
measured row-sum drift; NaN exactly where the oracle has NaN (the row max is
the reference's, exactly).
"""

import ctypes
import re

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from porch_amd import _lib
from tests.helpers import CONFIG_SIZES, assert_softmax_close, config_inputs, placeholder
from tests.kernel_emu import emulate as emu
from tests.test_max_order import special_rows

needs_clang = pytest.mark.skipif(not emu.available(), reason="host clang++ from ROCm is required")


def _kinds(expr):
    return [k["kind"] for k in porch.plan(expr)["kernels"]]


@pytest.mark.parametrize("cols, parts", [(32772, 3), (40964, 3), (65536, 4), (65540, 5), (131072, 8), (200004, 13),
                                         (262144, 16), (262148, 17)])
def test_planner_splits_long_softmax_rows(cols, parts):
    expr = porch.softmax(placeholder([7, cols]), 1)
    plan = porch.plan(expr)
    assert _kinds(expr) == ["pointwise.flat", "row.split"]
    # the temporary: one 64-bit word per row and part, zeroed by the first step
    assert plan["temps"] == [7 * parts * 2]
    assert plan["kernels"][0]["dest"] == "temp0" and plan["kernels"][1]["dest"] == "output"
    # at most two workgroups per compute unit, in whole row groups per XCD
    grid = plan["kernels"][1]["grid"][0]
    assert grid <= 512 and grid % (8 * parts) == 0
    source = porch.kernel_source(expr, 1)
    assert "__launch_bounds__(256, 2)" in source
    assert "__HIP_MEMORY_SCOPE_AGENT" in source and "__ATOMIC_RELAXED" in source
    assert re.search(r"#define porch_spin_limit \d+", source)


@pytest.mark.parametrize("build", [
    lambda: porch.softmax(placeholder([4, 32768]), 1),       # as fast in one workgroup
    lambda: porch.softmax(placeholder([4, 262147]), 1),      # odd length: no 128-bit loads
    lambda: porch.softmax(placeholder([4, 262144]) * placeholder([4, 262144]), 1),  # two leaves
    lambda: porch.sum(porch.exp(placeholder([4, 262144])), 1),  # no elementwise output
    lambda: porch.exp(placeholder([4, 262144]) - porch.broadcast_to(
        porch.max(placeholder([4, 262144]), 1, True), [4, 262144])),  # one reduction
])
def test_other_row_programs_are_not_split(build):
    assert "row.split" not in _kinds(build())


@needs_clang
@pytest.mark.parametrize("shape", [[3, 65540], [2, 262148], [2, 40964]])
def test_emulated_split_rows_match_the_oracle(shape):
    rng = np.random.default_rng(shape[1])
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    x[0, 7] = 25.0  # one part's max far above the others'
    t = placeholder(shape, x)
    expr = porch.softmax(t, 1)
    assert all(r["ok"] for r in emu.emulate(expr))
    assert_softmax_close(emu.evaluate(expr, [x]).reshape(shape), t, x)


@needs_clang
def test_emulated_special_rows_take_the_reference_max():
    shape = [10, 65540]
    x = special_rows(*shape, seed=5)
    t = placeholder(shape, x)
    expr = porch.softmax(t, 1)
    assert_softmax_close(emu.evaluate(expr, [x]).reshape(shape), t, x)
    # every max also recomputed in the reference's order
    assert_softmax_close(emu.evaluate(expr, [x], force_exact=True).reshape(shape), t, x)


# Other programs of the split form: f an expression of the leaf, the leaf a
# view (a column offset that keeps 128-bit alignment), more than one row
# dimension.  (`storage`: the leaf's values; `build`: the graph over it.)
FORMS = {
    "scaled": ([3, 65540], lambda t: porch.softmax(t * 0.5 + 1.0, 1), lambda x: x * np.float32(0.5) + np.float32(1.0)),
    "view": ([3, 65544], lambda t: porch.softmax(t[porch.slice(0, 3), porch.slice(4, 65544)], 1), lambda x: x[:, 4:]),
    "rank3": ([2, 3, 40964], lambda t: porch.softmax(t, 2), lambda x: x.reshape(6, 40964)),
}


@pytest.mark.parametrize("form", sorted(FORMS))
def test_other_forms_are_split(form):
    shape, build, _ = FORMS[form]
    assert _kinds(build(placeholder(shape))) == ["pointwise.flat", "row.split"]
    # a column offset that breaks 128-bit alignment is not split
    if form == "view":
        t = placeholder(shape)
        assert "row.split" not in _kinds(porch.softmax(t[porch.slice(0, 3), porch.slice(1, 65541)], 1))


@needs_clang
@pytest.mark.parametrize("form", sorted(FORMS))
def test_emulated_other_forms_match_the_oracle(form):
    shape, build, _ = FORMS[form]
    x = (np.random.default_rng(9).standard_normal(shape) * 3).astype(np.float32)
    expr = build(placeholder(shape, x))
    got = emu.evaluate(expr, [x])
    ref = host.evaluate(expr)
    rel = np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)), 1e-30)
    assert rel.max() <= 2e-6, rel.max()


def _evaluate_planted(expr, x, old, new):
    """emu.evaluate with `old` replaced by `new` in the split kernel."""
    original = porch.kernel_source

    def planted(e, index=0):
        source = original(e, index)
        if "row.split" in porch.plan(e)["kernels"][index]["kind"]:
            assert old in source
            source = source.replace(old, new)
        return source

    porch.kernel_source = planted
    try:
        return emu.evaluate(expr, [x])
    finally:
        porch.kernel_source = original


@needs_clang
@pytest.mark.parametrize("old, new, path", [
    # the exchange: partial sums taken without rescaling to the row max
    ("xps * porch_exp(xpm - rv0)", "xps", "exchange"),
    # the fallback: lane sums not rescaled to the row max
    ("(float)(acc_s * (double)porch_exp(acc_a - acc_m))", "(float)acc_s", "fallback"),
])
def test_emulation_catches_a_planted_mistake_in_each_path(old, new, path):
    shape = [2, 65540]
    x = (np.random.default_rng(3).standard_normal(shape) * 3).astype(np.float32)
    x[:, 70000 % shape[1]] = 30.0
    x[:, 5] = 20.0
    expr = porch.softmax(placeholder(shape, x), 1)
    ref = host.evaluate(expr)
    got = _evaluate_planted(expr, x, old, new).reshape(shape)
    err = np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)), 1e-30)
    assert err.max() > 1e-3, path


def test_softmax_bar_accepts_the_oracle_and_rejects_a_scaled_result():
    # the check used on the GPU below, on the CPU: the oracle's own result
    # passes; a result off by 3e-6 (or with one value off) does not
    shape = [4, 65540]
    x = (np.random.default_rng(8).standard_normal(shape) * 3).astype(np.float32)
    t = placeholder(shape, x)
    ref = np.asarray(host.evaluate(porch.softmax(t, 1)), np.float32).reshape(shape)
    assert_softmax_close(ref, t, x)
    with pytest.raises(AssertionError):
        assert_softmax_close((ref * np.float32(1 + 3e-6)).astype(np.float32), t, x)
    bad = ref.copy()
    bad[2, 100] = np.nextafter(np.nextafter(np.nextafter(bad[2, 100], 1), 1), 1) * np.float32(1 + 2e-6)
    with pytest.raises(AssertionError):
        assert_softmax_close(bad, t, x)


# -- GPU -----------------------------------------------------------------------


@pytest.mark.gpu
def test_vocab_softmax_full_size(gpu):
    size = CONFIG_SIZES["vocab_softmax"]
    (x,) = config_inputs("vocab_softmax")
    shape = [size["rows"], size["cols"]]
    t = gpu.tensor(shape, x)
    expr = gpu.softmax(t, 1)
    assert _kinds(expr) == ["pointwise.flat", "row.split"]
    out = gpu.materialize(expr).cpu().reshape(shape)
    assert_softmax_close(out, t, x)
    assert np.allclose(out.sum(axis=1), 1.0, atol=2e-5)
    # a second run on the same inputs: the temporary is zeroed again (bits
    # may differ only where a part took its own fallback)
    again = gpu.materialize(expr).cpu().reshape(shape)
    assert np.allclose(again, out, rtol=1e-6, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("rows, cols", [
    (1, 65540),      # one row, five parts, the last ragged
    (1000, 65540),   # many rounds
    (33, 131072),    # one round, partly filled
    (70, 262144),    # three rounds: the odd round ends the loop
    (97, 262144),    # four rounds, the last partly filled
    (40, 200004),
])
def test_split_rows_match_the_oracle(gpu, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    x[rng.random((rows, cols)) < 0.01] = 20.0
    t = gpu.tensor([rows, cols], x)
    expr = gpu.softmax(t, 1)
    assert _kinds(expr) == ["pointwise.flat", "row.split"]
    out = gpu.materialize(expr).cpu().reshape(rows, cols)
    assert_softmax_close(out, t, x)


@pytest.mark.gpu
def test_special_rows_split_on_gpu(gpu):
    shape = [30, 131076]
    x = special_rows(*shape, seed=17)
    t = gpu.tensor(shape, x)
    expr = gpu.softmax(t, 1)
    assert _kinds(expr) == ["pointwise.flat", "row.split"]
    out = gpu.materialize(expr).cpu().reshape(shape)
    assert_softmax_close(out, t, x)


@pytest.mark.gpu
def test_fallback_alone_matches_the_oracle(gpu):
    """Every part computes its row's max and sum itself: the kernel built
    with a spin limit of zero never reads a partner's word, as when the
    partners are not resident."""
    rows, cols = 45, 65540
    x = special_rows(rows, cols, seed=23)
    x[10:20] = np.random.default_rng(2).standard_normal((10, cols)).astype(np.float32) * 40
    t = gpu.tensor([rows, cols], x)
    expr = gpu.softmax(t, 1)
    plan = gpu.plan(expr)
    kernel = plan["kernels"][1]
    source = gpu.kernel_source(expr, 1)
    forced = re.sub(r"#define porch_spin_limit \d+", "#define porch_spin_limit 0", source)
    assert forced != source
    code = ctypes.c_void_p()
    _lib.check(_lib.lib.porch_compile(forced.encode(), None, 0, ctypes.byref(code)))
    try:
        size = _lib.lib.porch_code_object_size(code)
        data = _lib.lib.porch_code_object_data(code)
        # inputs as the planner lays them out: x, then the exchange words
        # (never read here, but still written)
        xs = gpu._Buffer.upload(x.reshape(-1))
        words = gpu._Buffer.upload(np.zeros(plan["temps"][0], np.float32))
        out = gpu._Buffer.upload(np.zeros(rows * cols, np.float32))
        ins = (ctypes.c_void_p * 2)(xs.handle, words.handle)
        # one 256-lane workgroup per "output": the kernel's own grid
        assert kernel["block"] == 256
        _lib.check(_lib.lib.porch_launch_fused_reduction(data, size, b"porch_row", ins, 2, out.handle,
                                                         kernel["grid"][0]))
        got = out.download(rows * cols).reshape(rows, cols)
    finally:
        _lib.lib.porch_code_object_release(code)
    assert_softmax_close(got, t, x)


@pytest.mark.gpu
def test_two_split_softmaxes_on_two_streams_at_once(gpu):
    """Two threads (each with its own stream) materialise split softmaxes
    at the same time.  Their workgroups then share the GPU, so a row's
    parts may not all be resident together; a part that waits too long
    computes its row alone.  Both results must still match the oracle."""
    import threading

    shape = [256, 131072]
    inputs = [(np.random.default_rng(50 + i).standard_normal(shape) * 3).astype(np.float32) for i in range(2)]
    tensors = [gpu.tensor(shape, x) for x in inputs]
    results = [None, None]
    errors = []

    def run(i):
        try:
            outs = [gpu.materialize(gpu.softmax(tensors[i], 1)) for _ in range(4)]
            results[i] = [o.cpu().reshape(shape) for o in outs]
        except Exception as e:  # reported below, on the main thread
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(2):
        for out in results[i]:
            assert_softmax_close(out, tensors[i], inputs[i])


@pytest.mark.gpu
@pytest.mark.parametrize("form", sorted(FORMS))
def test_other_forms_on_gpu(gpu, form):
    shape, build, rows_of = FORMS[form]
    x = (np.random.default_rng(19).standard_normal(shape) * 3).astype(np.float32)
    t = gpu.tensor(shape, x)
    expr = build(t)
    assert _kinds(expr) == ["pointwise.flat", "row.split"]
    out = gpu.materialize(expr).cpu()
    ref = host.evaluate(expr)
    # the oracle's softmax of the same rows: 1e-6 beyond its own row-sum
    # drift, and the float64 softmax of the same differences (the rows as
    # the leaf's values arrive at the row program)
    rows = np.ascontiguousarray(rows_of(x))
    flat = rows.reshape(-1, rows.shape[-1])
    t2 = placeholder(list(flat.shape), flat)
    assert_softmax_close(out.reshape(flat.shape), t2, flat)
    assert np.allclose(out.reshape(-1), ref.reshape(-1), rtol=3e-6, atol=0)
