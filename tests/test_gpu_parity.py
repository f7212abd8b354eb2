"""GPU results against the host evaluator on the same seeded inputs.

Bars (stated per test): bit-exact for view/index/concat/+-*/ graphs (kernels
are built with -ffp-contract=off, correctly rounded division); exp-based
graphs within 2 ulp or 1e-6 relative (softmax: beyond the oracle's own
row-sum drift, and against a float64 softmax of the same differences); reductions 1e-5 and matmul 1e-4
relative (their summation order is free).  Full-size configs are checked
against the oracle (on a row sample for the matmul, whose every output is
also checked against a float64 GEMM) and through properties that do not
depend on size.
"""

import numpy as np
import pytest

from oracle import host
from tests.helpers import (CONFIG_SIZES, assert_softmax_close, check_matmul_epilogue_every_output, config_graph,
                           config_inputs, config_shapes)

pytestmark = pytest.mark.gpu


def gpu_and_oracle(porch, name, size=None, inputs=None):
    shapes = config_shapes(name, size)
    inputs = inputs if inputs is not None else config_inputs(name, size)
    tensors = [porch.tensor(s, v) for s, v in zip(shapes, inputs)]
    expr = config_graph(name, tensors, size)
    out = porch.materialize(expr).cpu().reshape(expr.shape())
    return out, host.evaluate(expr), inputs


def assert_bits_equal(a, b):
    assert a.shape == b.shape
    diff = np.flatnonzero(a.reshape(-1).view(np.uint32) != b.reshape(-1).view(np.uint32))
    assert diff.size == 0, (diff[:8], a.reshape(-1)[diff[:8]], b.reshape(-1)[diff[:8]])


def ulp_distance(a, b):
    ai = a.reshape(-1).view(np.int32).astype(np.int64)
    bi = b.reshape(-1).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


def assert_close(gpu_out, ref, rel):
    assert gpu_out.shape == ref.shape
    err = np.abs(gpu_out.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)), 1e-30)
    assert err.max() <= rel, (err.max(), np.unravel_index(err.argmax(), err.shape))


# -- config 1: elementwise chain, bit-exact ----------------------------------

@pytest.mark.parametrize("n", [1, 3, 4, 5, 1000, 4099, 1 << 20])
def test_elementwise_bit_exact(gpu, n):
    out, ref, _ = gpu_and_oracle(gpu, "elementwise", {"n": n})
    assert_bits_equal(out, ref)


# -- config 2: strided slice + transpose + concat, bit-exact ------------------

@pytest.mark.parametrize("n", [2, 6, 62, 64, 130, 4096])
def test_view_chain_bit_exact(gpu, n):
    out, ref, (x,) = gpu_and_oracle(gpu, "view_chain", {"n": n})
    assert_bits_equal(out, ref)
    # size-independent closed form y[i, j] = x[2j, 2i+1] + 1 (top half)
    xm = x.reshape(n, n)
    assert np.array_equal(out[: n // 2], xm[0::2, 1::2].T + np.float32(1.0))


@pytest.mark.parametrize("shapes", [([4096, 4096], [4096, 4096]), ([8, 300, 64], [8, 300, 36]),
                                    ([37, 6], [37, 10])])
def test_concat_along_the_last_axis_bit_exact(gpu, shapes):
    """The flat kernel with one branch per group of 4 (splits at multiples
    of 4), and the per-element kernel where a group would straddle it."""
    porch = gpu
    rng = np.random.default_rng(sum(shapes[1]))
    xa = rng.standard_normal(int(np.prod(shapes[0]))).astype(np.float32)
    xb = rng.standard_normal(int(np.prod(shapes[1]))).astype(np.float32)
    axis = len(shapes[0]) - 1
    expr = porch.concat(porch.tensor(shapes[0], xa), porch.tensor(shapes[1], xb), axis) - 0.5
    kind = "pointwise.flat" if shapes[0][-1] % 4 == 0 else "pointwise.scalar"
    assert [k["kind"] for k in porch.plan(expr)["kernels"]] == [kind]
    out = porch.materialize(expr).cpu().reshape(-1)
    assert_bits_equal(out, host.evaluate(expr).reshape(-1))
    want = np.concatenate([xa.reshape(shapes[0]), xb.reshape(shapes[1])], axis) - np.float32(0.5)
    assert np.array_equal(out, want.reshape(-1))


# -- config 3: softmax, 1e-6 relative ----------------------------------------

@pytest.mark.parametrize("size", [{"rows": 3, "cols": 7}, {"rows": 17, "cols": 256},
                                  {"rows": 64, "cols": 4100}, {"rows": 8, "cols": 12288},
                                  {"rows": 300, "cols": 2048}, {"rows": 50, "cols": 3000},
                                  {"rows": 7, "cols": 2050}, {"rows": 8192, "cols": 4096},
                                  # workgroups of 8 and 16 waves; from 131072 on the row exceeds the
                                  # register cache and max and sum run as one online pass
                                  {"rows": 5, "cols": 33000}, {"rows": 3, "cols": 65536},
                                  {"rows": 2, "cols": 131072}, {"rows": 3, "cols": 262147},
                                  {"rows": 40, "cols": 200004}])
def test_softmax_within_1e6(gpu, size):
    # 1e-6 against the oracle beyond its own row-sum drift, and against the
    # float64 softmax of the same differences (assert_softmax_close)
    (x,) = config_inputs("softmax", size)
    shape = config_shapes("softmax", size)[0]
    t = gpu.tensor(shape, x)
    out = gpu.materialize(gpu.softmax(t, 1)).cpu().reshape(shape)
    assert_softmax_close(out, t, x)
    assert np.allclose(out.sum(axis=1), 1.0, atol=2e-5)


def test_softmax_full_size_ulp_histogram(gpu):
    # the workload's size: per-element distance to the oracle in ulp (the
    # oracle's exp is std::exp, the kernel's a polynomial within 1 ulp)
    out, ref, _ = gpu_and_oracle(gpu, "softmax", CONFIG_SIZES["softmax"])
    d = ulp_distance(out, ref)
    counts = {u: int((d == u).sum()) for u in range(4)}
    counts[">3"] = int((d > 3).sum())
    print("softmax [8192,4096] ulp histogram vs oracle:", counts, flush=True)
    assert sum(counts.values()) == out.size
    assert d.max() <= 8


@pytest.mark.parametrize("cols", [4096, 262147])
def test_softmax_special_values_match_oracle(gpu, cols):
    # rows with -inf entries (exp gives 0), one +inf (max is inf: inf - inf
    # is NaN), one NaN (the sum is NaN), and plain rows, on a row held in
    # registers and on one past the register cache (online max and sum)
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((5, cols)).astype(np.float32)
    x[0, ::7] = -np.inf
    x[1, cols // 3] = np.inf
    x[2, cols // 2] = np.nan
    x[3, :] = -np.inf
    x[3, 5] = 0.0
    t = gpu.tensor([5, cols], x.reshape(-1))
    expr = gpu.softmax(t, 1)
    out = gpu.materialize(expr).cpu().reshape(5, cols)
    ref = host.evaluate(expr)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    finite = ~np.isnan(ref)
    np.testing.assert_allclose(out[finite], ref[finite], rtol=1e-6, atol=1e-7)
    assert np.all(np.isnan(out[1])) and np.all(np.isnan(out[2]))
    assert out[3, 5] == 1.0 and np.count_nonzero(out[3]) == 1


@pytest.mark.parametrize("cols, kinds", [(262147, ["row"]), (262148, ["pointwise.flat", "row.split"])])
def test_softmax_online_pass_with_moving_anchors(gpu, cols, kinds):
    """Rows past the register cache run max and sum as one pass with a
    per-lane anchor that moves (rescaling the lane's sum) whenever a value
    exceeds it by more than 64; rows split over workgroups combine parts
    whose maxima lie far apart.  Wide-range rows make the anchors move many
    times within a lane: a scaled normal, a rising ramp, and a sawtooth whose
    teeth rise.  Bar: 1e-6 relative or 2 ulp per element (values far below
    the row max are denormal or zero)."""
    rng = np.random.default_rng(31)
    x = np.empty((4, cols), np.float32)
    x[0] = rng.standard_normal(cols) * 40
    x[1] = np.linspace(-300.0, 300.0, cols)
    x[2] = (np.arange(cols) % 4096) * 0.05 + np.arange(cols) * 1e-3
    x[3] = np.linspace(300.0, -300.0, cols)
    t = gpu.tensor([4, cols], x.reshape(-1))
    expr = gpu.softmax(t, 1)
    plan = gpu.plan(expr)
    assert [k["kind"] for k in plan["kernels"]] == kinds
    assert plan["kernels"][-1]["block"] == (1024 if kinds == ["row"] else 256)
    out = gpu.materialize(expr).cpu().reshape(4, cols)
    assert_softmax_close(out, t, x)
    assert np.allclose(out.sum(axis=1), 1.0, atol=2e-5)


# short rows: several rows per wave (lane segments of 1 to 32), row counts
# that leave the last wave's segments partly empty
@pytest.mark.parametrize("cols", [1, 2, 3, 5, 8, 31, 32, 33, 64, 100, 128, 200, 255])
def test_softmax_short_rows_within_1e6(gpu, cols):
    size = {"rows": 1001, "cols": cols}
    out, ref, _ = gpu_and_oracle(gpu, "softmax", size)
    assert_close(out, ref, 1e-6)
    assert np.allclose(out.sum(axis=1), 1.0, atol=2e-5)


@pytest.mark.parametrize("cols", [1, 4, 7, 16, 40, 128, 260])
def test_logistic_rowsum_short_rows_within_1e5(gpu, cols):
    out, ref, _ = gpu_and_oracle(gpu, "logistic_rowsum", {"rows": 999, "cols": cols})
    assert_close(out, ref, 1e-5)


def test_short_row_sums_exact_on_integers(gpu):
    # integer data: the segment butterflies must add every element once
    rng = np.random.default_rng(17)
    for cols in (1, 3, 8, 24, 64, 96):
        x = rng.integers(-50, 50, size=(777, cols)).astype(np.float32)
        t = gpu.tensor([777, cols], x.reshape(-1))
        out = gpu.materialize(gpu.sum(t, 1)).cpu()
        assert np.array_equal(out, x.sum(axis=1).astype(np.float32)), cols
        mx = gpu.materialize(gpu.max(t, 1)).cpu()
        assert np.array_equal(mx, x.max(axis=1)), cols


# -- config 4: broadcast + logistic + row sum, 1e-5 relative -----------------

@pytest.mark.parametrize("size", [{"rows": 5, "cols": 9}, {"rows": 33, "cols": 2048},
                                  {"rows": 16384, "cols": 2048}, {"rows": 4, "cols": 10000},
                                  {"rows": 100, "cols": 3001}, {"rows": 4097, "cols": 2044},
                                  {"rows": 3, "cols": 70000}])
def test_logistic_rowsum_within_1e5(gpu, size):
    out, ref, _ = gpu_and_oracle(gpu, "logistic_rowsum", size)
    assert_close(out, ref, 1e-5)


# -- config 5: matmul + epilogue, 1e-4 relative ------------------------------

@pytest.mark.parametrize("size", [{"m": 2, "k": 3, "n": 5}, {"m": 67, "k": 129, "n": 33},
                                  {"m": 256, "k": 4096, "n": 128}])
def test_matmul_epilogue_within_1e4(gpu, size):
    out, ref, _ = gpu_and_oracle(gpu, "matmul_epilogue", size)
    assert_close(out, ref, 1e-4)


def test_matmul_epilogue_full_size_every_output(gpu):
    """The 4096^3 workload: every output against a float64 GEMM (the
    product within its accumulation bound, the result within 1e-4), and a
    row sample against the oracle's sequential float32 K loop."""
    porch = gpu
    size = CONFIG_SIZES["matmul_epilogue"]
    a, b, bias = config_inputs("matmul_epilogue")
    m, k, n = size["m"], size["k"], size["n"]
    ta, tb, tbias = porch.tensor([m, k], a), porch.tensor([k, n], b), porch.tensor([1, n], bias)
    out = porch.materialize(config_graph("matmul_epilogue", [ta, tb, tbias])).cpu().reshape(m, n)
    delta, frac = check_matmul_epilogue_every_output(out, a, b, bias, m, k, n)
    print(f"matmul+epilogue 4096^3, all {m * n} outputs: max |delta| = {delta:.3e}, "
          f"max |delta| / bound = {frac:.3e}", flush=True)
    rows = np.array([0, 1, 2, 777, 2048, 4000, 4095])
    sample = porch.tensor([rows.size, k], a.reshape(m, k)[rows])
    ref = host.evaluate(porch.relu(porch.matmul(sample, tb) + porch.broadcast_to(tbias, [rows.size, n])) - 0.5)
    assert_close(out[rows], ref, 1e-4)


def test_matmul_full_size_product_against_float64(gpu):
    # the workload's A @ B without its epilogue, every output, against a
    # float64 GEMM: within the accumulation bound K * eps * sum |a| |b|
    porch = gpu
    size = CONFIG_SIZES["matmul_epilogue"]
    a, b, _ = config_inputs("matmul_epilogue")
    m, k, n = size["m"], size["k"], size["n"]
    am, bm = a.reshape(m, k).astype(np.float64), b.reshape(k, n).astype(np.float64)
    out = porch.materialize(porch.matmul(porch.tensor([m, k], a), porch.tensor([k, n], b))).cpu().reshape(m, n)
    exact = am @ bm
    bound = k * np.finfo(np.float32).eps * (np.abs(am) @ np.abs(bm))
    delta = np.abs(out - exact)
    print(f"matmul 4096^3 pre-epilogue, all outputs: max |delta| = {delta.max():.3e}, "
          f"max |delta| / bound = {(delta / bound).max():.3e}", flush=True)
    assert delta.max() < 5e-6
    assert np.all(delta <= bound)


# -- edge cases the reference's tests touch: empty, ragged, rank-3 ----------

def test_empty_results_and_empty_operands(gpu):
    porch = gpu
    x = porch.tensor([0, 4], [])
    assert porch.materialize(x + 1.0).numel() == 0
    y = porch.tensor([2, 4], np.arange(8, dtype=np.float32))
    # concat with an empty operand (the reference launches with an empty input
    # buffer and throws; porch_amd never reads it)
    out = porch.materialize(porch.concat(x, y, 0))
    assert np.array_equal(out.cpu(), np.arange(8, dtype=np.float32))
    assert porch.materialize(porch.sum(porch.tensor([3, 0], []), 1)).cpu().tolist() == [0, 0, 0]


def test_rank3_views_bit_exact(gpu):
    porch = gpu
    x = (np.arange(5 * 6 * 7, dtype=np.float32) * 0.37).reshape(5, 6, 7)
    t = porch.tensor([5, 6, 7], x)
    cases = [
        porch.tensor(t[porch.slice(1, 5, 2), porch.all, porch.slice(1, 7, 3)]) * 2.0,
        porch.reshape(porch.transpose(porch.reshape(t, [30, 7])), [7, 5, 6]) - 1.0,
        porch.concat(t, porch.tensor(t[porch.all, porch.slice(0, 2)]), 1) + 0.5,
        porch.broadcast_to(porch.unsqueeze(porch.tensor(t[2]), 0), [3, 6, 7]) / 4.0,
        porch.maximum(t, porch.minimum(t * 2.0, 3.0)),
    ]
    for expr in cases:
        assert_bits_equal(porch.materialize(expr).cpu().reshape(expr.shape()), host.evaluate(expr))


def test_reductions_over_every_axis(gpu):
    porch = gpu
    rng = np.random.default_rng(11)
    x = rng.integers(-50, 50, size=(6, 70, 9)).astype(np.float32)
    t = porch.tensor([6, 70, 9], x)
    for axis in range(3):
        for keep in (False, True):
            for op in (porch.sum, porch.max):
                expr = op(t, axis, keep)
                assert_bits_equal(porch.materialize(expr).cpu().reshape(expr.shape()),
                                  host.evaluate(expr))


@pytest.mark.parametrize("shape", [(6, 70, 9), (3, 5, 2100), (130, 7)])
def test_softmax_over_every_axis_within_1e6(gpu, shape):
    """Non-last axes plan the reductions into temporaries (and a column
    reduction); the last axis is one row program."""
    porch = gpu
    rng = np.random.default_rng(sum(shape))
    x = (rng.standard_normal(int(np.prod(shape))) * 3).astype(np.float32)
    t = porch.tensor(list(shape), x)
    for axis in range(len(shape)):
        expr = porch.softmax(t, axis)
        out = porch.materialize(expr).cpu().reshape(shape)
        ref = host.evaluate(expr)
        assert np.all(np.abs(out - ref) <= 1e-6 * np.abs(ref)), (shape, axis)


@pytest.mark.parametrize("shape,axis", [((8192, 300), 0), ((4, 3000, 100), 1), ((2049, 1000), 0)])
def test_long_column_reductions_bit_exact(gpu, shape, axis):
    """Reductions whose axis is split into chunks and recombined; integer
    values keep every order exact, so the result must equal the oracle's."""
    porch = gpu
    rng = np.random.default_rng(shape[0] + axis)
    x = rng.integers(-3, 4, size=int(np.prod(shape))).astype(np.float32)
    t = porch.tensor(list(shape), x)
    for op in (porch.sum, porch.max):
        for keep in (False, True):
            expr = op(t, axis, keep)
            assert porch.plan(expr)["kernels"][0]["grid"][1] > 1  # split
            assert_bits_equal(porch.materialize(expr).cpu().reshape(expr.shape()), host.evaluate(expr))


def test_softmax_over_a_long_first_axis_within_1e6(gpu):
    porch = gpu
    x = (np.random.default_rng(8).standard_normal(6000 * 200) * 3).astype(np.float32)
    t = porch.tensor([6000, 200], x)
    expr = porch.softmax(t, 0)
    # max and sum from one read of x, its axis split in parts, then combined
    assert [k["kind"] for k in porch.plan(expr)["kernels"]] == [
        "reduce.column_softmax", "reduce.column_softmax_combine", "pointwise.flat"]
    out = porch.materialize(expr).cpu().reshape(6000, 200)
    ref = host.evaluate(expr)
    assert np.all(np.abs(out - ref) <= 1e-6 * np.abs(ref))


def test_max_semantics_match_reference(gpu):
    porch = gpu
    t = porch.tensor([2, 5], [-np.inf] * 5 + [1, 2, 3, 4, 5])
    out = porch.materialize(porch.max(t, 1)).cpu()
    assert out[0] == np.float32(-3.4028234663852886e38) and out[1] == 5.0
    a = porch.tensor([3], [np.nan, 1.0, -0.0])
    b = porch.tensor([3], [2.0, np.nan, 0.0])
    hi = porch.materialize(porch.maximum(a, b)).cpu()
    assert hi[0] == 2.0 and np.isnan(hi[1]) and hi[2] == 0.0 and not np.signbit(hi[2])


def test_exp_within_2_ulp_of_host(gpu):
    porch = gpu
    xs = np.concatenate([np.linspace(-87.0, 88.0, 200003), [-104.0, -100.0, -90.0, 0.0, -0.0,
                                                            89.0, np.inf, -np.inf, np.nan]])
    xs = xs.astype(np.float32)
    t = porch.tensor([xs.size], xs)
    out = porch.materialize(porch.exp(t)).cpu()
    ref = host.evaluate(porch.exp(t))
    finite = np.isfinite(ref)
    assert ulp_distance(out[finite], ref[finite]).max() <= 2
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    assert np.array_equal(out[np.isinf(ref)], ref[np.isinf(ref)])


def test_logistic_and_reciprocal(gpu):
    porch = gpu
    xs = np.linspace(-30, 30, 100001).astype(np.float32)
    t = porch.tensor([xs.size], xs)
    out = porch.materialize(porch.logistic(t)).cpu()
    ref = host.evaluate(porch.logistic(t))
    # bar: within 2 ulp or 1e-6 relative (exp's last-bit differences pass
    # through 1 + e and the reciprocal)
    rel = np.abs(out.astype(np.float64) - ref) / np.abs(ref.astype(np.float64))
    assert ((ulp_distance(out, ref) <= 2) | (rel <= 1e-6)).all()
    r = porch.materialize(porch.reciprocal(t)).cpu()
    assert_bits_equal(r, host.evaluate(porch.reciprocal(t)))


# -- seeded random graphs: views and elementwise arithmetic, bit-exact -------

def random_graph(porch, rng, inputs):
    def fresh(shape):
        values = rng.integers(-8, 9, size=int(np.prod(shape))).astype(np.float32) * np.float32(0.5)
        t = porch.tensor(list(shape), values)
        inputs.append(t)
        return porch.tensor_expr(t)

    rank = int(rng.integers(1, 4))
    shape = [int(rng.integers(1, 9)) for _ in range(rank)]
    expr = fresh(shape)
    for _ in range(int(rng.integers(2, 7))):
        shape = expr.shape()
        choice = int(rng.integers(0, 10))
        if choice == 0:
            expr = expr * float(rng.choice([2.0, 0.5, -1.0])) + float(rng.integers(-3, 4))
        elif choice == 1:
            expr = porch.maximum(expr, fresh(shape)) - porch.minimum(expr, 0.5)
        elif choice == 2 and len(shape) == 2:
            expr = porch.transpose(expr)
        elif choice == 3:
            lazy = porch.tensor(expr)  # slicing an expression goes through a pending tensor
            items = []
            for extent in shape:
                start = int(rng.integers(0, extent))
                step = int(rng.integers(1, 3))
                items.append(porch.slice(start, extent, step))
            expr = lazy[tuple(items)]
        elif choice == 4:
            n = int(np.prod(shape))
            factors = [f for f in range(1, n + 1) if n % f == 0]
            f = int(rng.choice(factors))
            expr = porch.reshape(expr, [f, n // f])
        elif choice == 5:
            expr = porch.unsqueeze(expr, int(rng.integers(0, len(shape) + 1)))
        elif choice == 6:
            target = [int(rng.integers(1, 4))] + [e if e != 1 else int(rng.integers(1, 4)) for e in shape]
            expr = porch.broadcast_to(expr, target)
        elif choice == 7:
            axis = int(rng.integers(0, len(shape)))
            other = list(shape)
            other[axis] = int(rng.integers(1, 5))
            expr = porch.concat(expr, fresh(other), axis) if rng.integers(0, 2) else \
                porch.concat(fresh(other), expr, axis)
        elif choice == 8:
            expr = expr + fresh(shape) * 2.0
        else:
            expr = expr / 4.0
        if int(np.prod(expr.shape())) > 4096:
            break
    return expr


def test_random_view_graphs_bit_exact(gpu):
    porch = gpu
    rng = np.random.default_rng(20261201)
    for trial in range(150):
        inputs = []
        expr = random_graph(porch, rng, inputs)
        out = porch.materialize(expr).cpu().reshape(expr.shape())
        ref = host.evaluate(expr)
        assert out.shape == ref.shape, trial
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (trial, porch.plan(expr))


# -- the MFMA GEMM: tile edges, K tails, operand layouts ---------------------

def gemm_bound(a64, b64):
    """Scale of fp32 accumulation error: sum_k |a_ik| |b_kj|."""
    return np.abs(a64) @ np.abs(b64)


@pytest.mark.parametrize("m,k,n", [(200, 1000, 130), (128, 16, 128), (257, 33, 64),
                                   (1024, 4096, 96), (96, 2049, 300)])
def test_mfma_gemm_edges_and_tails(gpu, m, k, n):
    porch = gpu
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    a = rng.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(k, n)).astype(np.float32)
    expr = porch.matmul(porch.tensor([m, k], a), porch.tensor([k, n], b))
    # (1024 x 4096 x 96: eight tiles, split over K, then a combine)
    assert "gemm.mfma" in [x["kind"] for x in porch.plan(expr)["kernels"]]
    out = porch.materialize(expr).cpu().reshape(m, n)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert (np.abs(out - ref) <= 1e-5 * gemm_bound(a.astype(np.float64), b.astype(np.float64)) + 1e-30).all()


@pytest.mark.parametrize("transposed_a", [False, True])
def test_mfma_wide_tiles_with_tails(gpu, transposed_a):
    """Enough rows for 256-row tiles, with tails in m, n and k."""
    porch = gpu
    m, k, n = 4100, 333, 4000
    rng = np.random.default_rng(41 + transposed_a)
    a = rng.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(k, n)).astype(np.float32)
    ta = porch.transpose(porch.tensor([k, m], np.ascontiguousarray(a.T))) if transposed_a \
        else porch.tensor([m, k], a)
    expr = porch.matmul(ta, porch.tensor([k, n], b))
    source = porch.kernel_source(expr, len(porch.plan(expr)["kernels"]) - 1)
    assert "float As[2][2][256]" in source
    out = porch.materialize(expr).cpu().reshape(m, n)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    assert (np.abs(out - a64 @ b64) <= 1e-5 * gemm_bound(a64, b64) + 1e-30).all()


@pytest.mark.parametrize("layout", ["at", "bt", "both", "offset"])
def test_mfma_gemm_operand_layouts(gpu, layout):
    porch = gpu
    m, k, n = 192, 260, 136
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(k, n)).astype(np.float32)
    if layout == "at":
        lhs = porch.transpose(porch.tensor([k, m], np.ascontiguousarray(a.T)))
        rhs = porch.tensor([k, n], b)
    elif layout == "bt":
        lhs = porch.tensor([m, k], a)
        rhs = porch.transpose(porch.tensor([n, k], np.ascontiguousarray(b.T)))
    elif layout == "both":
        lhs = porch.transpose(porch.tensor([k, m], np.ascontiguousarray(a.T)))
        rhs = porch.transpose(porch.tensor([n, k], np.ascontiguousarray(b.T)))
    else:
        # operands as strided sub-views with odd offsets: scalar loads path
        big_a = np.zeros((m + 1, k + 3), dtype=np.float32)
        big_a[1:, 3:] = a
        lhs = porch.tensor([m + 1, k + 3], big_a)[porch.slice(1, m + 1), porch.slice(3, k + 3)]
        rhs = porch.tensor([k, n], b)
    expr = porch.relu(porch.matmul(lhs, rhs)) - 0.25
    out = porch.materialize(expr).cpu().reshape(m, n)
    ref = np.maximum(a.astype(np.float64) @ b.astype(np.float64), 0.0) - 0.25
    bound = gemm_bound(a.astype(np.float64), b.astype(np.float64))
    assert (np.abs(out - ref) <= 1e-5 * bound + 1e-7).all()
    # against the oracle (sequential fp32 sum): both within the bound, and
    # the epilogue's -0.25 cancels, so the comparison is absolute
    assert (np.abs(out - host.evaluate(expr)) <= 2e-5 * bound + 1e-7).all()


def test_mfma_keeps_denormals(gpu):
    # denormal operands (sums of denormals are exact: they are fixed point)
    # and denormal products: the MFMA path must not flush them, as an IEEE
    # fp32 multiply-add (the reference's loop) does not
    porch = gpu
    m, k, n = 256, 64, 256
    rng = np.random.default_rng(21)
    a = (rng.integers(1, 5, size=(m, k)) * np.float32(1e-40)).astype(np.float32)
    b = rng.integers(1, 4, size=(k, n)).astype(np.float32)
    expr = porch.matmul(porch.tensor([m, k], a.reshape(-1)), porch.tensor([k, n], b.reshape(-1)))
    assert porch.plan(expr)["kernels"][0]["kind"] == "gemm.mfma"
    out = porch.materialize(expr).cpu().reshape(m, n)
    assert np.array_equal(out, host.evaluate(expr))
    a2 = (rng.integers(1, 5, size=(m, k)) * np.float32(1e-20)).astype(np.float32)
    b2 = (rng.integers(1, 4, size=(k, n)) * np.float32(1e-20)).astype(np.float32)
    expr2 = porch.matmul(porch.tensor([m, k], a2.reshape(-1)), porch.tensor([k, n], b2.reshape(-1)))
    out2 = porch.materialize(expr2).cpu().reshape(m, n)
    ref2 = host.evaluate(expr2)
    assert np.count_nonzero(out2) == out2.size
    np.testing.assert_allclose(out2, ref2, rtol=1e-5)
