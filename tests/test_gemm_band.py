"""Products with a short K over many bands of rows (kernel kind gemm.band):
one workgroup per batch entry, 128-row band and run of column tiles, A held
in registers, the tiles walked with B through LDS, results stored as float4
rows through LDS.  The plan's choice, exactness on integer data (in CPU
emulation and on the GPU, against the oracle) and real data within the
matmul's accumulation bound (K - 1) 2^-24 sum |a||b| against float64."""

import re

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import placeholder
from tests.kernel_emu import emulate as emu

needs_clang = pytest.mark.skipif(not emu.available(), reason="host clang++ from ROCm is required")


def _kinds(expr):
    return [k["kind"] for k in porch.plan(expr)["kernels"]]


def _ints(shape, seed):
    return np.random.default_rng(seed).integers(-3, 4, size=shape).astype(np.float32)


def _reals(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def _product(a, b, batched):
    return porch.batched_matmul(a, b) if batched else porch.matmul(a, b)


# name: (A shape, B shape, graph over (product, bias tensor or None), epilogue on the float64 product
# and bias, bias shape or None)
CASES = {
    "attention-shaped, scaled": (
        [16, 4096, 64], [16, 64, 4096], lambda p, c: p * 0.125, lambda p, c: p * 0.125, None),
    "bias and relu, K of 16": (
        [4, 16384, 16], [4, 16, 256], lambda p, c: porch.relu(p + porch.broadcast_to(c, [4, 16384, 256])),
        lambda p, c: np.maximum(p + c, 0.0), [1, 1, 256]),
    "ragged last band and tile, K of 8": (
        [2, 32700, 8], [2, 8, 300], lambda p, c: p - porch.broadcast_to(c, [2, 32700, 300]),
        lambda p, c: p - c, [1, 1, 300]),
    "unbatched": (
        [65536, 64], [64, 512], lambda p, c: p, lambda p, c: p, None),
    "runs of column tiles": (
        [4096, 64], [64, 4096], lambda p, c: p * 2.0, lambda p, c: p * 2.0, None),
    "runs, the last of one tile, K of 8, bias": (
        [6016, 8], [8, 3968], lambda p, c: p + porch.broadcast_to(c, [6016, 3968]),
        lambda p, c: p + c, [1, 3968]),
    # staging passes over 10, 6 and 14 steps; non-temporal stores past K = 32
    "ragged runs, K of 40": (
        [8, 1000, 40], [8, 40, 2000], lambda p, c: p * 2.0, lambda p, c: p * 2.0, None),
    "K of 24": (
        [4, 4096, 24], [4, 24, 1024], lambda p, c: p, lambda p, c: p, None),
    "K of 56, bias": (
        [4, 8192, 56], [4, 56, 512], lambda p, c: p + porch.broadcast_to(c, [4, 8192, 512]),
        lambda p, c: p + c, [1, 1, 512]),
}


def _groups(sa, sb, cus=256):
    """Workgroups of the band kernel: bands of 128 rows, each split into
    runs of at least two column tiles until there are two a CU."""
    batch = sa[0] if len(sa) == 3 else 1
    bands = batch * -(-sa[-2] // 128)
    tiles = -(-sb[-1] // 128)
    chunks = min(max(1, -(-2 * cus // bands)), max(1, tiles // 2))
    per = -(-tiles // chunks)
    return bands * -(-tiles // per)


def _graph(name, make):
    sa, sb, graph, _, sbias = CASES[name]
    tensors = [make(sa, 1), make(sb, 2)] + ([make(sbias, 3)] if sbias else [])
    bias = tensors[2] if sbias else None
    return graph(_product(tensors[0], tensors[1], len(sa) == 3), bias), tensors


@pytest.mark.parametrize("name", sorted(CASES))
def test_band_products_take_the_band_kernel(name):
    expr, _ = _graph(name, lambda s, seed: placeholder(s))
    plan = porch.plan(expr, compile=True)
    assert [k["kind"] for k in plan["kernels"]] == ["gemm.band"]
    sa, sb = CASES[name][0], CASES[name][1]
    assert plan["kernels"][0]["grid"][0] == _groups(sa, sb)
    assert plan["temps"] == []


def test_band_bounds():
    # K from 8 to 64 in steps of 8, 256 columns or more, at least two bands
    # of 128 rows per compute unit (512 on 256 CUs)
    def kind(sa, sb):
        return _kinds(porch.batched_matmul(placeholder(sa), placeholder(sb)))[0]
    assert kind([16, 4096, 64], [16, 64, 4096]) == "gemm.band"
    assert kind([16, 4096, 72], [16, 72, 4096]) == "gemm.mfma"
    assert kind([16, 4096, 60], [16, 60, 4096]) == "gemm.mfma"
    assert kind([16, 4096, 8], [16, 8, 4096]) == "gemm.band"
    assert kind([16, 4096, 64], [16, 64, 256]) == "gemm.band"
    assert kind([16, 4096, 64], [16, 64, 252]) == "gemm.mfma"
    assert kind([16, 4096, 64], [16, 64, 128]) == "gemm.mfma"
    assert kind([1, 65408, 64], [1, 64, 256]) == "gemm.mfma"   # 511 bands of two tiles
    assert kind([1, 65409, 64], [1, 64, 256]) == "gemm.band"   # 512, the last of one row
    # fewer bands: runs of at least two column tiles, up to two workgroups a CU
    assert kind([2, 8192, 64], [2, 64, 8192]) == "gemm.band"   # 128 bands x 4 runs
    assert kind([8, 1024, 64], [8, 64, 1024]) == "gemm.mfma"   # 64 bands x 4 runs of 2
    # B stored transposed (k^T as a view of k [n, K]): read along K
    assert _kinds(porch.batched_matmul(placeholder([16, 4096, 64]),
                                       porch.permute(placeholder([16, 4096, 64]), [0, 2, 1])))[0] == "gemm.band"
    # neither B's rows nor its columns contiguous: a strided view of both
    assert _kinds(porch.batched_matmul(placeholder([16, 4096, 64]),
                                       placeholder([16, 128, 8192])[:, ::2, ::2]))[0] == "gemm.mfma"


# The kernel needs two workgroups a compute unit (at least ~16 M outputs),
# so the emulation runs the grid's first two and last two workgroups: the
# first band and run, and the last band and run of the last batch entry
# (ragged rows, ragged or single-tile runs).  Every output of every case is
# compared with the oracle on the GPU.  (The attention-shaped case, 1 GiB of
# outputs, takes the path of the two other cases with K of 64.)
@needs_clang
@pytest.mark.parametrize("name", sorted(set(CASES) - {"attention-shaped, scaled"}))
def test_emulated_band_products_are_exact(name):
    xs = {}

    def make(shape, seed):
        xs[seed] = _ints(shape, seed)
        return placeholder(shape, xs[seed])

    expr, _ = _graph(name, make)
    assert _kinds(expr) == ["gemm.band"]
    want = np.asarray(host.evaluate(expr), np.float32)
    assert emu.check_edges(expr, [xs[s] for s in sorted(xs)], want) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_band_products_bit_exact_on_integers(gpu, name):
    expr, _ = _graph(name, lambda s, seed: gpu.tensor(s, _ints(s, seed).reshape(-1)))
    assert [k["kind"] for k in gpu.plan(expr)["kernels"]] == ["gemm.band"]
    out = gpu.materialize(expr).cpu()
    ref = np.asarray(host.evaluate(expr), np.float32).reshape(-1)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_band_products_within_the_accumulation_bound(gpu, name):
    sa, sb, _, epi, sbias = CASES[name]
    vals = {1: _reals(sa, 11), 2: _reals(sb, 12)}
    if sbias:
        vals[3] = _reals(sbias, 13)
    expr, _ = _graph(name, lambda s, seed: gpu.tensor(s, vals[seed].reshape(-1)))
    out = gpu.materialize(expr).cpu().reshape(expr.shape()).astype(np.float64)
    a64, b64 = vals[1].astype(np.float64), vals[2].astype(np.float64)
    k = sa[-1]
    exact = np.matmul(a64, b64)
    bound = (k - 1) * 2.0 ** -24 * np.matmul(np.abs(a64), np.abs(b64))
    bias64 = vals[3].astype(np.float64) if sbias else None
    want = epi(exact, bias64)
    # the product's bound carried through the epilogue (a scale by 1/8 is
    # exact, relu does not widen an error), plus half an ulp of the result
    # for the one rounded add or subtract after the product
    scale = 0.125 if name.startswith("attention") else 2.0 if name in ("runs of column tiles", "ragged runs, K of 40") else 1.0
    slack = scale * bound + np.abs(want) * 2.0 ** -24
    frac = np.abs(out - want) / np.maximum(slack, 1e-300)
    assert np.all(frac <= 1.0), (float(frac.max()), np.unravel_index(frac.argmax(), frac.shape))


def _random_band_graph(make, form, b, m, k, n, epi):
    """Graph `form` of a short-K product: 0 batched, 1 unbatched, 2 one
    weight shared by every entry (B a broadcast view), 3 batched and 4
    unbatched with B stored transposed (a permuted or transposed view),
    with epilogue `epi` (0 none, 1 a scale, 2 relu of a bias add, less a
    half, 3 a bias subtracted)."""
    if form == 1:
        p = porch.matmul(make([m, k]), make([k, n]))
        out_shape, bias_shape = [m, n], [1, n]
    elif form == 3:
        p = porch.batched_matmul(make([b, m, k]), porch.permute(make([b, n, k]), [0, 2, 1]))
        out_shape, bias_shape = [b, m, n], [1, 1, n]
    elif form == 4:
        p = porch.matmul(make([m, k]), porch.transpose(make([n, k])))
        out_shape, bias_shape = [m, n], [1, n]
    elif form == 2:
        p = porch.batched_matmul(make([b, m, k]), porch.broadcast_to(make([k, n]), [b, k, n]))
        out_shape, bias_shape = [b, m, n], [1, 1, n]
    else:
        p = porch.batched_matmul(make([b, m, k]), make([b, k, n]))
        out_shape, bias_shape = [b, m, n], [1, 1, n]
    if epi == 1:
        return p * 0.25
    if epi == 2:
        return porch.relu(p + porch.broadcast_to(make(bias_shape), out_shape)) - 0.5
    if epi == 3:
        return p - porch.broadcast_to(make(bias_shape), out_shape)
    return p


def random_band_product(rng):
    """Shape and form of a product the band kernel takes, drawn until the
    plan says so: K of 8 to 64 in steps of 8, 256 to 3196 columns (a
    multiple of 4, the last tile often ragged), ragged row counts, batched,
    unbatched, with a shared weight or with B stored transposed, and a
    random epilogue; at most 40 M outputs."""
    while True:
        k = 8 * int(rng.integers(1, 9))
        n = 4 * int(rng.integers(64, 800))
        form = int(rng.integers(0, 5))
        b = 1 if form in (1, 4) else int(rng.integers(1, 9))
        m = int(rng.integers(100, 20000))
        epi = int(rng.integers(0, 4))
        if b * m * n > 40_000_000:
            continue
        expr = _random_band_graph(lambda s: placeholder(s), form, b, m, k, n, epi)
        if _kinds(expr) == ["gemm.band"]:
            return form, b, m, k, n, epi


def test_random_band_products_plan_as_band():
    rng = np.random.default_rng(21)
    shapes = [random_band_product(rng) for _ in range(12)]
    assert len({s[3] for s in shapes}) >= 4            # several K
    assert any(s[2] % 128 for s in shapes) and any(s[4] % 128 for s in shapes)  # ragged edges
    forms = {s[0] for s in shapes}
    assert len(forms) >= 4 and forms & {3, 4}            # B stored transposed among them


@pytest.mark.gpu
def test_random_band_products_bit_exact(gpu):
    rng = np.random.default_rng(21)
    data = np.random.default_rng(22)
    for trial in range(12):
        form, b, m, k, n, epi = random_band_product(rng)

        def make(shape):
            return gpu.tensor(list(shape), _ints(shape, int(data.integers(0, 1 << 30))).reshape(-1))

        expr = _random_band_graph(make, form, b, m, k, n, epi)
        plan = gpu.plan(expr)
        print("band fuzz", trial, (form, b, m, k, n, epi), plan["kernels"][0]["grid"][0], flush=True)
        assert [x["kind"] for x in plan["kernels"]] == ["gemm.band"]
        out = gpu.materialize(expr).cpu()
        ref = np.asarray(host.evaluate(expr), np.float32).reshape(-1)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (trial, form, b, m, k, n, epi)


# B stored transposed: (A shape, shape of the tensor whose transpose is B,
# graph over (product, bias or None), epilogue on the float64 product and
# bias, bias shape or None)
TRANSPOSED = {
    "attention-shaped, k^T a view": (
        [4, 4096, 64], [4, 2048, 64], lambda p, c: p * 0.125, lambda p, c: p * 0.125, None),
    "unbatched, ragged tile, K of 32, bias": (
        [16384, 32], [1000, 32], lambda p, c: p + porch.broadcast_to(c, [16384, 1000]),
        lambda p, c: p + c, [1, 1000]),
    "ragged band, K of 8": (
        [2, 32700, 8], [2, 300, 8], lambda p, c: p, lambda p, c: p, None),
}


def _transposed_graph(name, make):
    sa, sk, graph, _, sbias = TRANSPOSED[name]
    tensors = [make(sa, 1), make(sk, 2)] + ([make(sbias, 3)] if sbias else [])
    if len(sa) == 3:
        p = porch.batched_matmul(tensors[0], porch.permute(tensors[1], [0, 2, 1]))
    else:
        p = porch.matmul(tensors[0], porch.transpose(tensors[1]))
    return graph(p, tensors[2] if sbias else None)


@pytest.mark.parametrize("name", sorted(TRANSPOSED))
def test_transposed_b_takes_the_band_kernel(name):
    expr = _transposed_graph(name, lambda s, seed: placeholder(s))
    plan = porch.plan(expr, compile=True)
    assert [k["kind"] for k in plan["kernels"]] == ["gemm.band"]
    sa, sk = TRANSPOSED[name][0], TRANSPOSED[name][1]
    sb = sk[:-2] + [sk[-1], sk[-2]]
    assert plan["kernels"][0]["grid"][0] == _groups(sa, sb)
    # B's columns are read in place (no copy of the transpose)
    assert plan["temps"] == []


@needs_clang
def test_edge_emulation_catches_a_dropped_store_guard():
    # without the guard on ragged bands and tiles, the last workgroup's
    # stores run past the output
    expr, _ = _graph("ragged runs, K of 40", lambda s, seed: placeholder(s))
    plan = porch.plan(expr)
    kernel = plan["kernels"][0]
    source = porch.kernel_source(expr, 0)
    planted = re.sub(r"\n *if \(q0 < \d+ && q1 < \d+\)", "", source)
    assert planted != source
    _, _, _, inputs, _ = porch.serialize(expr._root)
    sizes = [int(np.prod(t.shape())) for t in inputs] + [int(np.prod(plan["out_shape"]))]
    edges = emu.edge_blocks(kernel["grid"][0])
    ok, _ = emu.run_kernel(planted, kernel["name"], sizes, kernel["grid"], kernel["block"], only=edges)
    assert not ok
    ok, detail = emu.run_kernel(source, kernel["name"], sizes, kernel["grid"], kernel["block"], only=edges)
    assert ok, detail


@needs_clang
@pytest.mark.parametrize("name", sorted(TRANSPOSED))
def test_emulated_transposed_b_is_exact(name):
    xs = {}

    def make(shape, seed):
        xs[seed] = _ints(shape, seed)
        return placeholder(shape, xs[seed])

    expr = _transposed_graph(name, make)
    assert _kinds(expr) == ["gemm.band"]
    want = np.asarray(host.evaluate(expr), np.float32)
    assert emu.check_edges(expr, [xs[s] for s in sorted(xs)], want) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(TRANSPOSED))
def test_transposed_b_bit_exact_on_integers(gpu, name):
    expr = _transposed_graph(name, lambda s, seed: gpu.tensor(s, _ints(s, seed).reshape(-1)))
    assert [k["kind"] for k in gpu.plan(expr)["kernels"]] == ["gemm.band"]
    out = gpu.materialize(expr).cpu()
    ref = np.asarray(host.evaluate(expr), np.float32).reshape(-1)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(TRANSPOSED))
def test_transposed_b_within_the_accumulation_bound(gpu, name):
    sa, sk, _, epi, sbias = TRANSPOSED[name]
    vals = {1: _reals(sa, 31), 2: _reals(sk, 32)}
    if sbias:
        vals[3] = _reals(sbias, 33)
    expr = _transposed_graph(name, lambda s, seed: gpu.tensor(s, vals[seed].reshape(-1)))
    out = gpu.materialize(expr).cpu().reshape(expr.shape()).astype(np.float64)
    a64 = vals[1].astype(np.float64)
    b64 = np.swapaxes(vals[2].astype(np.float64), -1, -2)
    k = sa[-1]
    bound = (k - 1) * 2.0 ** -24 * np.matmul(np.abs(a64), np.abs(b64))
    want = epi(np.matmul(a64, b64), vals[3].astype(np.float64) if sbias else None)
    scale = 0.125 if name.startswith("attention") else 1.0
    slack = scale * bound + np.abs(want) * 2.0 ** -24
    frac = np.abs(out - want) / np.maximum(slack, 1e-300)
    assert np.all(frac <= 1.0), (float(frac.max()), np.unravel_index(frac.argmax(), frac.shape))
