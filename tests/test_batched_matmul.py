"""batched_matmul: [B, M, K] @ [B, K, N] -> [B, M, N] (an extension; the
reference's matmul is rank-2 only, src/tensor.cpp:366-385).

The oracle's batched product is pinned against numpy's matmul on integer
data (every sum exact in binary32, so order-free), against the oracle's own
rank-2 matmul (the reference's per-element k order) entry by entry, and by a
planted mistake (one entry's operand reused for all).  The planner tests pin
that strided, permuted and broadcast (shared) operands are read in place and
which kernel class each size reaches; the GPU tests check the MFMA and
scalar kernels bit-exact on integer data and within a float64-derived bound
on real-valued data.
"""

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import CONFIG_SIZES, check_matmul_epilogue_every_output, config_graph, config_inputs, placeholder


def ints(shape, rng, lo=-3, hi=4):
    return rng.integers(lo, hi, size=shape).astype(np.float32)


@pytest.mark.parametrize("shape", [(1, 4, 5, 3), (3, 5, 7, 4), (6, 17, 33, 9), (2, 8, 0, 5)])
def test_oracle_matches_numpy(shape):
    b, m, k, n = shape
    rng = np.random.default_rng(sum(shape))
    x, y = ints([b, m, k], rng), ints([b, k, n], rng)
    out = host.evaluate(porch.batched_matmul(placeholder([b, m, k], x), placeholder([b, k, n], y)))
    assert out.shape == (b, m, n)
    assert np.array_equal(out, np.matmul(x.astype(np.float64), y.astype(np.float64)).astype(np.float32))


def test_oracle_entries_equal_rank_two_matmul_bit_for_bit():
    # real-valued data: each entry must follow the rank-2 matmul's k order
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 9, 50)).astype(np.float32)
    y = rng.standard_normal((4, 50, 7)).astype(np.float32)
    out = host.evaluate(porch.batched_matmul(placeholder([4, 9, 50], x), placeholder([4, 50, 7], y)))
    for e in range(4):
        ref = host.evaluate(porch.matmul(placeholder([9, 50], x[e]), placeholder([50, 7], y[e])))
        assert np.array_equal(out[e].view(np.uint32), ref.view(np.uint32)), e


def test_oracle_planted_mistake_is_caught():
    # every entry multiplied by entry 0's right operand: numpy disagrees
    rng = np.random.default_rng(5)
    x, y = ints([3, 4, 6], rng), ints([3, 6, 5], rng)
    wrong = host.evaluate(porch.batched_matmul(
        placeholder([3, 4, 6], x), porch.broadcast_to(placeholder([1, 6, 5], y[:1]), [3, 6, 5])))
    assert not np.array_equal(wrong, np.matmul(x, y))


@pytest.mark.parametrize("lhs, rhs, message", [
    ([2, 3, 4], [3, 4, 5], "batched_matmul batch dimensions must match"),
    ([2, 3, 4], [2, 5, 6], "batched_matmul inner dimensions must match"),
    ([3, 4], [4, 5], "batched_matmul requires rank-3 tensors"),
    ([2, 3, 4], [4, 5], "batched_matmul requires rank-3 tensors"),
])
def test_shape_errors(lhs, rhs, message):
    with pytest.raises(porch.InvalidArgument, match=message):
        porch.batched_matmul(placeholder(lhs), placeholder(rhs)).shape()


def test_scalar_operand_is_rejected():
    with pytest.raises(porch.InvalidArgument, match="batched_matmul operands must be tensors"):
        porch.batched_matmul(placeholder([2, 3, 4]), 2.0).shape()


def test_rank_two_matmul_still_rejects_rank_three():
    # the reference's own rule for matmul is unchanged
    with pytest.raises(porch.InvalidArgument, match="matmul requires rank-2 tensors"):
        porch.matmul(placeholder([2, 3, 4]), placeholder([2, 4, 5])).shape()


def plain(make, b, m, k, n):
    return porch.batched_matmul(make([b, m, k]), make([b, k, n]))


def with_epilogue(make, b, m, k, n):
    bias = porch.broadcast_to(make([1, 1, n]), [b, m, n])
    return porch.relu(porch.batched_matmul(make([b, m, k]), make([b, k, n])) + bias) - 0.5


def shared_weight(make, b, m, k, n):
    # one [k, n] weight for every entry: a broadcast view, batch stride 0
    return porch.batched_matmul(make([b, m, k]), porch.broadcast_to(make([k, n]), [b, k, n]))


def permuted_operands(make, b, m, k, n):
    # A stored [m, b, k] (heads interleaved), B stored [b, n, k] (transposed)
    a = porch.permute(make([m, b, k]), [1, 0, 2])
    bt = porch.permute(make([b, n, k]), [0, 2, 1])
    return porch.batched_matmul(a, bt) * 2.0


def expression_operand(make, b, m, k, n):
    # an operand that is itself arithmetic: materialised first
    return porch.batched_matmul(make([b, m, k]) * 2.0 - 1.0, make([b, k, n]))


def attention_scores(make, b, m, k, n):
    # softmax over the last axis of a batched product (row program after gemm)
    return porch.softmax(porch.batched_matmul(make([b, m, k]), make([b, k, n])) * 0.125, 2)


FORMS = {
    "plain": plain,
    "with_epilogue": with_epilogue,
    "shared_weight": shared_weight,
    "permuted_operands": permuted_operands,
    "expression_operand": expression_operand,
}

SIZES = [(4, 256, 256, 256), (3, 130, 70, 200), (8, 64, 300, 130), (2, 33, 17, 40), (1, 96, 64, 160),
         (5, 1, 40, 64)]


@pytest.mark.parametrize("form", sorted(FORMS))
def test_forms_plan_and_compile(form):
    for size in SIZES:
        plan = porch.plan(FORMS[form](placeholder, *size), compile=True)
        kinds = [k["kind"] for k in plan["kernels"]]
        assert kinds[-1] in ("gemm.mfma", "gemm.scalar"), (form, size, plan)
        if form == "expression_operand":
            assert len(kinds) == 2 and kinds[0].startswith("pointwise"), (size, plan)
        else:
            assert len(kinds) == 1, (form, size, plan)  # operands read in place


def test_large_products_use_mfma_over_every_entry():
    plan = porch.plan(plain(placeholder, 16, 512, 64, 512))
    (kernel,) = plan["kernels"]
    assert kernel["kind"] == "gemm.mfma"
    assert kernel["grid"][0] == 16 * 4 * 4  # (entry, 128x128 tile) pairs


def test_many_tiles_use_persistent_workgroups():
    # more (entry, tile) pairs than two per compute unit: each workgroup
    # walks tiles, prefetching its next tile during the current one's last
    # step (fewer than 512 runs of two column tiles, which the band kernel
    # would take)
    for b, m, k, n in [(15, 1024, 32, 1024), (14, 1024, 40, 1024), (7, 2048, 16, 1024), (13, 1024, 64, 1024),
                       (32, 1024, 36, 1024)]:
        plan = porch.plan(plain(placeholder, b, m, k, n))
        (kernel,) = plan["kernels"]
        assert kernel["kind"] == "gemm.mfma" and kernel["grid"][0] == 512, (b, m, k, n)
        assert "rr += gridDim.x" in porch.kernel_source(plain(placeholder, b, m, k, n), 0)
    # exactly 512 tiles, or a K of 5 steps and more, keep one workgroup per tile
    for expr in (porch.matmul(placeholder([2048, 32]), placeholder([32, 4096])),
                 plain(placeholder, 32, 1024, 80, 1024)):
        assert "rr += gridDim.x" not in porch.kernel_source(expr, 0)


def test_shared_weight_has_no_batch_offset():
    source = porch.kernel_source(shared_weight(placeholder, 4, 256, 256, 256), 0)
    assert "const float* __restrict__ B = a1 + 0;" in source
    assert "const float* __restrict__ A = a0 + 0 + qb * 65536;" in source


def test_softmax_over_product_forms_gemm_then_row():
    kinds = [k["kind"] for k in porch.plan(attention_scores(placeholder, 4, 128, 64, 128))["kernels"]]
    assert kinds == ["gemm.mfma", "row"]


@pytest.mark.gpu
def test_batched_forms_bit_exact_on_integers(gpu):
    rng = np.random.default_rng(8)

    def make(shape):
        return gpu.tensor(list(shape), ints(shape, rng).reshape(-1))

    for form in sorted(FORMS):
        for size in SIZES:
            print("batched case", form, size, flush=True)
            expr = FORMS[form](make, *size)
            ref = host.evaluate(expr)
            out = gpu.materialize(expr).cpu().reshape(expr.shape())
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (form, size)


@pytest.mark.gpu
def test_batched_real_values_within_float64_bound(gpu):
    rng = np.random.default_rng(9)
    b, m, k, n = 6, 384, 512, 320
    x = rng.uniform(-1, 1, size=(b, m, k)).astype(np.float32)
    y = rng.uniform(-1, 1, size=(b, k, n)).astype(np.float32)
    out = gpu.materialize(porch.batched_matmul(gpu.tensor([b, m, k], x.reshape(-1)),
                                               gpu.tensor([b, k, n], y.reshape(-1)))).cpu().reshape(b, m, n)
    exact = np.matmul(x.astype(np.float64), y.astype(np.float64))
    # |sum error| <= k * eps * sum |x||y| for any summation order
    bound = k * np.finfo(np.float32).eps * np.matmul(np.abs(x).astype(np.float64), np.abs(y).astype(np.float64))
    assert np.all(np.abs(out - exact) <= bound)


# shapes with more tiles than resident workgroups and a short K: even K-step
# counts (loads two slices ahead) and odd ones (the LDS buffer parity
# carried across tiles), a ragged K, ragged rows, a single step, and the
# rank-2 product with a transposed operand (batch counts kept below the
# two workgroups a compute unit that would take the band kernel)
PERSISTENT = [
    (lambda make: plain(make, 12, 1024, 64, 1024)),
    (lambda make: with_epilogue(make, 14, 1024, 40, 1024)),
    (lambda make: plain(make, 20, 1020, 36, 1024)),
    (lambda make: shared_weight(make, 20, 1024, 32, 768)),
    (lambda make: with_epilogue(make, 40, 512, 16, 516)),
    (lambda make: porch.matmul(make([5116, 20]), porch.transpose(make([5120, 20]))) * 2.0),
]


@pytest.mark.gpu
def test_persistent_products_bit_exact(gpu):
    rng = np.random.default_rng(11)

    def make(shape):
        return gpu.tensor(list(shape), ints(shape, rng).reshape(-1))

    for i, build in enumerate(PERSISTENT):
        print("persistent case", i, flush=True)
        expr = build(make)
        kernel = gpu.plan(expr)["kernels"][-1]
        assert kernel["kind"] == "gemm.mfma"
        assert "rr += gridDim.x" in gpu.kernel_source(expr, len(gpu.plan(expr)["kernels"]) - 1), i
        ref = host.evaluate(expr)
        out = gpu.materialize(expr).cpu().reshape(expr.shape())
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), i


def random_persistent_product(rng, make):
    """A product with more than 512 tiles and K of 4 to 64 (the persistent
    kernel, which needs 128-bit operand loads: K and the contiguous extent
    of each operand multiples of 4), ragged row counts, operands that are
    plain, transposed or permuted views or shared weights, and a random
    epilogue."""
    k = 4 * int(rng.integers(1, 17))
    if rng.integers(0, 3):
        b, m, n = int(rng.integers(6, 40)), int(rng.integers(400, 1100)), 4 * int(rng.integers(100, 275))
        b = max(b, 600 // (((m + 127) // 128) * ((n + 127) // 128)) + 1)
        form = int(rng.integers(0, 3))
        if form == 0:
            expr = plain(make, b, m, k, n)
        elif form == 1:
            expr = shared_weight(make, b, m, k, n)
        else:
            expr = permuted_operands(make, b, m, k, n)
    else:
        transposed_a = bool(rng.integers(0, 2))
        m = int(rng.integers(2900, 5200)) // (4 if transposed_a else 1) * (4 if transposed_a else 1)
        n = 4 * int(rng.integers(725, 1300))
        a = porch.transpose(make([k, m])) if transposed_a else make([m, k])
        bt = porch.transpose(make([n, k])) if rng.integers(0, 2) else make([k, n])
        expr = porch.matmul(a, bt)
    if rng.integers(0, 2):
        shape = expr.shape()
        bias = porch.broadcast_to(make([1] * (len(shape) - 1) + [shape[-1]]), shape)
        expr = porch.relu(expr + bias) - 2.0
    return expr


def test_random_persistent_products_plan_as_persistent():
    rng = np.random.default_rng(12)
    count = 0
    for _ in range(16):
        expr = random_persistent_product(rng, placeholder)
        kernel = porch.plan(expr)["kernels"][-1]
        if kernel["kind"] == "gemm.mfma" and "rr += gridDim.x" in porch.kernel_source(expr, len(porch.plan(expr)["kernels"]) - 1):
            count += 1
    assert count >= 10


@pytest.mark.gpu
def test_random_persistent_products_bit_exact(gpu):
    rng = np.random.default_rng(13)

    def make(shape):
        return gpu.tensor(list(shape), ints(shape, rng).reshape(-1))

    for trial in range(12):
        expr = random_persistent_product(rng, make)
        plan = gpu.plan(expr)
        print("persistent fuzz", trial, expr.shape(), [k["grid"][0] for k in plan["kernels"]], flush=True)
        ref = host.evaluate(expr)
        out = gpu.materialize(expr).cpu().reshape(expr.shape())
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), (trial, plan)


@pytest.mark.gpu
def test_softmax_of_batched_scores(gpu):
    rng = np.random.default_rng(10)

    def make(shape):
        return gpu.tensor(list(shape), ints(shape, rng).reshape(-1))

    expr = attention_scores(make, 4, 128, 64, 128)
    ref = host.evaluate(expr)
    out = gpu.materialize(expr).cpu().reshape(expr.shape())
    np.testing.assert_allclose(out, ref, rtol=2e-6, atol=1e-7)


@pytest.mark.gpu
def test_softmax_of_persistent_scores(gpu):
    # the persistent product writes a temporary that the row program reads
    rng = np.random.default_rng(14)

    def make(shape):
        return gpu.tensor(list(shape), ints(shape, rng).reshape(-1))

    expr = attention_scores(make, 12, 1024, 64, 1024)
    plan = gpu.plan(expr)
    assert [k["kind"] for k in plan["kernels"]] == ["gemm.mfma", "row"]
    assert "rr += gridDim.x" in gpu.kernel_source(expr, 0)
    ref = host.evaluate(expr)
    out = gpu.materialize(expr).cpu().reshape(expr.shape())
    np.testing.assert_allclose(out, ref, rtol=2e-6, atol=1e-7)


@pytest.mark.gpu
@pytest.mark.parametrize("shape_a, shape_b", [([2, 3, 0], [2, 0, 4]), ([0, 3, 5], [0, 5, 4]),
                                              ([2, 0, 5], [2, 5, 4])])
def test_empty_extents(gpu, shape_a, shape_b):
    # an empty inner axis gives zeros (the sum of no products); an empty
    # batch or row axis gives an empty result
    a = gpu.tensor(shape_a, np.zeros(int(np.prod(shape_a)), np.float32))
    b = gpu.tensor(shape_b, np.zeros(int(np.prod(shape_b)), np.float32))
    out = gpu.materialize(gpu.batched_matmul(a, b) + 1.0)
    expected_shape = (shape_a[0], shape_a[1], shape_b[2])
    assert tuple(out.shape()) == expected_shape
    assert np.array_equal(out.cpu().reshape(expected_shape), np.ones(expected_shape, np.float32))


@pytest.mark.gpu
def test_attention_scores_every_output(gpu):
    """The benchmark's attention product, batched_matmul(q, k) * 0.125 over
    16 heads of [4096, 64] @ [64, 4096], on its seeded inputs: all 268 M
    outputs against a float64 product of the same float32 operands, within
    the accumulation bound (K - 1) 2^-24 sum |q||k| (scaled like the
    product; the scale by a power of two is exact), head by head."""
    size = CONFIG_SIZES["attention_scores"]
    nb, m, k, n = size["batch"], size["m"], size["k"], size["n"]
    q, kt = config_inputs("attention_scores")
    expr = config_graph("attention_scores", [gpu.tensor([nb, m, k], q), gpu.tensor([nb, k, n], kt)])
    assert [x["kind"] for x in gpu.plan(expr)["kernels"]] == ["gemm.band"]
    out = gpu.materialize(expr).cpu().reshape(nb, m, n)
    q64 = np.asarray(q, np.float32).reshape(nb, m, k).astype(np.float64)
    k64 = np.asarray(kt, np.float32).reshape(nb, k, n).astype(np.float64)
    worst = 0.0
    for h in range(nb):
        exact = (q64[h] @ k64[h]) * 0.125
        bound = (k - 1) * 2.0 ** -24 * 0.125 * (np.abs(q64[h]) @ np.abs(k64[h]))
        frac = np.abs(out[h].astype(np.float64) - exact) / bound
        worst = max(worst, float(frac.max()))
        assert np.all(frac <= 1.0), (h, float(frac.max()), np.unravel_index(frac.argmax(), frac.shape))
    print("attention scores: max |err| / bound", worst)


@pytest.mark.gpu
def test_batched_matmul_benchmark_size_every_output(gpu):
    """The benchmark's batched product, relu(batched_matmul(A, B) + bias) -
    0.5 over 32 entries of [1024, 1024] @ [1024, 1024] on its seeded inputs:
    every output of every entry against a float64 product (the product
    within the accumulation bound, the result within 1e-4 relative)."""
    size = CONFIG_SIZES["batched_matmul"]
    nb, m, k, n = size["batch"], size["m"], size["k"], size["n"]
    a, b, bias = config_inputs("batched_matmul")
    expr = config_graph("batched_matmul", [gpu.tensor([nb, m, k], a), gpu.tensor([nb, k, n], b),
                                           gpu.tensor([1, 1, n], bias)])
    out = gpu.materialize(expr).cpu().reshape(nb, m, n)
    a3 = np.asarray(a, np.float32).reshape(nb, m, k)
    b3 = np.asarray(b, np.float32).reshape(nb, k, n)
    for e in range(nb):
        check_matmul_epilogue_every_output(out[e], a3[e], b3[e], bias, m, k, n)

