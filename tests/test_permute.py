"""permute: the rank-N axis permutation (an extension; the reference's only
axis reordering is the rank-2 transpose, src/tensor.cpp:1142-1150).

The oracle's permute is pinned against numpy.transpose over every
permutation of ranks 1-4 on ragged shapes, against the reference's own
transpose (permute [1, 0]), and through composition with the inverse
permutation (the identity).  The planner tests pin which kernel class each
form reaches (an inner axis kept in place streams through the flat kernel
with 128-bit loads; a moved inner axis goes through the LDS transpose), and
the GPU tests check every case bit-exact against the oracle.
"""

import itertools

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import placeholder

SHAPES = {1: [7], 2: [5, 9], 3: [3, 5, 7], 4: [2, 3, 5, 4]}


def values(shape, seed=0):
    rng = np.random.default_rng(seed)
    return rng.integers(-1000, 1000, size=shape).astype(np.float32) / np.float32(4)


@pytest.mark.parametrize("rank", sorted(SHAPES))
def test_oracle_permute_matches_numpy_for_every_permutation(rank):
    x = values(SHAPES[rank])
    t = placeholder(SHAPES[rank], x)
    for perm in itertools.permutations(range(rank)):
        out = host.evaluate(porch.permute(t, list(perm)))
        expected = np.transpose(x, perm)
        assert out.shape == expected.shape, perm
        assert np.array_equal(out, expected), perm


def test_oracle_permute_of_rank_two_is_the_reference_transpose():
    x = values([6, 11])
    t = placeholder([6, 11], x)
    assert np.array_equal(host.evaluate(porch.permute(t, [1, 0])), host.evaluate(porch.transpose(t)))


def test_oracle_permute_then_inverse_is_identity():
    x = values([3, 4, 5, 6])
    t = placeholder([3, 4, 5, 6], x)
    for perm in itertools.permutations(range(4)):
        inverse = list(np.argsort(perm))
        assert np.array_equal(host.evaluate(porch.permute(porch.permute(t, list(perm)), inverse)), x)


def test_oracle_planted_mistake_is_caught():
    # reading a 3-cycle with its inverse (a plausible index slip) keeps the
    # shape of a cube but not the values: the numpy check rejects it
    x = values([4, 4, 4])
    t = placeholder([4, 4, 4], x)
    wrong = host.evaluate(porch.permute(t, [int(a) for a in np.argsort([1, 2, 0])]))
    expected = np.transpose(x, (1, 2, 0))
    assert wrong.shape == expected.shape
    assert not np.array_equal(wrong, expected)


@pytest.mark.parametrize("dims", [[0, 0, 1], [0, 1], [0, 1, 3], [0, 1, 2, 3], [-1, 0, 1]])
def test_invalid_permutations_are_rejected(dims):
    t = placeholder([3, 5, 7])
    with pytest.raises(porch.InvalidArgument,
                       match="permute axes must be a permutation of the operand's dimensions"):
        porch.permute(t, dims).shape()


def test_scalar_operand_is_rejected():
    with pytest.raises(porch.InvalidArgument, match="permute operand must be a tensor"):
        porch.permute(porch.tensor_expr(2.0), []).shape()


def test_shape_is_permuted():
    assert porch.permute(placeholder([2, 3, 5, 7]), [3, 1, 0, 2]).shape() == [7, 3, 2, 5]


def batched_transpose(make):
    return porch.permute(make([8, 192, 320]), [0, 2, 1])


def heads_split(make):
    # [batch, seq, heads, dim] -> [batch, heads, seq, dim]: the inner axis stays
    return porch.permute(make([4, 96, 8, 64]), [0, 2, 1, 3]) * 2.0


def heads_to_last(make):
    return porch.permute(make([4, 8, 96, 64]), [0, 2, 3, 1]) + 1.0


def reverse_axes(make):
    return porch.permute(make([33, 65, 17]), [2, 1, 0])


def permute_plus_leaf(make):
    x = make([40, 70, 6])
    return porch.permute(x, [2, 0, 1]) - make([6, 40, 70])


def permute_of_expression(make):
    x = make([24, 36, 10])
    return porch.permute(porch.relu(x) * 3.0 + 1.0, [1, 2, 0])


def sum_over_permuted(make):
    return porch.sum(porch.permute(make([30, 50, 20]), [2, 0, 1]), 2)


def softmax_after_permute(make):
    return porch.softmax(porch.permute(make([16, 48, 40]), [0, 2, 1]), 2)


def matmul_of_permuted(make):
    # [40, 6, 16] -> [40, 96] merges axes with strides 16 and 640: not an
    # affine view, so the operand is materialised first
    a = porch.reshape(porch.permute(make([6, 40, 16]), [1, 0, 2]), [40, 96])
    return porch.matmul(a, make([96, 72]))


def matmul_of_permuted_view(make):
    # [96, 1, 40] -> [1, 40, 96] -> [40, 96]: an affine (transposed) view
    a = porch.reshape(porch.permute(make([96, 1, 40]), [1, 2, 0]), [40, 96])
    return porch.matmul(a, make([96, 72])) + 1.0


# name -> (graph, kernel kinds the planner forms)
CASES = {
    "batched_transpose": (batched_transpose, ["pointwise.tiled"]),
    "heads_split": (heads_split, ["pointwise.flat"]),
    "heads_to_last": (heads_to_last, ["pointwise.tiled"]),
    "reverse_axes": (reverse_axes, ["pointwise.tiled"]),
    "permute_plus_leaf": (permute_plus_leaf, ["pointwise.tiled"]),
    "permute_of_expression": (permute_of_expression, ["pointwise.tiled"]),
    "sum_over_permuted": (sum_over_permuted, None),
    "softmax_after_permute": (softmax_after_permute, None),
    "matmul_of_permuted": (matmul_of_permuted, ["pointwise.scalar", "gemm.mfma"]),
    "matmul_of_permuted_view": (matmul_of_permuted_view, ["gemm.mfma"]),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_permute_cases_plan_and_compile(name):
    fn, kinds = CASES[name]
    expr = fn(placeholder)
    plan = porch.plan(expr, compile=True)
    if kinds is not None:
        assert [k["kind"] for k in plan["kernels"]] == kinds, plan
    assert all(k["code_bytes"] > 0 for k in plan["kernels"])


def test_kept_inner_axis_streams_with_vector_loads():
    source = porch.kernel_source(heads_split(placeholder), 0)
    assert "__builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(a0" in source


@pytest.mark.gpu
def test_permute_cases_bit_exact(gpu):
    rng = np.random.default_rng(31)

    def make(shape):
        v = rng.integers(-64, 64, size=int(np.prod(shape))).astype(np.float32) / np.float32(8)
        return gpu.tensor(list(shape), v)

    for name in sorted(CASES):
        print("permute case", name, flush=True)
        expr = CASES[name][0](make)
        ref = host.evaluate(expr)
        out = gpu.materialize(expr).cpu().reshape(expr.shape())
        if name == "softmax_after_permute":
            # exp differs from the oracle's std::exp by at most a few ulp
            np.testing.assert_allclose(out, ref, rtol=2e-6, atol=1e-7)
        else:
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), name


@pytest.mark.gpu
@pytest.mark.parametrize("rank", [3, 4])
def test_every_permutation_bit_exact(gpu, rank):
    shape = {3: [19, 33, 70], 4: [5, 7, 34, 66]}[rank]
    x = values(shape, seed=rank)
    t = gpu.tensor(shape, x.reshape(-1))
    for perm in itertools.permutations(range(rank)):
        out = gpu.materialize(porch.permute(t, list(perm))).cpu().reshape(np.transpose(x, perm).shape)
        assert np.array_equal(out, np.transpose(x, perm)), perm


@pytest.mark.gpu
def test_large_batched_transpose_bit_exact(gpu):
    shape = [64, 512, 512]
    x = values(shape, seed=5)
    t = gpu.tensor(shape, x.reshape(-1))
    out = gpu.materialize(porch.permute(t, [0, 2, 1])).cpu().reshape(64, 512, 512)
    assert np.array_equal(out, np.transpose(x, (0, 2, 1)))


@pytest.mark.gpu
def test_permute_of_an_empty_tensor(gpu):
    t = gpu.tensor([3, 0, 2], np.zeros(0, np.float32))
    out = gpu.materialize(gpu.permute(t, [2, 0, 1]) * 2.0)
    assert tuple(out.shape()) == (2, 3, 0) and out.cpu().size == 0


@pytest.mark.gpu
def test_heads_permute_benchmark_size_bit_exact(gpu):
    """The benchmark's heads permute, permute(x, [0, 2, 1, 3]) over x
    [32, 1024, 16, 128] on its seeded input: every element moved exactly."""
    from porch_amd.workloads import config_graph, config_inputs, config_shapes
    (shape,) = config_shapes("heads_permute")
    (x,) = config_inputs("heads_permute")
    expr = config_graph("heads_permute", [gpu.tensor(shape, x)])
    out = gpu.materialize(expr).cpu().reshape(shape[0], shape[2], shape[1], shape[3])
    assert np.array_equal(out, np.transpose(np.asarray(x, np.float32).reshape(shape), (0, 2, 1, 3)))

