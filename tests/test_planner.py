"""The planner's kernel choices and offline hiprtc compilation (no GPU)."""

import re

import pytest

import porch_amd as porch
from tests.helpers import config_graph, config_shapes, placeholder

EXPECTED_KIND = {
    "elementwise": "pointwise.flat",
    "view_chain": "pointwise.tiled",
    "softmax": "row",
    "logistic_rowsum": "row",
    "matmul_epilogue": "gemm",
}


@pytest.mark.parametrize("name", sorted(EXPECTED_KIND))
def test_each_benchmark_graph_is_one_fused_kernel(name):
    tensors = [placeholder(s) for s in config_shapes(name)]
    plan = porch.plan(config_graph(name, tensors), compile=True)
    assert len(plan["kernels"]) == 1, plan
    assert plan["temps"] == []
    kernel = plan["kernels"][0]
    assert kernel["kind"].startswith(EXPECTED_KIND[name]), kernel
    assert kernel["code_bytes"] > 0 and kernel["dest"] == "output"


def test_softmax_reads_the_row_once():
    x = placeholder([8192, 4096])
    source = porch.kernel_source(porch.softmax(x, 1))
    # one 128-bit (non-temporal: read once) load per column chunk, in the
    # first pass only, and 128-bit stores of the result
    assert source.count("__builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(a0") == 1
    assert source.count("*reinterpret_cast<float4*>(out + ") == 1
    assert len(re.findall(r"\bexpf\(", source)) == 4  # one pass, four lanes


def test_flat_kernel_streams_leaves_read_once():
    # each element of x is read once: non-temporal; the broadcast row w is
    # re-read by every row: an ordinary (cached) 128-bit load
    x = placeholder([64, 2048])
    w = placeholder([1, 2048])
    source = porch.kernel_source(x * porch.broadcast_to(w, [64, 2048]), 0)
    assert "__builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(a0 + " in source
    assert "*reinterpret_cast<const float4*>(a1 + " in source


@pytest.mark.parametrize("widths, kind", [
    ((4096, 4096), "pointwise.flat"),   # the split at a multiple of 4: float4 per lane, one branch per group
    ((8, 12), "pointwise.flat"),
    ((6, 10), "pointwise.scalar"),      # a group of 4 would straddle the split
    ((5, 11), "pointwise.scalar"),
])
def test_concat_along_the_last_axis(widths, kind):
    a, b = widths
    expr = porch.concat(placeholder([64, a]), placeholder([64, b]), 1) + 1.0
    assert [k["kind"] for k in porch.plan(expr)["kernels"]] == [kind]
    if kind == "pointwise.flat":
        source = porch.kernel_source(expr, 0)
        assert source.count("__builtin_nontemporal_load(reinterpret_cast<const porch_v4f*>(") == 2
        assert "make_float4(" in source


def test_shared_reductions_are_materialised_once():
    """softmax over a non-last axis cannot be one row program; its max is
    still computed once (the reference computes it twice): with its sum in
    one kernel, or, where the max is also read elsewhere, as its own column
    reduction feeding both."""
    x = placeholder([64, 32])
    plan = porch.plan(porch.softmax(x, 0))
    assert [k["kind"] for k in plan["kernels"]] == ["reduce.column_softmax", "pointwise.flat"]
    assert plan["temps"] == [2 * 32]  # the max and the sum side by side
    m = porch.broadcast_to(porch.max(x, 0, True), [64, 32])
    plan = porch.plan(porch.softmax(x, 0) * m)
    kinds = [k["kind"] for k in plan["kernels"]]
    assert kinds.count("reduce.column") == 2, kinds  # max and sum, once each
    assert len(plan["temps"]) == 2


def test_long_column_reductions_split_the_axis():
    """Few outputs over a long axis: partial folds over chunks of the axis
    (grid y), then one pass combining them in order."""
    plan = porch.plan(porch.sum(placeholder([8192, 4096]), 0), compile=True)
    first, second = plan["kernels"]
    assert first["kind"] == second["kind"] == "reduce.column"
    parts = first["grid"][1]
    assert parts > 1 and first["dest"] == "temp0" and second["dest"] == "output"
    assert plan["temps"] == [parts * 4096]
    # enough outputs to fill the machine: one kernel
    assert len(porch.plan(porch.sum(placeholder([64, 262144]), 0))["kernels"]) == 1


def test_nested_reduction_feeds_elementwise_kernel():
    x = placeholder([1, 513])
    plan = porch.plan(porch.sum(x, 1) * 2.0 + 1.0)
    assert [k["kind"] for k in plan["kernels"]] == ["row", "pointwise.scalar"]


def test_matmul_operand_expressions_are_materialised():
    a = placeholder([2, 3])
    b = placeholder([3, 2])
    plan = porch.plan(porch.matmul(a + a, b))
    kinds = [k["kind"] for k in plan["kernels"]]
    assert kinds[-1].startswith("gemm") and len(kinds) == 2


def test_matmul_read_through_a_view_is_not_fused_as_epilogue():
    a = placeholder([4, 4])
    m = porch.matmul(a, a)
    plan = porch.plan(m + porch.transpose(m))
    kinds = [k["kind"] for k in plan["kernels"]]
    assert kinds[0].startswith("gemm") and kinds[-1].startswith("pointwise")
    assert len(plan["temps"]) == 1


def test_product_read_by_reductions_is_computed_once():
    # softmax over a product: one gemm into a temporary, one row program
    # (not a second gemm recomputing the product in an epilogue)
    m = porch.matmul(placeholder([256, 64]), placeholder([64, 256]))
    plan = porch.plan(porch.softmax(m * 0.125, 1))
    assert [k["kind"] for k in plan["kernels"]] == ["gemm.mfma", "row"]
    # a column reduction of the product beside it: also one gemm
    plan = porch.plan(m - porch.broadcast_to(porch.sum(m, 0, True), [256, 256]))
    assert [k["kind"] for k in plan["kernels"]].count("gemm.mfma") == 1


def test_transposed_operand_feeds_gemm_without_copy():
    a = placeholder([64, 32])
    b = placeholder([64, 48])
    plan = porch.plan(porch.matmul(porch.transpose(a), b))
    assert len(plan["kernels"]) == 1 and plan["kernels"][0]["kind"].startswith("gemm")


@pytest.mark.parametrize("expr_fn", [
    lambda x: porch.transpose(x) + 1.0,
    lambda x: porch.concat(x, x, 1) * 2.0,
    lambda x: porch.reshape(porch.transpose(x), [6, 4]) - 1.0,
    lambda x: porch.broadcast_to(porch.sum(x, 1, True), [4, 6]) / x,
    lambda x: porch.max(porch.exp(x), 0, True),
    lambda x: porch.relu(porch.matmul(x, porch.transpose(x))) - 0.5,
])
def test_small_graphs_compile_offline(expr_fn):
    x = placeholder([4, 6])
    plan = porch.plan(expr_fn(x), compile=True)
    assert all(k["code_bytes"] > 0 for k in plan["kernels"])


def test_large_tensors_use_64_bit_indices():
    x = placeholder([1 << 16, 1 << 15])  # 2^31 elements
    assert "typedef long long idx_t" in porch.kernel_source(x + 1.0)
    y = placeholder([1024, 1024])
    assert "typedef int idx_t" in porch.kernel_source(y + 1.0)


def test_scalars_are_emitted_exactly():
    x = placeholder([8])
    for value in (0.1, 1e-45, 3.4028234663852886e38, -0.0):
        source = porch.kernel_source(x * value)
        assert "f" in source
    inf_source = porch.kernel_source(x * float("inf"))
    assert "__uint_as_float(0x7f800000u)" in inf_source


def test_long_softmax_rows_read_twice():
    # rows within the register cache: one read of x; beyond it, max and sum
    # share one pass, so two reads (not three), with ordinary loads (a
    # softmax over a product of two leaves: not the split form)
    def reads(expr):
        source = porch.kernel_source(expr)
        return source.count("a0 + ("), "__builtin_nontemporal_load" in source, "acc_a" in source

    assert reads(porch.softmax(placeholder([4, 32768]), 1)) == (1, True, False)
    assert reads(porch.softmax(placeholder([4, 262144]) * placeholder([4, 262144]), 1)) == (2, False, True)
    # the second read walks the row backwards
    x, y = placeholder([4, 262144]), placeholder([4, 262144])
    source = porch.kernel_source(porch.softmax(x * y, 1))
    assert source.count("for (int j = 63; j >= 0; --j)") == 1
    # a plain sum of exp over such rows stays one streaming pass
    source = porch.kernel_source(porch.sum(porch.exp(placeholder([4, 262144])), 1))
    assert source.count("a0 + (") == 1 and "acc_a" not in source


def test_lane_reductions_use_dpp_within_rows_and_bpermute_across():
    # a 32-column row takes an 8-lane segment: three DPP steps, no bpermute
    short = porch.kernel_source(porch.sum(placeholder([1000, 32]), 1))
    assert [c for c in ("0xB1", "0x4E", "0x141", "0x140") if c in short] == ["0xB1", "0x4E", "0x141"]
    assert "__shfl_xor" not in short
    # a full wave: four DPP steps, then distances 16 and 32 across rows
    full = porch.kernel_source(porch.sum(placeholder([1000, 2048]), 1))
    assert all(c in full for c in ("0xB1", "0x4E", "0x141", "0x140"))
    assert "__shfl_xor(acc_out, 16, 64)" in full and "__shfl_xor(acc_out, 32, 64)" in full
