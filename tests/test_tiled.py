"""The LDS-transpose kernel class (pointwise.tiled) over ragged and aligned
shapes: concat boundaries inside and on tile edges, strided and offset
transposed leaves, and batched (rank-3) tiles.

The CPU tests plan and compile each case offline and pin which variant the
emitter chose (vector width along the transposed leaf, per-tile select
decisions, 128-bit stores); the GPU test checks every case bit-exact against
the oracle.
"""

import numpy as np
import pytest

import porch_amd as porch
from oracle import host
from tests.helpers import placeholder


def sl(start, stop, step=1):
    return porch.slice(start, stop, step)


def interleaved_concat(make, rows, cols):
    """concat(transpose(x[0::2, 1::2]), transpose(x[1::2, 0::2]), 0) + 1 on
    x [rows, cols]: the headline view pattern at other sizes."""
    x = make([rows, cols])
    return porch.concat(porch.transpose(x[sl(0, rows, 2), sl(1, cols, 2)]),
                        porch.transpose(x[sl(1, rows, 2), sl(0, cols, 2)]), 0) + 1.0


def transpose_plus(make, rows, cols):
    """transpose(x) + y: a unit-stride transposed leaf next to a contiguous one."""
    x = make([rows, cols])
    y = make([cols, rows])
    return porch.transpose(x) + y * 2.0


def offset_transpose(make, rows, cols):
    """transpose of x[1:, 2:cols-2] (leaf offset 2 + row stride cols)."""
    x = make([rows, cols])
    return porch.transpose(x[sl(1, rows), sl(2, cols - 2)]) - 0.5


def odd_stride_transpose(make, rows, cols):
    """transpose of a stride-3 column slice: no vector form exists."""
    x = make([rows, cols])
    return porch.transpose(x[sl(0, rows), sl(0, cols, 3)]) * 3.0


def batched_transpose(make, batch, rows, cols):
    """A transposed leaf broadcast over a batch plus a batched contiguous leaf."""
    x = make([rows, cols])
    z = make([batch, cols, rows])
    t = porch.unsqueeze(porch.transpose(x), 0)
    return porch.broadcast_to(t, [batch, cols, rows]) + z


def concat_inside_transpose(make, rows, cols):
    """A select along the output's contiguous axis whose both branches are
    transposed leaves: decided once per tile."""
    x = make([rows, cols])
    y = make([rows + 4, cols])
    a = porch.concat(porch.transpose(x), porch.transpose(y), 1)
    return a + porch.transpose(porch.concat(x, y, 0))


def select_in_store_phase(make, rows, cols, split):
    """transpose(x) plus a concat of contiguous leaves split at `split` along
    the output's contiguous axis (the select lives in the store phase)."""
    x = make([rows, cols])
    u = make([cols, split])
    v = make([cols, rows - split])
    return porch.transpose(x) + porch.concat(u, v, 1)


def transposed_concat_branch(make, rows, cols):
    """concat(x1, transpose(x2), 1): the transposed leaf is staged in phase 1
    but sits in the select's second branch, so it is loaded only where that
    branch is taken (elsewhere its index runs before the start of x2)."""
    x1 = make([rows, cols])
    x2 = make([cols, rows])
    return porch.concat(x1, porch.transpose(x2), 1) + 1.0


# (builder, sizes, phase-1 vector type or None, hoisted select count, float4 stores)
CASES = {
    "interleave_512x256": (interleaved_concat, (512, 256), "float4", 1, True),
    "interleave_384x192": (interleaved_concat, (384, 192), "float4", 1, True),
    "interleave_520x390": (interleaved_concat, (520, 390), None, 1, True),
    "interleave_130x66": (interleaved_concat, (130, 66), None, 1, False),
    "transpose_200x136": (transpose_plus, (200, 136), "float4", 0, True),
    "transpose_70x33": (transpose_plus, (70, 33), None, 0, False),
    # 33 x 47 = 1551 tiles of 128 x 64, ragged on both axes: persistent workgroups
    "transpose_3000x4100": (transpose_plus, (3000, 4100), "float4", 0, True),
    "offset_201x140": (offset_transpose, (201, 140), "float2", 0, True),
    "odd_stride_96x300": (odd_stride_transpose, (96, 300), None, 0, True),
    "batched_3x72x132": (batched_transpose, (3, 72, 132), "float4", 0, True),
    "concat_inside_100x68": (concat_inside_transpose, (100, 68), "float4", 1, True),
    "store_select_132x64_68": (select_in_store_phase, (132, 64, 68), "float4", 0, True),
    "store_select_132x64_70": (select_in_store_phase, (132, 64, 70), "float4", 0, False),
    "concat_branch_300x4": (transposed_concat_branch, (300, 4), "float4", 0, True),
    "concat_branch_130x6": (transposed_concat_branch, (130, 6), "float2", 0, False),
}


def build_case(name, make):
    fn, sizes, *_ = CASES[name]
    return fn(make, *sizes)


@pytest.mark.parametrize("name", sorted(CASES))
def test_tiled_variant_choice(name):
    _, _, vector, n_hoisted, stores4 = CASES[name]
    expr = build_case(name, placeholder)
    plan = porch.plan(expr, compile=True)
    kinds = [k["kind"] for k in plan["kernels"]]
    assert kinds == ["pointwise.tiled"], plan
    assert plan["kernels"][0]["code_bytes"] > 0
    source = porch.kernel_source(expr, 0)
    phase1 = source.split("__syncthreads();")[0]
    vector_forms = {"float4": ("reinterpret_cast<const float4*>", "reinterpret_cast<const porch_v4f*>"),
                    "float2": ("reinterpret_cast<const float2*>",)}
    if vector is None:
        assert "reinterpret_cast<const float" not in phase1
        assert "reinterpret_cast<const porch_v4f" not in phase1
    else:
        assert any(form in phase1 for form in vector_forms[vector])
    assert source.count("const int mode") == n_hoisted
    assert ("reinterpret_cast<float4*>(out" in source) == stores4


def test_many_tiles_use_persistent_workgroups():
    many = porch.plan(build_case("transpose_3000x4100", placeholder), compile=True)["kernels"][0]
    few = porch.plan(build_case("transpose_200x136", placeholder), compile=True)["kernels"][0]
    # at most four workgroups per compute unit walk the 1551 tiles
    assert many["grid"][0] == 4 * 256
    assert "for (idx_t tile_id = blockIdx.x; tile_id < 1551;" in porch.kernel_source(
        build_case("transpose_3000x4100", placeholder), 0)
    assert few["grid"][0] == 2 * 4  # 136 x 200 outputs: 2 x 4 tiles of 128 x 64


@pytest.mark.gpu
def test_tiled_cases_bit_exact(gpu):
    rng = np.random.default_rng(77)

    def make(shape):
        values = rng.integers(-1000, 1000, size=int(np.prod(shape))).astype(np.float32) / np.float32(8)
        return gpu.tensor(list(shape), values)

    for name in sorted(CASES):
        print("tiled case", name, flush=True)
        expr = build_case(name, make)
        assert gpu.plan(expr)["kernels"][0]["kind"] == "pointwise.tiled"
        out = gpu.materialize(expr).cpu().reshape(expr.shape())
        ref = host.evaluate(expr)
        assert out.shape == ref.shape, name
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), name
