"""Runs a graph's generated kernels on the CPU with guarded buffers —
TEST INFRASTRUCTURE ONLY (see prelude.hpp).

emulate(expr) compiles each kernel of the graph's plan as host C++ with
clang, runs it over its whole grid twice (buffers against their upper
guard, then against their lower one), and reports, per kernel, whether
every access stayed inside the buffers it was given, sized exactly as on
the device (inputs, temporaries and the destination).
"""

from __future__ import annotations

import hashlib
import os
import re
import subprocess

import numpy as np

import porch_amd as porch

HERE = os.path.dirname(os.path.abspath(__file__))
CLANG = os.environ.get("PORCH_EMU_CXX", "/opt/rocm/llvm/bin/clang++")
BUILD = os.path.join(HERE, "_build")


def available() -> bool:
    return os.path.exists(CLANG)


def _input_floats(t) -> int:
    if t.is_contiguous():
        return int(np.prod(t.shape(), dtype=np.int64)) if len(t.shape()) else 1
    return t.layout().span()


def _program(source: str, name: str, sizes: list[int], grid, block: int, only=None) -> str:
    args = ", ".join(f"b{i}" for i in range(len(sizes)))
    subset = ", {" + ", ".join(str(int(x)) for x in only) + "}" if only else ""
    decls = "".join(f"    float* b{i} = emu::guarded({n}, tail);\n"
                    f"    emu::load(b{i}, {n}, dir, {i});\n" for i, n in enumerate(sizes))
    return (
        '#include "prelude.hpp"\n#include "runner.hpp"\n' + source +
        "\nint main(int argc, char** argv) {\n"
        "    const bool tail = argc > 1 && argv[1][0] == '1';\n"
        "    const char* dir = argc > 2 ? argv[2] : nullptr;\n" + decls +
        f"    emu::run({{{grid[0]}, {grid[1]}, {grid[2]}}}, {block}, [&] {{ {name}({args}); }}{subset});\n"
        f"    emu::save(b{len(sizes) - 1}, {sizes[-1]}, dir);\n"
        '    std::puts("ok");\n    return 0;\n}\n'
    )


def run_kernel(source: str, name: str, sizes: list[int], grid, block: int = 256,
               timeout: float = 120.0, only=None, values=None) -> tuple[bool, str]:
    """Builds and runs one kernel over `grid` (or only the block x indices
    in `only`) with guarded buffers of `sizes` floats (its parameters in
    order); (stayed in bounds, detail).  `values`: a directory holding
    b<i>.bin contents for the buffers; the destination is written to
    out.bin there."""
    os.makedirs(BUILD, exist_ok=True)
    program = _program(source, name, sizes, grid, block, only)
    key = hashlib.sha1(program.encode()).hexdigest()[:16]
    cpp = os.path.join(BUILD, f"k_{key}.cpp")
    exe = os.path.join(BUILD, f"k_{key}")
    if not os.path.exists(exe):
        with open(cpp, "w") as f:
            f.write(program)
        built = subprocess.run([CLANG, "-std=c++20", "-O1", "-pthread", "-w", "-I", HERE, cpp, "-o", exe + ".tmp"],
                               capture_output=True, text=True, timeout=300)
        if built.returncode != 0:
            return False, "build: " + built.stderr[-2000:]
        os.replace(exe + ".tmp", exe)
    for placement in ("1", "0"):
        try:
            ran = subprocess.run([exe, placement] + ([values] if values else []),
                                 capture_output=True, text=True, timeout=timeout)
        except subprocess.TimeoutExpired:
            return False, f"timed out (placement {placement})"
        if ran.returncode != 0 or "ok" not in ran.stdout:
            return False, f"placement {placement}: exit {ran.returncode} {ran.stderr[-500:]}"
    return True, ""


# The test of a max reduction's result that sends it down the path in the
# reference's order (a NaN, or a +0 maximum); force_exact replaces it.
_ORDER_TEST = "return m != m || __builtin_bit_cast(unsigned, m) == 0u;"


# Blocks run one after another here, so a wait on a later block's partial
# never ends: a few hundred polls (each yielding, time for the other waves
# of the block to publish theirs), then the waiting wave's own fallback.
_SPIN = re.compile(r"#define porch_spin_limit \d+")


def _emulated(source: str) -> str:
    return _SPIN.sub("#define porch_spin_limit 200", source)


def emulate(expr, timeout: float = 120.0, only=None, force_exact: bool = False) -> list[dict]:
    """Per kernel of the plan: {"kind", "ok", "detail"}.  `only`: run just
    these block x indices of each kernel (for persistent grids whose
    workgroups each walk many tiles).  `force_exact`: every max reduction
    also takes its path in the reference's order, whatever the values."""
    expr = porch.tensor_expr(expr)
    plan = porch.plan(expr)
    _, _, _, inputs, _ = porch.serialize(expr._root)
    input_floats = [max(_input_floats(t), 1) for t in inputs]
    temps = [max(int(n), 1) for n in plan["temps"]]
    out_floats = max(int(np.prod(plan["out_shape"], dtype=np.int64)) if plan["out_shape"] else 1, 1)
    results = []
    for i, k in enumerate(plan["kernels"]):
        slots = input_floats + temps
        dest = out_floats if k["dest"] == "output" else temps[int(k["dest"][4:])]
        source = _emulated(porch.kernel_source(expr, i))
        if force_exact:
            assert _ORDER_TEST in source
            source = source.replace(_ORDER_TEST, "return true;")
        ok, detail = run_kernel(source, k["name"], slots[: k["slots"]] + [dest],
                                k["grid"], k["block"], timeout, only)
        results.append({"kind": k["kind"], "ok": ok, "detail": detail})
    return results


# The bits of an output no workgroup wrote (a NaN with a payload that no
# kernel computes from finite inputs) when a subset of workgroups runs.
UNWRITTEN = np.uint32(0x7FC0DEAD)


def edge_blocks(grid_x: int) -> list[int]:
    """The first two and the last two workgroups of a grid of `grid_x`: with
    the kernels' block-to-tile maps they own the first outputs and the
    ragged last ones (the last band, run, row group or column tile)."""
    return sorted({0, 1, grid_x - 2, grid_x - 1} & set(range(grid_x)))


def written(out: np.ndarray) -> np.ndarray:
    """Where `evaluate(..., only=...)` wrote the output."""
    return np.ascontiguousarray(out, np.float32).view(np.uint32) != UNWRITTEN


def evaluate(expr, inputs: list[np.ndarray], force_exact: bool = False, timeout: float = 120.0,
             only=None) -> np.ndarray:
    """The graph's result computed by its generated kernels run on the CPU
    (in plan order, temporaries carried between them), for input values
    `inputs` (the serialised input order).  Arithmetic follows the host's
    libm where the kernels call device math, so only exact operations
    (views, + - * /, max, reductions of integers) compare bit for bit.
    `only`: run just these block x indices of a single-kernel plan; the
    outputs of the other blocks keep the bits UNWRITTEN (see written())."""
    import tempfile

    expr = porch.tensor_expr(expr)
    plan = porch.plan(expr)
    _, _, _, tensors, _ = porch.serialize(expr._root)
    input_floats = [max(_input_floats(t), 1) for t in tensors]
    buffers = [np.ascontiguousarray(np.asarray(v, np.float32).reshape(-1)) for v in inputs]
    assert [b.size for b in buffers] == input_floats, ([b.size for b in buffers], input_floats)
    temps = [np.zeros(max(int(n), 1), np.float32) for n in plan["temps"]]
    out = np.zeros(max(int(np.prod(plan["out_shape"], dtype=np.int64)) if plan["out_shape"] else 1, 1),
                   np.float32)
    if only is not None:
        assert len(plan["kernels"]) == 1, "a subset of workgroups needs a single-kernel plan"
        out.view(np.uint32)[:] = UNWRITTEN
    with tempfile.TemporaryDirectory() as work:
        for i, k in enumerate(plan["kernels"]):
            slots = (buffers + temps)[: k["slots"]]
            dest = out if k["dest"] == "output" else temps[int(k["dest"][4:])]
            for j, b in enumerate(slots + [dest]):
                b.tofile(os.path.join(work, f"b{j}.bin"))
            source = _emulated(porch.kernel_source(expr, i))
            if force_exact:
                source = source.replace(_ORDER_TEST, "return true;")
            ok, detail = run_kernel(source, k["name"], [b.size for b in slots] + [dest.size],
                                    k["grid"], k["block"], timeout, only, values=work)
            assert ok, detail
            dest[:] = np.fromfile(os.path.join(work, "out.bin"), np.float32)
    return out.reshape(plan["out_shape"])


def check_edges(expr, inputs: list[np.ndarray], want: np.ndarray, timeout: float = 600.0) -> int:
    """Runs the first two and last two workgroups of a single-kernel plan:
    their accesses must stay inside the buffers (both placements), they
    must write the first and the last output, and every output they write
    must equal `want` bit for bit.  Returns the number of outputs checked."""
    plan = porch.plan(porch.tensor_expr(expr))
    assert len(plan["kernels"]) == 1, plan["kernels"]
    edges = edge_blocks(int(plan["kernels"][0]["grid"][0]))
    results = emulate(expr, timeout=timeout, only=edges)
    assert all(r["ok"] for r in results), results
    got = evaluate(expr, inputs, timeout=timeout, only=edges).reshape(want.shape)
    mask = written(got)
    assert mask.reshape(-1)[0] and mask.reshape(-1)[-1], "the edge workgroups missed the first or last output"
    assert np.array_equal(got[mask].view(np.uint32), np.ascontiguousarray(want, np.float32)[mask].view(np.uint32))
    return int(mask.sum())
