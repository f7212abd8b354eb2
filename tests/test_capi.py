"""The C-ABI library loads, exports every entry point include/porch_amd.h
declares, and validates graphs with the reference's exception types and
messages — all without a GPU."""

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import porch_amd as porch
from porch_amd import _lib
from tests.helpers import placeholder

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    with open(os.path.join(ROOT, "include", "porch_amd.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(porch_[a-z_0-9]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    """By libporch_amd.so, or (the allocation-free entry point) by its
    companion libporch_amd_noalloc.so."""
    names = declared_functions()
    assert len(names) >= 32
    lib = ctypes.CDLL(_lib.LIBRARY_PATH)
    companion = ctypes.CDLL(_lib.NOALLOC_LIBRARY_PATH)
    missing = [n for n in names if not hasattr(lib, n) and not hasattr(companion, n)]
    assert not missing, missing
    assert hasattr(companion, "porch_materialize_noalloc") and not hasattr(lib, "porch_materialize_noalloc")


def test_every_declared_symbol_has_a_python_binding():
    assert set(declared_functions()) <= set(_lib._SIGNATURES) | set(_lib._NOALLOC_SIGNATURES)


def test_library_links_no_rocm_library():
    out = subprocess.run(["ldd", _lib.LIBRARY_PATH], capture_output=True, text=True).stdout
    assert "amdhip" not in out and "hiprtc" not in out


def test_noalloc_companion_links_the_hip_runtime_and_the_library():
    out = subprocess.run(["ldd", _lib.NOALLOC_LIBRARY_PATH], capture_output=True, text=True).stdout
    assert "libamdhip64" in out and "libporch_amd.so" in out and "not found" not in out


def test_unavailable_when_hip_runtime_is_missing(tmp_path):
    code = ("import porch_amd as p, sys; "
            "sys.exit(0 if p.is_available() is False and "
            "p.is_backend_available(p.backend()) is False else 1)")
    env = dict(os.environ, PORCH_HIP_LIBRARY=str(tmp_path / "missing.so"))
    rc = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env).returncode
    assert rc == 0


def test_construction_without_runtime_raises_runtime_error(tmp_path):
    code = ("import porch_amd as p\n"
            "try:\n    p.tensor([2], [1.0, 2.0])\nexcept p.PorchError as e:\n"
            "    assert 'libamdhip64' in str(e), e\n    raise SystemExit(0)\nraise SystemExit(1)\n")
    env = dict(os.environ, PORCH_HIP_LIBRARY=str(tmp_path / "missing.so"))
    assert subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env).returncode == 0


def test_backend_selection_matches_reference_spelling():
    chosen = porch.backend_for(porch.device())
    assert chosen.is_cuda_jit()
    assert porch.backend_name(chosen) == "cuda-jit"
    assert porch.is_available() == porch.is_backend_available(porch.backend(porch.backend_kind.cuda_jit))


def test_rejects_invalid_shapes_before_any_device_call():
    with pytest.raises(porch.InvalidArgument, match="tensor data size does not match shape"):
        porch.tensor([2, 2], [1.0, 2.0, 3.0])


def test_empty_tensor_needs_no_device():
    t = porch.tensor([0, 3], [])
    assert t.numel() == 0 and t.device_data().empty_buffer()


@pytest.mark.parametrize("build, message", [
    (lambda a, b: porch.matmul(a, b), "matmul inner dimensions must match"),
    (lambda a, b: a + b, "tensor expression shapes must match"),
    (lambda a, b: porch.transpose(porch.reshape(a, [6])), "transpose currently requires a rank-2 tensor"),
    (lambda a, b: porch.reshape(a, [4]), "reshape must preserve tensor element count"),
    (lambda a, b: porch.sum(a, 2), "reduction axis is out of bounds"),
    (lambda a, b: porch.concat(a, b, 0), "concat non-axis dimensions must match"),
    (lambda a, b: porch.concat(a, porch.reshape(b, [4]), 0), "concat operands must have the same rank"),
    (lambda a, b: porch.broadcast_to(a, [3, 3]), "broadcast shapes are not compatible"),
    (lambda a, b: porch.broadcast_to(a, [6]), "broadcast target rank must be at least source rank"),
    (lambda a, b: porch.unsqueeze(a, 3), "unsqueeze axis is out of bounds"),
    (lambda a, b: porch.matmul(porch.reshape(a, [6]), b), "matmul requires rank-2 tensors"),
    (lambda a, b: porch.matmul(porch.tensor_expr(1.0), b), "matmul operands must be tensors"),
    (lambda a, b: porch.sum(porch.tensor_expr(1.0) + 2.0, 0), "reduction operand must be a tensor"),
])
def test_shape_errors_use_reference_messages(build, message):
    a = placeholder([2, 3])
    b = placeholder([2, 2])
    with pytest.raises(porch.InvalidArgument, match=message):
        build(a, b).shape()


def test_expression_shape_metadata_is_lazy():
    values = placeholder([2, 3])
    expr = porch.unsqueeze(values + 1.0, 1)
    assert expr.shape() == [2, 1, 3] and expr.rank() == 3 and expr.numel() == 6
    assert (porch.tensor_expr(2.0) * 3.0).shape() == []


def test_slice_subscripts_follow_reference_rules():
    x = placeholder([3, 4])
    assert x[1, porch.slice(1, 4, 2)].shape() == [2]
    assert x[porch.slice(-2, 100)].shape() == [2, 4]
    assert x[porch.slice(3, 1)].shape() == [0, 4]
    with pytest.raises(porch.OutOfRange, match="tensor index is out of bounds"):
        x[3]
    with pytest.raises(porch.InvalidArgument, match="tensor slice step must be positive"):
        x[porch.slice(0, 3, 0)]
    with pytest.raises(porch.InvalidArgument, match="too many tensor indices"):
        x[0, 0, 0]


def test_malformed_node_tables_are_rejected():
    nodes = (_lib.Node * 1)()
    nodes[0].op = 99
    dims = (ctypes.c_int64 * 1)()
    g = _lib.Graph(ctypes.cast(nodes, ctypes.POINTER(_lib.Node)), 1,
                   ctypes.cast(dims, ctypes.POINTER(ctypes.c_int64)), 0)
    rc = _lib.lib.porch_infer_shape(ctypes.byref(g), None, 0, None, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT
    # an operand that points forward
    nodes[0].op = _lib.OP["exp"]
    nodes[0].lhs = 3
    assert _lib.lib.porch_infer_shape(ctypes.byref(g), None, 0, None, None) == _lib.ERR_INVALID_ARGUMENT


def test_slices_outside_their_source_are_rejected():
    """A node table can describe any strides; reads beyond the source must
    be refused before any kernel is generated."""
    nodes = (_lib.Node * 2)()
    nodes[0].op = _lib.OP["input"]
    nodes[0].input = 0
    nodes[0].rank = 1
    nodes[0].dims = 0
    nodes[1].op = _lib.OP["slice"]
    nodes[1].lhs = 0
    nodes[1].rank = 1
    nodes[1].dims = 1
    nodes[1].offset = 2
    dims = (ctypes.c_int64 * 3)(4, 3, 1)  # input [4]; slice shape [3] stride 1 from 2
    g = _lib.Graph(ctypes.cast(nodes, ctypes.POINTER(_lib.Node)), 2,
                   ctypes.cast(dims, ctypes.POINTER(ctypes.c_int64)), 3)
    assert _lib.lib.porch_infer_shape(ctypes.byref(g), None, 0, None, None) == _lib.ERR_OUT_OF_RANGE


def test_compile_error_reports_hiprtc_log():
    code = ctypes.c_void_p()
    rc = _lib.lib.porch_compile(b"extern \"C\" __global__ void k() { this is not C++; }",
                                None, 0, ctypes.byref(code))
    assert rc == _lib.ERR_COMPILATION
    assert "error" in _lib.lib.porch_last_error().decode()


def test_compile_produces_gfx950_code_object():
    code = ctypes.c_void_p()
    src = b"extern \"C\" __global__ void add_kernel(const float* a, const float* b, float* o)" \
          b" { o[threadIdx.x] = a[threadIdx.x] + b[threadIdx.x]; }"
    _lib.check(_lib.lib.porch_compile(src, None, 0, ctypes.byref(code)))
    size = _lib.lib.porch_code_object_size(code)
    data = ctypes.string_at(_lib.lib.porch_code_object_data(code), size)
    _lib.lib.porch_code_object_release(code)
    assert data[:4] == b"\x7fELF" and b"add_kernel" in data and b"gfx950" in data


def test_synthetic_generator_matches_published_splitmix64():
    mask = (1 << 64) - 1

    def splitmix64(seed, count):
        state = seed
        for _ in range(count):
            state = (state + 0x9E3779B97F4A7C15) & mask
            z = state
            z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
            z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
            yield z ^ (z >> 31)

    from porch_amd import synth

    raw = list(splitmix64(101, 1000))
    u = np.array([(x >> 40) * 2.0 ** -24 for x in raw])
    assert np.array_equal(synth.uniform(1000, 101, -1.0, 1.0), (-1.0 + 2.0 * u).astype(np.float32))
    import math
    raw = list(splitmix64(201, 10))
    normal = synth.normal(10, 201, 0.0, 1.0)
    for j in range(5):
        u1 = ((raw[2 * j] >> 40) + 1) * 2.0 ** -24
        u2 = (raw[2 * j + 1] >> 40) * 2.0 ** -24
        r = math.sqrt(-2.0 * math.log(u1))
        assert normal[2 * j] == np.float32(r * math.cos(2 * math.pi * u2))
        assert normal[2 * j + 1] == np.float32(r * math.sin(2 * math.pi * u2))
    x = np.zeros(100000, dtype=np.float32)
    synth.replace(x, 302, 0.01, 20.0)
    assert 800 < (x == 20.0).sum() < 1200
