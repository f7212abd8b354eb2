"""The five benchmark graphs at their full sizes built through porch's public
C++ API (tests/cpp/configs_test.cpp: porch::tensor, porch::ops and the
tensor_expr operators, the front end that include/porch/tensor.hpp
declares), against the oracle on the same seeded inputs:

* elementwise and view chain: bit for bit;
* softmax: 1e-6 relative per element;
* logistic row sum: 1e-5 relative;
* matmul with its epilogue: every output against a float64 GEMM (the
  product within its accumulation bound, the result within 1e-4 relative),
  and 1e-4 relative to the oracle on a sample of rows (the oracle's
  sequential fp32 product of a 4096^3 graph takes minutes on the host).

Each result also equals, bit for bit, the same graph materialised through
the Python mirror and the C ABI: the C++ front end records the same graph,
which plans to the same kernels.
"""

import os
import subprocess

import numpy as np
import pytest

from oracle import host
from tests.helpers import CONFIG_SIZES, check_matmul_epilogue_every_output, config_graph, config_inputs, config_shapes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "cpp", "_build", "configs_test")
CONFIGS = ["elementwise", "view_chain", "softmax", "logistic_rowsum", "matmul_epilogue"]


def built():
    assert os.path.exists(BINARY), "build first: make -C tests/cpp (or __graft_entry__.build())"
    return BINARY


def test_program_lists_the_five_graphs():
    listed = subprocess.run([built()], capture_output=True, text=True, timeout=60).stdout.split()
    assert listed == CONFIGS


def test_program_rejects_an_unknown_graph(tmp_path):
    result = subprocess.run([built(), "bogus", str(tmp_path / "out.bin")], capture_output=True, text=True,
                            timeout=60)
    assert result.returncode == 1 and "unknown config: bogus" in result.stderr


def run_cpp(name, path):
    result = subprocess.run([built(), name, str(path)], capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stderr
    print(result.stdout.strip(), flush=True)
    return np.fromfile(path, dtype=np.float32)


def bits_equal(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", CONFIGS)
def test_full_size_graph_through_the_cpp_api(gpu, name, tmp_path):
    porch = gpu
    out = run_cpp(name, tmp_path / f"{name}.bin")
    inputs = config_inputs(name)
    tensors = [porch.tensor(s, v) for s, v in zip(config_shapes(name), inputs)]
    expr = config_graph(name, tensors)
    shape = expr.shape()
    assert out.size == int(np.prod(shape))
    out = out.reshape(shape)

    # the same graph through the Python mirror: the same kernels, the same bits
    assert bits_equal(out, porch.materialize(expr).cpu().reshape(shape))

    if name == "matmul_epilogue":
        s = CONFIG_SIZES[name]
        m, k, n = s["m"], s["k"], s["n"]
        a, b, bias = inputs
        delta, frac = check_matmul_epilogue_every_output(out, a, b, bias, m, k, n)
        print(f"all {m * n} outputs: max |delta| = {delta:.3e}, max |delta| / bound = {frac:.3e}", flush=True)
        rows = np.array([0, 1, 1000, 2047, 2048, 3071, 4095])
        sample = porch.tensor([rows.size, k], a.reshape(m, k)[rows])
        ref = host.evaluate(porch.relu(porch.matmul(sample, tensors[1]) +
                                       porch.broadcast_to(tensors[2], [rows.size, n])) - 0.5)
        got = out[rows]
    else:
        ref = host.evaluate(expr).reshape(shape)
        got = out
    if name in ("elementwise", "view_chain"):
        assert bits_equal(got, ref)
        return
    bar = {"softmax": 1e-6, "logistic_rowsum": 1e-5, "matmul_epilogue": 1e-4}[name]
    err = np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)), 1e-30)
    assert err.max() <= bar, (name, err.max(), np.unravel_index(err.argmax(), err.shape))
