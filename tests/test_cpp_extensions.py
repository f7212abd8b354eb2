"""The C++ API of the IR extensions (permute, batched_matmul, tensors over
strided storage) through a test program built against include/porch/*.hpp
and libporch_amd.so (tests/cpp/extensions_test.cpp, recipe
tests/cpp/Makefile).  The program's own assertions decide: exact
values computed by plain loops in the program."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "cpp", "_build", "extensions_test")

NO_GPU_CASES = [
    "permute_shape_is_lazy_metadata",
    "permute_rejects_non_permutations",
    "batched_matmul_rejects_shapes",
    "strided_storage_must_cover_the_layout",
]
GPU_CASES = ["permute_values", "batched_matmul_values", "strided_tensor_reads_its_layout"]


def run(case):
    assert os.path.exists(BINARY), "build first: make -C tests/cpp (or __graft_entry__.build())"
    return subprocess.run([BINARY, case], capture_output=True, text=True, timeout=120)


def test_case_list_is_complete():
    assert os.path.exists(BINARY), "build first: make -C tests/cpp (or __graft_entry__.build())"
    listed = subprocess.run([BINARY], capture_output=True, text=True, timeout=60).stdout.split()
    assert sorted(listed) == sorted(NO_GPU_CASES + GPU_CASES)


@pytest.mark.parametrize("case", NO_GPU_CASES)
def test_case_without_gpu(case):
    result = run(case)
    assert result.returncode == 0, result.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("case", GPU_CASES)
def test_case_on_gpu(case):
    result = run(case)
    assert result.returncode == 0, result.stderr
