"""The reference's own test program, compiled unchanged from its
tests/tensor_test.cpp against include/porch/*.hpp and libporch_amd.so
(recipe: oracle/Makefile `ref`).  Its own assertions decide each case."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "oracle", "_ref", "porch_tensor_test")

NO_GPU_CASES = [
    "tensor_is_small_handle",
    "rejects_invalid_shapes",
    "cuda_devices_select_cuda_jit_backend",
    "cuda_jit_availability_matches_backend_availability",
    "cuda_jit_compiles_or_reports_missing_nvrtc",
]

GPU_CASES = [
    "construction_tracks_shape_and_device", "construction_builds_contiguous_layout",
    "bracket_slice_selects_contiguous_copy", "bracket_slice_returns_lazy_expression",
    "bracket_slice_handles_multiple_dimensions", "zeros_fills_gpu_tensor",
    "add_uses_cuda_backend", "subtract_uses_cuda_backend", "multiply_uses_cuda_backend",
    "elementwise_arithmetic_matches_expected_values", "chained_arithmetic_matches_expected_values",
    "fused_expression_materializes_once", "multiline_expression_stays_lazy_with_auto",
    "tensor_assignment_keeps_graph_lazy", "explicit_gpu_sync_and_cpu_copy",
    "concurrent_same_lazy_tensor_materializes_once_safely",
    "concurrent_independent_lazy_tensors_use_thread_streams",
    "scalar_elementwise_ops_use_cuda_backend", "scalar_arithmetic_order_matches_expected_values",
    "matmul_uses_cuda_backend", "matmul_rectangular_values_are_correct",
    "matmul_returns_lazy_expression", "matmul_composes_with_elementwise_ir",
    "matmul_accepts_expression_operands", "matmul_rejects_invalid_shapes",
    "reshape_uses_lazy_device_ir", "transpose_uses_lazy_device_ir",
    "broadcast_to_uses_lazy_device_ir", "concat_uses_lazy_device_ir",
    "reductions_use_lazy_device_ir", "keepdim_reductions_use_lazy_device_ir",
    "block_reductions_handle_axis_larger_than_block",
    "nested_reductions_materialize_with_block_reduction",
    "softmax_style_expression_uses_nested_block_reduction", "relu_compound_op_uses_primitives",
    "softmax_compound_op_uses_primitives", "logistic_compound_op_uses_primitives",
    "exp_uses_lazy_device_ir", "divide_and_reciprocal_use_lazy_device_ir",
    "elementwise_minimum_maximum_use_lazy_device_ir",
    "unsqueeze_and_expression_shape_are_lazy_metadata", "device_buffer_round_trips_values",
]

needs_binary = pytest.mark.skipif(
    not os.path.exists(BINARY),
    reason="oracle/_ref/porch_tensor_test is built only where the reference tree is present")


@needs_binary
@pytest.mark.parametrize("case", NO_GPU_CASES)
def test_reference_case_without_gpu(case):
    result = subprocess.run([BINARY, case], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stderr


@needs_binary
def test_reference_case_list_is_complete():
    assert len(NO_GPU_CASES) + len(GPU_CASES) == 47


@pytest.mark.gpu
def test_reference_suite_on_gpu(gpu):
    """All 47 cases in one process (the binary's no-argument mode); on a
    failure, each case runs alone to name it.  On a GPU run the binary must
    be there (built where the reference tree is, and carried with the tree):
    its absence fails the test rather than skipping it."""
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is missing: build it with `make -C oracle ref` before a GPU run")
    result = subprocess.run([BINARY], capture_output=True, text=True, timeout=300)
    if result.returncode == 0:
        assert "skipped" not in result.stdout
        return
    failed = []
    for case in NO_GPU_CASES + GPU_CASES:
        r = subprocess.run([BINARY, case], capture_output=True, text=True, timeout=120)
        if r.returncode != 0 or "skipped" in r.stdout:
            failed.append((case, r.returncode, r.stderr[-300:]))
    assert not failed, failed
