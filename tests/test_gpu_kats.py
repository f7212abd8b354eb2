"""The reference's known-answer tests on the GPU, through porch_amd (C ABI)."""

import threading

import numpy as np
import pytest

from tests.helpers import build, check_kat, kat_cases, kat_input_values

pytestmark = pytest.mark.gpu

CASES, ERRORS = kat_cases()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_kat_materialize(gpu, case):
    porch = gpu
    tensors = [porch.tensor(spec["shape"], kat_input_values(spec)) for spec in case["inputs"]]
    expr = build(case["expr"], tensors)
    result = porch.tensor(expr)  # lazy, as `const porch::tensor r = expr;`
    assert list(result.shape()) == case["shape"]
    check_kat(case, result.cpu())
    assert not result.device_data().empty_buffer()
    again = porch.materialize(expr)  # cache hit, same bits
    assert np.array_equal(again.cpu().view(np.uint32), result.cpu().view(np.uint32))


def test_matmul_rejects_invalid_shapes(gpu):
    porch = gpu
    (case,) = ERRORS
    tensors = [porch.tensor(spec["shape"], kat_input_values(spec)) for spec in case["inputs"]]
    with pytest.raises(porch.InvalidArgument):
        porch.tensor(build(case["expr"], tensors))


def test_construction_tracks_shape_and_device(gpu):
    porch = gpu
    values = porch.tensor([2, 3], [1, 2, 3, 4, 5, 6], porch.device(1))
    assert values.rank() == 2 and values.numel() == 6 and values.shape() == (2, 3)
    assert values.placement().is_cuda() and values.placement().ordinal() == 1


def test_construction_builds_contiguous_layout(gpu):
    porch = gpu
    values = porch.tensor([2, 3, 4], [1.0] * 24)
    assert values.is_contiguous() and values.storage_offset() == 0
    assert values.strides() == (12, 4, 1)


def test_zeros_fills_gpu_tensor(gpu):
    porch = gpu
    values = porch.zeros([2, 2])
    assert values.numel() == 4 and not values.device_data().empty_buffer()
    assert (values.data() == 0.0).all()


def test_explicit_gpu_sync_and_cpu_copy(gpu):
    porch = gpu
    lhs = porch.tensor([2, 2], [1, 2, 3, 4])
    rhs = porch.tensor([2, 2], [10, 20, 30, 40])
    result = porch.tensor(lhs + rhs)
    result.realize()
    assert not result.device_data().empty_buffer()
    result.synchronize()
    assert result.cpu().tolist() == [11, 22, 33, 44]


def test_tensor_assignment_keeps_graph_lazy(gpu):
    porch = gpu
    lhs = porch.tensor([2, 2], [1, 2, 3, 4])
    rhs = porch.tensor([2, 2], [10, 20, 30, 40])
    delayed = porch.tensor(lhs + rhs)
    assert delayed.shape() == (2, 2)
    result = porch.tensor(delayed * 2.0 - 1.0)
    assert result.cpu().tolist() == [21, 43, 65, 87]
    assert delayed.cpu().tolist() == [11, 22, 33, 44]


def test_concurrent_same_lazy_tensor_materializes_once_safely(gpu):
    porch = gpu
    lhs = porch.tensor([2, 2], [1, 2, 3, 4])
    rhs = porch.tensor([2, 2], [10, 20, 30, 40])
    result = porch.tensor((lhs + rhs) * 2.0 - 1.0)
    before = porch.jit_stats()["plan_hits"] + porch.jit_stats()["plan_misses"]
    outputs, errors = [None, None], []

    def read(i):
        try:
            outputs[i] = result.cpu()
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    threads = [threading.Thread(target=read, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert outputs[0].tolist() == outputs[1].tolist() == [21, 43, 65, 87]
    after = porch.jit_stats()["plan_hits"] + porch.jit_stats()["plan_misses"]
    assert after - before == 1  # materialised exactly once


def test_concurrent_independent_lazy_tensors_use_thread_streams(gpu):
    porch = gpu
    lhs = porch.tensor([2, 2], [1, 2, 3, 4])
    rhs = porch.tensor([2, 2], [10, 20, 30, 40])
    left = porch.tensor(lhs + rhs)
    right = porch.tensor(rhs - lhs)
    outputs, errors = {}, []

    def read(name, t):
        try:
            outputs[name] = t.cpu().tolist()
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    threads = [threading.Thread(target=read, args=("l", left)),
               threading.Thread(target=read, args=("r", right))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert outputs == {"l": [11, 22, 33, 44], "r": [9, 18, 27, 36]}


def test_result_produced_on_another_thread_is_ordered(gpu):
    """A buffer written on thread A's stream and read on thread B's."""
    porch = gpu
    x = porch.tensor([1 << 20], np.arange(1 << 20, dtype=np.float32))
    holder = {}

    def produce():
        holder["t"] = porch.materialize(x * 3.0)  # launched on this thread's stream

    t = threading.Thread(target=produce)
    t.start()
    t.join()
    out = porch.materialize(holder["t"] + 1.0).cpu()  # consumed on the main stream
    assert np.array_equal(out, np.arange(1 << 20, dtype=np.float32) * 3.0 + 1.0)


def test_device_buffer_round_trips_values(gpu):
    porch = gpu
    buf = porch._Buffer.upload(np.array([1, 2, 3, 4], dtype=np.float32))
    assert buf.download(4).tolist() == [1, 2, 3, 4]
