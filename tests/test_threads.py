"""The host library from several threads at once (no GPU): planning, offline
hiprtc compilation through the shared code-object cache, and per-thread
error messages.  Each thread's results must equal the single-threaded ones.
Also the program run under ThreadSanitizer (make -C porch_amd tsan)."""

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import porch_amd as porch
from tests.helpers import placeholder
from tests.test_gpu_fuzz import integer_leaf, random_graph


def _graphs():
    rng = np.random.default_rng(77)
    graphs = [random_graph(rng, integer_leaf) for _ in range(6)]
    graphs += [porch.softmax(placeholder([64, 100 + k]), 1) for k in range(3)]
    graphs += [porch.softmax(placeholder([3, 65540]), 1)]
    return graphs


def _describe(expr):
    plan = porch.plan(expr, compile=True)
    sources = [porch.kernel_source(expr, i) for i in range(len(plan["kernels"]))]
    kernels = [(k["kind"], tuple(k["grid"]), k["block"], k["dest"], k["code_bytes"] > 0) for k in plan["kernels"]]
    return kernels, plan["temps"], sources


def test_concurrent_planning_and_compilation_match_one_thread():
    graphs = _graphs()
    alone = [_describe(g) for g in graphs]
    # every thread walks all graphs, starting at a different one, so the
    # same graph is planned and compiled by several threads at once
    def walk(start):
        return [(i, _describe(graphs[i])) for i in [(start + k) % len(graphs) for k in range(len(graphs))]]

    with ThreadPoolExecutor(6) as pool:
        for results in pool.map(walk, range(6)):
            for i, described in results:
                assert described == alone[i], i


def _failures(k):
    """The error of an invalid graph of thread k (each thread's own), raised
    50 times with valid calls in between."""
    bad = [lambda: porch.matmul(placeholder([2, 3]), placeholder([2, 2])).shape(),
           lambda: placeholder([3, 4])[3],
           lambda: placeholder([3, 4])[porch.slice(0, 3, 0)],
           lambda: porch.concat(placeholder([2, 3]), placeholder([3, 4]), 0).shape()][k]
    messages = []
    for _ in range(50):
        with pytest.raises((porch.InvalidArgument, porch.OutOfRange)) as caught:
            bad()
        messages.append(str(caught.value))
        assert (placeholder([2, 3]) + 1.0).shape() == [2, 3]
    return messages


def test_error_messages_stay_with_their_thread():
    expected = [_failures(k)[0] for k in range(4)]
    assert len(set(expected)) == 4, expected
    with ThreadPoolExecutor(4) as pool:
        for k, messages in enumerate(pool.map(_failures, range(4))):
            assert messages == [expected[k]] * 50, (k, messages[:3])
