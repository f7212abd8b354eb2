"""Child process of tests/test_disk_cache.py's GPU tests (not collected by
pytest): materialises the five benchmark graphs at small sizes with the
persistent code-object cache in the directory named by PORCH_CACHE_DIR,
compares each with the oracle, and prints one JSON line: the JIT counters
of this process, the number of kernels the graphs launched, and which
graphs matched the oracle (bit for bit for the elementwise and view graphs,
1e-6 / 1e-5 / 1e-4 relative for softmax, the logistic row sum and the
matmul)."""

import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

import porch_amd as porch  # noqa: E402
from oracle import host  # noqa: E402
from porch_amd.workloads import config_graph, config_inputs, config_shapes  # noqa: E402

SIZES = {
    "elementwise": {"n": 4099},
    "view_chain": {"n": 130},
    "softmax": {"rows": 7, "cols": 2100},
    "logistic_rowsum": {"rows": 35, "cols": 40},
    "matmul_epilogue": {"m": 200, "k": 70, "n": 136},
}
BARS = {"elementwise": 0.0, "view_chain": 0.0, "softmax": 1e-6, "logistic_rowsum": 1e-5, "matmul_epilogue": 1e-4}


def main():
    assert porch.disk_cache_directory() == os.environ["PORCH_CACHE_DIR"]
    kernels = 0
    matched = {}
    for name, size in SIZES.items():
        tensors = [porch.tensor(s, v) for s, v in zip(config_shapes(name, size), config_inputs(name, size))]
        expr = config_graph(name, tensors, size)
        kernels += len(porch.plan(expr)["kernels"])
        out = porch.materialize(expr).cpu().reshape(expr.shape())
        ref = host.evaluate(expr)
        if BARS[name] == 0.0:
            matched[name] = bool(np.array_equal(out.view(np.uint32), ref.view(np.uint32)))
        else:
            err = np.abs(out.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)), 1e-30)
            matched[name] = bool(err.max() <= BARS[name])
    stats = porch.jit_stats()
    print(json.dumps({"compiles": stats["compiles"], "disk_hits": stats["disk_hits"], "kernels": kernels,
                      "matched": matched}))


if __name__ == "__main__":
    main()
