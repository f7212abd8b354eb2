"""The five benchmark graphs of the MI355X fused-graph path, at any size.

Each is porch source over seeded synthetic inputs (splitmix64, see
porch_amd.synth):
  elementwise      (a + b) * 2 - 1       a, b ~ U[-1,1] length 2^20
  view_chain       concat(transpose(x[0::2,1::2]), transpose(x[1::2,0::2]), 0) + 1
                                         x ~ N(0,1) [4096,4096]
  softmax          softmax(x, 1)         x ~ N(0,3) [8192,4096], 1% set to +20
  logistic_rowsum  sum(logistic(relu(x*w + bias)), 1)
                                         x ~ N(0,1) [16384,2048], w ~ U(.5,1.5),
                                         bias ~ N(0,.1) [1,2048]
  matmul_epilogue  relu(A @ B + bias) - 0.5
                                         A, B ~ U(-1,1)/64 [4096,4096],
                                         bias ~ N(0,.01) [1,4096]
and `copy`, reshape(x) over x [8192,8192]: a plain copy of known size used to
calibrate hardware byte counters.

Three more measure the IR extensions (permute, batched_matmul):
  batched_transpose  permute(x, [0, 2, 1])  x ~ U[-1,1] [64,512,512]
  heads_permute      permute(x, [0, 2, 1, 3])
                                         x ~ U[-1,1] [32,1024,16,128]
  batched_matmul     relu(batched_matmul(A, B) + bias) - 0.5
                                         A, B ~ U(-1,1)/32 [32,1024,1024],
                                         bias ~ N(0,.01) [1,1,1024]

Two more, not in the default run, measure shapes the others do not reach:
  attention_scores   batched_matmul(q, k) * 0.125
                                         q ~ U(-1,1) [16,4096,64], k ~ U(-1,1)
                                         [16,64,4096] (a short K: the
                                         persistent product kernel)
  vocab_softmax      softmax(x, 1)       x ~ N(0,3) [512,262144], 1% set to +20
                                         (rows beyond the register cache)
"""

from __future__ import annotations

import numpy as np

import porch_amd as porch
from porch_amd import synth

# -----------------------------------------------------------------------------

def config_inputs(name: str, size: dict | None = None) -> list[np.ndarray]:
    s = dict(CONFIG_SIZES[name])
    s.update(size or {})
    if name == "elementwise":
        n = s["n"]
        return [synth.uniform(n, 101, -1.0, 1.0), synth.uniform(n, 102, -1.0, 1.0)]
    if name == "view_chain":
        n = s["n"]
        return [synth.normal(n * n, 201, 0.0, 1.0)]
    if name == "softmax":
        rows, cols = s["rows"], s["cols"]
        x = synth.normal(rows * cols, 301, 0.0, 3.0)
        synth.replace(x, 302, 0.01, 20.0)
        return [x]
    if name == "logistic_rowsum":
        rows, cols = s["rows"], s["cols"]
        return [synth.normal(rows * cols, 401, 0.0, 1.0), synth.uniform(cols, 402, 0.5, 1.5),
                synth.normal(cols, 403, 0.0, 0.1)]
    if name == "copy":
        return [synth.uniform(s["n"] * s["n"], 601, -1.0, 1.0)]
    if name in ("batched_transpose", "heads_permute"):
        return [synth.uniform(int(np.prod(config_shapes(name, size)[0])), 701, -1.0, 1.0)]
    if name == "batched_matmul":
        b, m, k, n = s["batch"], s["m"], s["k"], s["n"]
        return [synth.uniform(b * m * k, 801, -1.0, 1.0) / np.float32(32.0),
                synth.uniform(b * k * n, 802, -1.0, 1.0) / np.float32(32.0),
                synth.normal(n, 803, 0.0, 0.01)]
    if name == "attention_scores":
        b, m, k, n = s["batch"], s["m"], s["k"], s["n"]
        return [synth.uniform(b * m * k, 811, -1.0, 1.0), synth.uniform(b * k * n, 812, -1.0, 1.0)]
    if name == "vocab_softmax":
        rows, cols = s["rows"], s["cols"]
        x = synth.normal(rows * cols, 901, 0.0, 3.0)
        synth.replace(x, 902, 0.01, 20.0)
        return [x]
    if name == "matmul_epilogue":
        m, k, n = s["m"], s["k"], s["n"]
        return [synth.uniform(m * k, 501, -1.0, 1.0) / np.float32(64.0),
                synth.uniform(k * n, 502, -1.0, 1.0) / np.float32(64.0),
                synth.normal(n, 503, 0.0, 0.01)]
    if name in ("narrow_product", "wide_product"):
        m, k, n = s["m"], s["k"], s["n"]
        seed = 1001 if name == "narrow_product" else 1011
        return [synth.uniform(m * k, seed, -1.0, 1.0), synth.uniform(k * n, seed + 1, -1.0, 1.0)]
    raise ValueError(name)


CONFIG_SIZES = {
    "elementwise": {"n": 1 << 20},
    "view_chain": {"n": 4096},
    "softmax": {"rows": 8192, "cols": 4096},
    "logistic_rowsum": {"rows": 16384, "cols": 2048},
    "matmul_epilogue": {"m": 4096, "k": 4096, "n": 4096},
    "copy": {"n": 8192},
    "batched_transpose": {"batch": 64, "rows": 512, "cols": 512},
    "heads_permute": {"batch": 32, "seq": 1024, "heads": 16, "dim": 128},
    "batched_matmul": {"batch": 32, "m": 1024, "k": 1024, "n": 1024},
    "attention_scores": {"batch": 16, "m": 4096, "k": 64, "n": 4096},
    "vocab_softmax": {"rows": 512, "cols": 262144},
    # products with one short side: 16 columns (gemm.narrow), 32 rows (gemm.wide)
    "narrow_product": {"m": 4096, "k": 4096, "n": 16},
    "wide_product": {"m": 32, "k": 4096, "n": 4096},
}


def config_shapes(name: str, size: dict | None = None) -> list[list[int]]:
    s = dict(CONFIG_SIZES[name])
    s.update(size or {})
    if name == "elementwise":
        return [[s["n"]], [s["n"]]]
    if name == "view_chain":
        return [[s["n"], s["n"]]]
    if name == "softmax":
        return [[s["rows"], s["cols"]]]
    if name == "logistic_rowsum":
        return [[s["rows"], s["cols"]], [1, s["cols"]], [1, s["cols"]]]
    if name == "matmul_epilogue":
        return [[s["m"], s["k"]], [s["k"], s["n"]], [1, s["n"]]]
    if name == "copy":
        return [[s["n"], s["n"]]]
    if name == "batched_transpose":
        return [[s["batch"], s["rows"], s["cols"]]]
    if name == "heads_permute":
        return [[s["batch"], s["seq"], s["heads"], s["dim"]]]
    if name == "batched_matmul":
        b, m, k, n = s["batch"], s["m"], s["k"], s["n"]
        return [[b, m, k], [b, k, n], [1, 1, n]]
    if name == "attention_scores":
        b, m, k, n = s["batch"], s["m"], s["k"], s["n"]
        return [[b, m, k], [b, k, n]]
    if name == "vocab_softmax":
        return [[s["rows"], s["cols"]]]
    if name in ("narrow_product", "wide_product"):
        return [[s["m"], s["k"]], [s["k"], s["n"]]]
    raise ValueError(name)


def config_graph(name: str, tensors, size: dict | None = None):
    """The benchmark graph of config `name` over `tensors` (porch source)."""
    s = dict(CONFIG_SIZES[name])
    s.update(size or {})
    if name == "elementwise":
        a, b = tensors
        return (a + b) * 2.0 - 1.0
    if name == "view_chain":
        (x,) = tensors
        n = s["n"]
        return porch.concat(
            porch.transpose(x[porch.slice(0, n, 2), porch.slice(1, n, 2)]),
            porch.transpose(x[porch.slice(1, n, 2), porch.slice(0, n, 2)]), 0) + 1.0
    if name == "softmax":
        (x,) = tensors
        return porch.softmax(x, 1)
    if name == "logistic_rowsum":
        x, w, b = tensors
        shape = [s["rows"], s["cols"]]
        return porch.sum(porch.logistic(porch.relu(
            x * porch.broadcast_to(w, shape) + porch.broadcast_to(b, shape))), 1)
    if name == "matmul_epilogue":
        a, b, bias = tensors
        shape = [s["m"], s["n"]]
        return porch.relu(porch.matmul(a, b) + porch.broadcast_to(bias, shape)) - 0.5
    if name == "copy":
        (x,) = tensors
        return porch.reshape(x, [s["n"] * s["n"]])
    if name == "batched_transpose":
        (x,) = tensors
        return porch.permute(x, [0, 2, 1])
    if name == "heads_permute":
        (x,) = tensors
        return porch.permute(x, [0, 2, 1, 3])
    if name == "batched_matmul":
        a, b, bias = tensors
        shape = [s["batch"], s["m"], s["n"]]
        return porch.relu(porch.batched_matmul(a, b) + porch.broadcast_to(bias, shape)) - 0.5
    if name == "attention_scores":
        q, k = tensors
        return porch.batched_matmul(q, k) * 0.125
    if name == "vocab_softmax":
        (x,) = tensors
        return porch.softmax(x, 1)
    if name in ("narrow_product", "wide_product"):
        a, b = tensors
        return porch.matmul(a, b)
    raise ValueError(name)
