# SPDX-License-Identifier: BSD-3-Clause
"""Every named operation of `loop-explore --op-name` on the GPU.

The reference's operation registry (src/xtc/artifacts, restated in
xtc_amd.artifacts) names 76 layer shapes: the convolutions of Yolo9000,
MobileNet, ResNet18, SqueezeNet and AlexNet, and the matmuls of Llama3,
Gemma, Polybench and AlexNet.  Each is built as `loop-explore` builds it
(xtc_amd.cli.explore.build_graph, the reference's input shapes), compiled
with the backend's default schedule, in fp32 and in bf16 (bf16 operands,
fp32 accumulation and output), run on seeded inputs and compared with the
float64 oracle under the tolerance max|out-ref| / (sqrt(K) max|A| max|B|)
<= 1e-4 (fp32) or 1e-2 (bf16).  Convolutions are checked on every output; matmuls on 48
rows spread over M and on a 64-column band through all of M.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import reference as ref
from xtc_amd.artifacts import list_operations
from xtc_amd.backends.hip import Backend
from xtc_amd.cli.explore import _operation_dims, build_graph

pytestmark = pytest.mark.gpu

TOL = {"float32": 1e-4, "bfloat16": 1e-2}
OPS = list_operations()
CASES = [(op, name, dtype) for dtype in ("float32", "bfloat16") for op, name in OPS]


def _inputs(op: str, dims: list[int], seed: int, dtype: str) -> list[np.ndarray]:
    rng = np.random.default_rng(seed)
    if op == "matmul":
        i, j, k = dims
        out = [ref.seeded_uniform(rng, (i, k), -1, 1), ref.seeded_uniform(rng, (k, j), -1, 1)]
    else:
        n, h, w, f, r, s, c, sh, sw = dims
        x = ref.seeded_uniform(rng, (n, h * sh + r - 1, w * sw + s - 1, c), 0, 1)
        wt = ref.seeded_normal(rng, (r, s, c, f), float(np.sqrt(2.0 / (r * s * c))))
        out = [x, wt]
    # bf16 operands: the oracle sees the rounded values (fp32 accumulation, fp32 output)
    return [ref.round_bf16(a) for a in out] if dtype == "bfloat16" else out


@pytest.mark.parametrize("op,name,dtype", CASES, ids=[f"{name}-{dtype}" for _, name, dtype in CASES])
def test_named_operation_parity(op, name, dtype):
    dims = _operation_dims(op, name)
    print(f"[named] {op} {name} {dtype} dims={dims}", flush=True)
    graph = build_graph(op, dims, dtype, name=name.lower())
    backend = Backend(graph)
    module = backend.get_compiler().compile(backend.get_scheduler().schedule())
    inputs = _inputs(op, dims, OPS.index((op, name)), dtype)
    tol = TOL[dtype]
    outs = [np.empty(t.constant_shape, np.float32) for t in graph.outputs_types]
    res, code, msg = module.get_evaluator(parameters=(inputs, outs), repeat=1, number=1, min_repeat_ms=0).evaluate()
    assert code == 0, msg
    (out,) = outs
    a, b = inputs
    amax_a, amax_b = float(np.abs(a).max()), float(np.abs(b).max())
    if op == "conv2d":
        sh, sw = dims[7], dims[8]
        k = int(np.prod(b.shape[:3]))
        expect = ref.conv2d(a, b, (sh, sw))
        assert ref.scaled_error(out, expect, k, amax_a, amax_b) <= tol
        return
    m, n, k = dims
    rows = np.unique(np.linspace(0, m - 1, min(m, 48)).astype(int))
    expect = ref.matmul(a[rows], b)
    assert ref.scaled_error(out[rows], expect, k, amax_a, amax_b) <= tol
    cols = slice(max(0, n - 64), n)
    expect = a.astype(np.float64) @ b[:, cols].astype(np.float64)
    assert ref.scaled_error(out[:, cols], expect, k, amax_a, amax_b) <= tol
