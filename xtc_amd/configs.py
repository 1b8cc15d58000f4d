# SPDX-License-Identifier: BSD-3-Clause
"""The benchmark workloads C1-C5 as XTC graphs, their seeded inputs, and the
tuned schedules that bench.py measures and the GPU parity tests check.

  C1  fp32 matmul 512^3
  C2  fp32 matmul 4096^3
  C3a bf16-input matmul 8192^3, fp32 accumulate and output
  C3b bf16-input matmul M=16, N=K=8192, fp32 output
  C4  NHWC fp32 pad2d(1) -> conv2d 3x3 -> relu, N=8, H=W=56, C=F=64
  C5  fp32 MLP X[2048,1024] @ W1[1024,4096] -> relu -> @ W2[4096,1024]

Inputs: one numpy default_rng(0) per workload, drawn in graph-input order in
float64, cast to float32 (bf16 inputs rounded to nearest even).
"""

from __future__ import annotations

from typing import Any

import numpy as np

__all__ = ["WORKLOADS", "SCHEDULES", "graph", "inputs", "apply_schedule", "flops", "alg_bytes"]

WORKLOADS = ("C1", "C2", "C3a", "C3b", "C4", "C5")


def graph(cfg: str) -> Any:
    """The XTC graph of workload `cfg`."""
    from .graphs.xtc import op as O

    if cfg == "C3a":
        a = O.tensor((8192, 8192), "bfloat16", name="A")
        b = O.tensor((8192, 8192), "bfloat16", name="B")
        with O.graph(name="matmul_bf16") as gb:
            O.matmul(a, b, name="C", out_dtype="float32")
    elif cfg == "C3b":
        a = O.tensor((16, 8192), "bfloat16", name="A")
        b = O.tensor((8192, 8192), "bfloat16", name="B")
        with O.graph(name="matmul_skinny") as gb:
            O.matmul(a, b, name="C", out_dtype="float32")
    elif cfg in ("C1", "C2"):
        n = 512 if cfg == "C1" else 4096
        a = O.tensor((n, n), "float32", name="A")
        b = O.tensor((n, n), "float32", name="B")
        with O.graph(name="matmul") as gb:
            O.matmul(a, b, name="C")
    elif cfg == "C4":
        x = O.tensor((8, 56, 56, 64), "float32", name="I")
        w = O.tensor((3, 3, 64, 64), "float32", name="W")
        with O.graph(name="conv_relu") as gb:
            p = O.pad2d(x, padding=1, axes=(1, 2), name="pad")
            c = O.conv2d(p, w, name="conv")
            O.relu(c, name="relu")
    elif cfg == "C5":
        x = O.tensor((2048, 1024), "float32", name="X")
        w1 = O.tensor((1024, 4096), "float32", name="W1")
        w2 = O.tensor((4096, 1024), "float32", name="W2")
        with O.graph(name="mlp") as gb:
            h = O.relu(O.matmul(x, w1, name="fc1"), name="act")
            O.matmul(h, w2, name="fc2")
    else:
        raise ValueError(f"unknown workload {cfg!r} (one of {', '.join(WORKLOADS)})")
    return gb.graph


def inputs(cfg: str, g: Any) -> list[np.ndarray]:
    """Seeded inputs of workload `cfg` for its graph `g`."""
    from .utils.bf16 import round_to_bf16

    rng = np.random.default_rng(0)
    out = []
    for t in g.inputs_types:
        shape = tuple(t.constant_shape)
        if cfg == "C4" and len(shape) == 4 and shape[0] == 3:
            arr = rng.normal(0.0, np.sqrt(2.0 / (9 * 64)), size=shape)
        elif cfg == "C4":
            arr = rng.uniform(0.0, 1.0, size=shape)
        elif cfg == "C5" and shape != (2048, 1024):
            arr = rng.normal(0.0, 0.02, size=shape)
        else:
            arr = rng.uniform(-1.0, 1.0, size=shape)
        arr = arr.astype(np.float32)
        out.append(round_to_bf16(arr) if t.constant_dtype == "bfloat16" else arr)
    return out


# Tuned schedules, written with XTC's scheduling primitives: the first tile
# level of i/j is the workgroup tile, the second the wave tile, k's first
# level the LDS slab; parallelize on k splits K (its first level is then the
# slice per split, its second the slab); unroll of the loop that walks the
# slabs sets the pipeline depth (LDS stages).  The mapping onto kernel template
# parameters is in xtc_amd/backends/hip/mapping.py.  Picked with
# loop-explore --strategy tile_hip on MI355X; nodes without an entry keep the
# library's default tile.
SCHEDULES: dict[str, dict[str, dict[str, Any]]] = {
    "C3a": {"C": {"tile": {"i": {"i1": 256, "i2": 128}, "j": {"j1": 256, "j2": 64}, "k": {"k1": 32}}}},
    "C2": {"C": {"tile": {"i": {"i1": 128, "i2": 64}, "j": {"j1": 256, "j2": 64}, "k": {"k1": 32}},
                 "unroll": {"k": 2}}},
    "C1": {"C": {"tile": {"i": {"i1": 32, "i2": 32}, "j": {"j1": 32, "j2": 32}, "k": {"k1": 128, "k2": 16}},
                 "parallelize": ["i", "j", "k"]}},
    "C5": {
        "fc1": {"tile": {"i": {"i1": 128, "i2": 64}, "j": {"j1": 256, "j2": 64}, "k": {"k1": 32}}},
        "fc2": {"tile": {"i": {"i1": 128, "i2": 64}, "j": {"j1": 128, "j2": 32}, "k": {"k1": 2048, "k2": 32}},
                "parallelize": ["i", "j", "k"]},
    },
}


def apply_schedule(sch: Any, cfg: str) -> Any:
    """Applies SCHEDULES[cfg] to the HIP scheduler `sch`; returns it."""
    for node, spec in SCHEDULES.get(cfg, {}).items():
        node_sch = sch.for_node(node)
        for dim, tiles in spec.get("tile", {}).items():
            node_sch.tile(dim, tiles)
        if "interchange" in spec:
            node_sch.interchange(spec["interchange"])
        if "parallelize" in spec:
            node_sch.parallelize(spec["parallelize"])
        if "vectorize" in spec:
            node_sch.vectorize(spec["vectorize"])
        if "unroll" in spec:
            node_sch.unroll(spec["unroll"])
    return sch


def flops(cfg: str) -> int:
    """Useful FLOP of one step (2 per multiply-accumulate)."""
    return {
        "C1": 2 * 512**3,
        "C2": 2 * 4096**3,
        "C3a": 2 * 8192**3,
        "C3b": 2 * 16 * 8192 * 8192,
        "C4": 2 * 8 * 56 * 56 * 64 * 576,
        "C5": 2 * 2048 * 4096 * 1024 * 2,
    }[cfg]


def alg_bytes(cfg: str) -> int:
    """Algorithmic HBM bytes of one step: every input read once, every
    output written once (C5 also writes and reads its hidden activation)."""
    return {
        "C1": 3 * 512 * 512 * 4,
        "C2": 3 * 4096 * 4096 * 4,
        "C3a": 2 * 8192 * 8192 * 2 + 8192 * 8192 * 4,
        "C3b": 16 * 8192 * 2 + 8192 * 8192 * 2 + 16 * 8192 * 4,
        "C4": 8 * 56 * 56 * 64 * 4 * 2 + 9 * 64 * 64 * 4,
        "C5": (2048 * 1024 + 1024 * 4096 + 2 * 2048 * 4096 + 4096 * 1024 + 2048 * 1024) * 4,
    }[cfg]
