# SPDX-License-Identifier: BSD-3-Clause
"""float64 numpy oracle for the XTC operators on the HIP hot path.

Test infrastructure only (see oracle/__init__.py).  Each function cites the
reference code whose semantics it restates.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np

__all__ = [
    "np_init",
    "matmul",
    "conv2d",
    "conv2d_direct",
    "relu",
    "pad",
    "pad2d_padding",
    "unpad",
    "round_bf16",
    "scaled_error",
    "seeded_uniform",
    "seeded_normal",
    "CONFIG_INPUTS",
]


def np_init(shape: Sequence[int], dtype: str) -> np.ndarray:
    """Default evaluation inputs: integers 1..9 cycling in C order.

    Follows src/xtc/utils/numpy.py:12-19 (arange(n) % 9 + 1, cast).
    """
    n = int(np.prod(shape)) if len(shape) else 1
    return (np.arange(n) % 9 + 1).reshape(shape).astype(dtype)


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """C = A @ B in float64 with XTC's reshape rules.

    Follows XTCOperMatmul.forward (src/xtc/graphs/xtc/operators.py:210-221):
    A is viewed as (shape[0], prod(rest)), B as (prod(rest[:-1]), last).
    """
    a2 = np.asarray(a, dtype=np.float64).reshape((a.shape[0], -1))
    b2 = np.asarray(b, dtype=np.float64).reshape((-1, b.shape[-1]))
    return a2 @ b2


def conv2d(inp: np.ndarray, weight: np.ndarray, stride: tuple[int, int] = (1, 1)) -> np.ndarray:
    """NHWC x RSCF -> NHWC valid convolution of an already padded input.

    Follows XTCOperConv2D.forward (src/xtc/graphs/xtc/operators.py:326-347):
    O[b,oh,ow,f] = sum_{r,s,c} I[b, oh*sh+r, ow*sw+s, c] * W[r,s,c,f] with
    OH = (H-R)//SH + 1; leading dims before H are flattened into the batch.
    Computed as im2col + float64 matmul (the reference loops per output).
    """
    x = np.asarray(inp, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    lead = x.shape[:-3]
    h, wd, c = x.shape[-3:]
    r, s, wc, f = w.shape
    assert wc == c, f"channel mismatch {c} != {wc}"
    sh, sw = stride
    oh, ow = (h - r) // sh + 1, (wd - s) // sw + 1
    xb = x.reshape((-1, h, wd, c))
    cols = np.empty((xb.shape[0], oh, ow, r, s, c), dtype=np.float64)
    for i in range(r):
        for j in range(s):
            cols[:, :, :, i, j, :] = xb[:, i : i + sh * (oh - 1) + 1 : sh, j : j + sw * (ow - 1) + 1 : sw, :]
    out = cols.reshape((-1, r * s * c)) @ w.reshape((r * s * c, f))
    return out.reshape((*lead, oh, ow, f))


def conv2d_direct(inp: np.ndarray, weight: np.ndarray, stride: tuple[int, int] = (1, 1)) -> np.ndarray:
    """Direct per-output loop (the reference's own formulation) for tiny shapes.

    Same loop structure as src/xtc/graphs/xtc/operators.py:337-341; used to
    cross-check the im2col restatement.
    """
    x = np.asarray(inp, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    h, wd, c = x.shape[-3:]
    r, s, _, f = w.shape
    sh, sw = stride
    oh, ow = (h - r) // sh + 1, (wd - s) // sw + 1
    xb = x.reshape((-1, h, wd, c))
    out = np.zeros((xb.shape[0], oh, ow, f), dtype=np.float64)
    for b, y, z, k in np.ndindex(out.shape):
        view = xb[b, y * sh : y * sh + r, z * sw : z * sw + s, :]
        out[b, y, z, k] = np.sum(view * w[:, :, :, k])
    return out.reshape((*x.shape[:-3], oh, ow, f))


def relu(x: np.ndarray, threshold: float = 0.0) -> np.ndarray:
    """max(x, threshold), NaN propagated.

    Follows XTCOperRelu.forward (src/xtc/graphs/xtc/operators.py:246-249).
    """
    return np.maximum(x, threshold)


def pad(x: np.ndarray, pads: Sequence[tuple[int, int]], value: float = 0.0) -> np.ndarray:
    """Constant padding with per-axis (before, after).

    Follows _OperPadImpl.forward (src/xtc/graphs/xtc/operators.py:413-433),
    i.e. numpy.pad(mode="constant").
    """
    return np.pad(x, list(pads), mode="constant", constant_values=value)


def unpad(x: np.ndarray, pads: Sequence[tuple[int, int]]) -> np.ndarray:
    """Crop of per-axis (before, after) elements: the inverse of pad.

    Follows XTCOperUnpad.forward (src/xtc/graphs/xtc/operators.py:683-702):
    the slice [before : dim - after] on every axis.
    """
    if len(pads) != x.ndim:
        raise ValueError("one (before, after) pair per axis")
    return x[tuple(slice(lo, d - hi) for d, (lo, hi) in zip(x.shape, pads))].copy()


def pad2d_padding(ndim: int, padding: int | tuple, axes: tuple[int, int] = (-3, -2)) -> list[tuple[int, int]]:
    """Per-axis pads of pad2d(padding, axes) (operators.py:484-541 forms)."""
    pads = [(0, 0)] * ndim
    if isinstance(padding, int):
        per = {axes[0]: (padding, padding), axes[1]: (padding, padding)}
    elif len(padding) == 1:
        per = {axes[0]: (padding[0], padding[0]), axes[1]: (padding[0], padding[0])}
    elif len(padding) == 2 and all(isinstance(p, int) for p in padding):
        per = {axes[0]: (padding[0], padding[1]), axes[1]: (padding[0], padding[1])}
    elif len(padding) == 2:
        per = {axes[0]: tuple(padding[0]), axes[1]: tuple(padding[1])}
    else:
        per = {axes[0]: (padding[0], padding[1]), axes[1]: (padding[2], padding[3])}
    for ax, p in per.items():
        pads[ax] = (int(p[0]), int(p[1]))
    return pads


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to nearest-even bf16, returned as float32."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, out)


def scaled_error(out: np.ndarray, ref: np.ndarray, k: int, amax_a: float, amax_b: float) -> float:
    """max|out - ref| / (sqrt(K) * max|A| * max|B|): the parity metric.

    Pass thresholds: 1e-4 for fp32 inputs, 1e-2 for bf16-rounded inputs.
    """
    denom = np.sqrt(k) * max(amax_a, 1e-30) * max(amax_b, 1e-30)
    return float(np.max(np.abs(np.asarray(out, np.float64) - np.asarray(ref, np.float64))) / denom)


def seeded_uniform(rng: np.random.Generator, shape: Sequence[int], low: float, high: float) -> np.ndarray:
    return rng.uniform(low, high, size=tuple(shape)).astype(np.float32)


def seeded_normal(rng: np.random.Generator, shape: Sequence[int], sigma: float) -> np.ndarray:
    return rng.normal(0.0, sigma, size=tuple(shape)).astype(np.float32)


def _c1(rng):
    return [seeded_uniform(rng, (512, 512), -1, 1), seeded_uniform(rng, (512, 512), -1, 1)]


def _c2(rng):
    return [seeded_uniform(rng, (4096, 4096), -1, 1), seeded_uniform(rng, (4096, 4096), -1, 1)]


def _c3a(rng):
    return [round_bf16(seeded_uniform(rng, (8192, 8192), -1, 1)), round_bf16(seeded_uniform(rng, (8192, 8192), -1, 1))]


def _c3b(rng):
    return [round_bf16(seeded_uniform(rng, (16, 8192), -1, 1)), round_bf16(seeded_uniform(rng, (8192, 8192), -1, 1))]


def _c4(rng):
    return [seeded_uniform(rng, (8, 56, 56, 64), 0, 1), seeded_normal(rng, (3, 3, 64, 64), float(np.sqrt(2.0 / (9 * 64))))]


def _c5(rng):
    return [
        seeded_uniform(rng, (2048, 1024), -1, 1),
        seeded_normal(rng, (1024, 4096), 0.02),
        seeded_normal(rng, (4096, 1024), 0.02),
    ]


# Seeded inputs of the BASELINE configurations: one default_rng(0) per
# configuration, inputs drawn in graph-input order.
CONFIG_INPUTS = {"C1": _c1, "C2": _c2, "C3a": _c3a, "C3b": _c3b, "C4": _c4, "C5": _c5}


def config_inputs(name: str) -> list[np.ndarray]:
    return CONFIG_INPUTS[name](np.random.default_rng(0))
