# SPDX-License-Identifier: BSD-3-Clause
"""DSL functions: `O.tensor`, `O.matmul`, ... (src/xtc/graphs/xtc/op_factory.py:22-112)."""

from __future__ import annotations

from typing import Any

from .context import XTCGraphContext
from .data import XTCTensorType
from .expr import OP_EXPRS, XTCExpr, XTCTensorExpr

__all__ = [
    "matmul",
    "conv2d",
    "pad2d",
    "unpad",
    "pad",
    "relu",
    "reshape",
    "transpose",
    "bias_add",
    "tensor",
    "inputs",
    "outputs",
    "type",
]


def _append(op: str, *args: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    return XTCGraphContext.append(OP_EXPRS[op](*args, **attrs), name=name)


def matmul(a: XTCExpr, b: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    return _append("matmul", a, b, name=name, **attrs)


def conv2d(inp: XTCExpr, weight: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    return _append("conv2d", inp, weight, name=name, **attrs)


def pad2d(inp: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    return _append("pad2d", inp, name=name, **attrs)


def unpad(inp: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    return _append("unpad", inp, name=name, **attrs)


def pad(inp: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    return _append("pad", inp, name=name, **attrs)


def relu(inp: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    return _append("relu", inp, name=name, **attrs)


def reshape(inp: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    return _append("reshape", inp, name=name, **attrs)


def transpose(inp: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    return _append("transpose", inp, name=name, **attrs)


def bias_add(inp: XTCExpr, bias: XTCExpr, name: str | None = None, **attrs: Any) -> XTCExpr:
    """Extension: adds a per-last-axis bias (fused into the producing GEMM)."""
    return _append("bias_add", inp, bias, name=name, **attrs)


def tensor(*args: Any, name: str | None = None, **attrs: Any) -> XTCExpr:
    return XTCGraphContext.append(XTCTensorExpr(*args, **attrs), name=name)


def inputs(*inps: XTCExpr) -> None:
    XTCGraphContext.inputs(*inps)


def outputs(*outs: XTCExpr) -> None:
    XTCGraphContext.outputs(*outs)


def type(*args: Any, **attrs: Any) -> XTCTensorType:  # noqa: A001 - mirrors the DSL name
    return XTCTensorType(*args, **attrs)
