# SPDX-License-Identifier: BSD-3-Clause
"""Expressions built by the DSL functions (src/xtc/graphs/xtc/expr.py).

Every expression gets a process-wide increasing index; its uid is "%<idx>".
"""

from __future__ import annotations

import itertools
import threading
from collections.abc import Sequence
from typing import Any

from ...itf.data import Tensor, TensorType
from .data import XTCTensor, XTCTensorType
from .operators import (
    XTCOperator,
    XTCOperBiasAdd,
    XTCOperConv2D,
    XTCOperMatmul,
    XTCOperPad,
    XTCOperPad2D,
    XTCOperRelu,
    XTCOperReshape,
    XTCOperTensor,
    XTCOperTranspose,
    XTCOperUnpad,
)

__all__ = ["XTCExpr", "XTCTensorExpr", "XTCOpExpr", "OP_EXPRS"]

_counter = itertools.count()
_counter_lock = threading.Lock()


def _next_index() -> int:
    with _counter_lock:
        return next(_counter)


class XTCExpr:
    _idx_map: dict[int, "XTCExpr"] = {}

    def __init__(self) -> None:
        self._idx = _next_index()
        self._idx_map[self._idx] = self

    @property
    def uid(self) -> str:
        return f"%{self._idx}"

    @property
    def args(self) -> tuple["XTCExpr", ...]:
        return ()

    @property
    def op_name(self) -> str:
        raise NotImplementedError

    def forward_types(self, inputs_types: Sequence[TensorType]) -> Sequence[XTCTensorType]:
        raise NotImplementedError

    def forward(self, inputs: Sequence[Tensor]) -> Sequence[XTCTensor]:
        raise NotImplementedError

    def to_dict(self) -> dict[str, Any]:
        raise NotImplementedError

    def __str__(self) -> str:
        return f"{self.uid} = ?"


class XTCTensorExpr(XTCExpr):
    """A graph input: `O.tensor()`, `O.tensor((M, K), "float32")`,
    `O.tensor(shape=..., dtype=..., device=...)` or from a type/tensor."""

    def __init__(
        self,
        tensor: Any = None,
        shape: Any = None,
        dtype: str | None = None,
        device: Any = None,
        const: bool = False,
        layout: list[int] | None = None,
    ) -> None:
        super().__init__()
        if tensor is None:
            value = XTCTensor(type=XTCTensorType(shape, dtype, device, const, layout))
        elif isinstance(tensor, XTCTensorType):
            if shape is not None or dtype is not None or layout is not None or const:
                raise ValueError("tensor type given together with shape/dtype/layout/const")
            value = XTCTensor(type=tensor)
        elif isinstance(tensor, XTCTensor):
            if shape is not None or dtype is not None or layout is not None or const:
                raise ValueError("tensor value given together with shape/dtype/layout/const")
            value = tensor
        elif isinstance(tensor, tuple):
            if isinstance(shape, str):
                # O.tensor((M, K), "float32"): the dtype in second position
                if dtype is not None:
                    raise ValueError("dtype given twice")
                dtype, shape = shape, None
            value = XTCTensor(type=XTCTensorType(tensor, dtype, device, const, layout))
        else:
            raise TypeError(f"cannot build a tensor from {tensor!r}")
        self._value = value
        self._device = device
        self._op = XTCOperTensor()

    @property
    def value(self) -> XTCTensor:
        return self._value

    @property
    def type(self) -> XTCTensorType:
        return self._value.type

    @property
    def op_name(self) -> str:
        return self._op.name

    def forward_types(self, inputs_types: Sequence[TensorType]) -> Sequence[XTCTensorType]:
        if not self.type.is_constant():
            raise ValueError(f"tensor {self.uid} has no constant type")
        return [self.type]

    def forward(self, inputs: Sequence[Tensor]) -> Sequence[XTCTensor]:
        if not self.type.is_constant():
            raise ValueError(f"tensor {self.uid} has no constant type")
        return [self._value]

    def to_dict(self) -> dict[str, Any]:
        return {"type": self.type.to_dict()}

    @classmethod
    def from_dict(cls, spec: dict[str, Any]) -> "XTCTensorExpr":
        return cls(tensor=XTCTensorType.from_dict(spec["type"]))

    def __str__(self) -> str:
        return f"{self.uid} = {self.op_name}()"


class XTCOpExpr(XTCExpr):
    """An operator applied to argument expressions."""

    def __init__(self, op: XTCOperator, args: tuple[XTCExpr, ...]) -> None:
        super().__init__()
        self._op = op
        self._args = tuple(args)

    @property
    def op(self) -> XTCOperator:
        return self._op

    @property
    def op_name(self) -> str:
        return self._op.name

    @property
    def args(self) -> tuple[XTCExpr, ...]:
        return self._args

    def forward_types(self, inputs_types: Sequence[TensorType]) -> Sequence[XTCTensorType]:
        if len(inputs_types) != len(self._args):
            raise ValueError(f"{self.op_name}: {len(inputs_types)} input types for {len(self._args)} args")
        return self._op.forward_types(inputs_types)

    def forward(self, inputs: Sequence[Tensor]) -> Sequence[XTCTensor]:
        if len(inputs) != len(self._args):
            raise ValueError(f"{self.op_name}: {len(inputs)} inputs for {len(self._args)} args")
        return self._op.forward(inputs)

    def to_dict(self) -> dict[str, Any]:
        return {"op": self._op.to_dict(), "args": [a.uid for a in self._args]}

    def __str__(self) -> str:
        params = [a.uid for a in self._args] + [f"{k}={v}" for k, v in vars(self._op.attrs).items()]
        return f"{self.uid} = {self.op_name}({', '.join(params)})"


def _op_expr(cls: type[XTCOperator], arity: int):  # type: ignore[no-untyped-def]
    def make(*args: XTCExpr, **attrs: Any) -> XTCOpExpr:
        if len(args) != arity:
            raise TypeError(f"{cls.__name__} takes {arity} argument(s), got {len(args)}")
        return XTCOpExpr(cls(**attrs), tuple(args))

    return make


# DSL function name -> expression constructor
OP_EXPRS = {
    "matmul": _op_expr(XTCOperMatmul, 2),
    "conv2d": _op_expr(XTCOperConv2D, 2),
    "relu": _op_expr(XTCOperRelu, 1),
    "pad2d": _op_expr(XTCOperPad2D, 1),
    "pad": _op_expr(XTCOperPad, 1),
    "unpad": _op_expr(XTCOperUnpad, 1),
    "reshape": _op_expr(XTCOperReshape, 1),
    "transpose": _op_expr(XTCOperTranspose, 1),
    "bias_add": _op_expr(XTCOperBiasAdd, 2),
}
