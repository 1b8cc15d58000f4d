# SPDX-License-Identifier: BSD-3-Clause
"""Graph nodes: one per expression, one output each (src/xtc/graphs/xtc/node.py)."""

from __future__ import annotations

from collections.abc import Sequence
from typing import Any

from ...itf.data import Tensor, TensorType
from ...itf.graph import Node
from .data import XTCTensor, XTCTensorType
from .expr import XTCExpr, XTCOpExpr, XTCTensorExpr
from .operation import XTCOperation
from .operators import XTCOperator

__all__ = ["XTCNode"]


class XTCNode(Node):
    _by_uid: dict[str, "XTCNode"] = {}

    def __init__(self, expr: XTCExpr, name: str | None = None) -> None:
        self._expr = expr
        self._name = name if name is not None else expr.uid
        self._inputs_types: list[XTCTensorType] | None = None
        self._outputs_types: list[XTCTensorType] | None = None
        self._by_uid[expr.uid] = self

    @classmethod
    def lookup(cls, uid: str) -> "XTCNode":
        if uid not in cls._by_uid:
            raise KeyError(f"no node with uid {uid}")
        return cls._by_uid[uid]

    @property
    def expr(self) -> XTCExpr:
        return self._expr

    @property
    def uid(self) -> str:
        return self._expr.uid

    @property
    def name(self) -> str:
        return self._name

    @property
    def operator(self) -> XTCOperator:
        return self._expr._op  # type: ignore[attr-defined,no-any-return]

    @property
    def inputs(self) -> list[str]:
        return [a.uid for a in self._expr.args]

    @property
    def outputs(self) -> list[str]:
        return [self.uid]

    @property
    def preds(self) -> Sequence[str]:
        return list(dict.fromkeys(self.inputs))

    @property
    def preds_nodes(self) -> Sequence["XTCNode"]:
        return [self.lookup(uid) for uid in self.preds]

    @property
    def inputs_types(self) -> Sequence[XTCTensorType] | None:
        return self._inputs_types

    @property
    def outputs_types(self) -> Sequence[XTCTensorType] | None:
        return self._outputs_types

    def is_tensor(self) -> bool:
        return isinstance(self._expr, XTCTensorExpr)

    def forward_types(self, inputs_types: Sequence[TensorType]) -> Sequence[XTCTensorType]:
        self._inputs_types = list(inputs_types)  # type: ignore[arg-type]
        self._outputs_types = list(self._expr.forward_types(inputs_types))
        return self._outputs_types

    def forward(self, inputs: Sequence[Tensor]) -> Sequence[XTCTensor]:
        return self._expr.forward(inputs)

    @property
    def operation(self) -> XTCOperation:
        if self._inputs_types is None or self._outputs_types is None:
            raise ValueError(f"node {self.uid}: types were not forwarded")
        return self.operator.get_operation(self._inputs_types, self._outputs_types)

    def to_dict(self) -> dict[str, Any]:
        out: dict[str, Any] = {}
        if self._name != self.uid:
            out["name"] = self._name
        out["uid"] = self.uid
        out["expr"] = self._expr.to_dict()
        return out

    def __str__(self) -> str:
        text = str(self._expr).split("=", 1)[1].strip()
        if self._name != self.uid:
            text += f" {{name = {self._name!r}}}"
        if self._inputs_types is not None and self._outputs_types is not None:
            text += f" : {self._inputs_types} -> {self._outputs_types}"
        return text

    def __repr__(self) -> str:
        return f"XTCNode({self.uid})"


def is_op_node(node: XTCNode) -> bool:
    return isinstance(node.expr, XTCOpExpr)
