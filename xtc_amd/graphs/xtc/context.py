# SPDX-License-Identifier: BSD-3-Clause
"""Graph-building scopes (src/xtc/graphs/xtc/context.py:17-135).

A thread-local stack of scopes; the bottom one is global.  Every expression
built by a DSL function is recorded in every open scope, so nested
`with O.graph(...)` blocks each see the expressions built inside them.  A
scope's graph inputs are the expressions it uses but does not define (plus
any declared with O.inputs); its outputs are the expressions it defines that
nothing in it uses (plus any declared with O.outputs).
"""

from __future__ import annotations

import threading
from typing import Any

from .expr import XTCExpr, XTCTensorExpr
from .graph import XTCGraph
from .node import XTCNode

__all__ = ["XTCGraphContext", "XTCGraphScope"]

_nodes_lock = threading.Lock()
_expr_nodes: dict[int, XTCNode] = {}


def node_of(expr: XTCExpr, name: str | None = None) -> XTCNode:
    """The unique node of an expression (created on first request)."""
    with _nodes_lock:
        node = _expr_nodes.get(expr._idx)
        if node is None:
            node = XTCNode(expr, name=name)
            _expr_nodes[expr._idx] = node
        return node


def _unique(exprs: list[XTCExpr]) -> list[XTCExpr]:
    return list({e._idx: e for e in exprs}.values())


class XTCGraphScope:
    def __init__(self, **graph_kwargs: Any) -> None:
        self._exprs: list[XTCExpr] = []
        self._names: list[str | None] = []
        self._inputs: list[XTCExpr] = []
        self._outputs: list[XTCExpr] = []
        self.graph_kwargs = dict(graph_kwargs)

    def add_expr(self, expr: XTCExpr, name: str | None = None) -> None:
        self._exprs.append(expr)
        self._names.append(name)

    def add_inputs(self, *exprs: XTCExpr) -> None:
        self._inputs.extend(exprs)

    def add_outputs(self, *exprs: XTCExpr) -> None:
        self._outputs.extend(exprs)

    def set_inputs(self, *exprs: XTCExpr) -> None:
        self._inputs = list(exprs)

    def set_outputs(self, *exprs: XTCExpr) -> None:
        self._outputs = list(exprs)

    def _graph_inputs(self) -> list[XTCExpr]:
        defined = {e._idx for e in self._exprs}
        used = [a for e in self._exprs for a in e.args if a._idx not in defined]
        return _unique(self._inputs + sorted(_unique(used), key=lambda e: e._idx))

    def _graph_outputs(self) -> list[XTCExpr]:
        used = {a._idx for e in self._exprs for a in e.args}
        return _unique(self._outputs + [e for e in self._exprs if e._idx not in used])

    @property
    def graph(self) -> XTCGraph:
        graph = XTCGraph(**self.graph_kwargs)
        graph.add_nodes([node_of(e, n) for e, n in zip(self._exprs, self._names)])
        inputs = [node_of(e) for e in self._graph_inputs()]
        graph.set_inputs(inputs)
        graph.set_outputs([node_of(e) for e in self._graph_outputs()])
        exprs = [n.expr for n in inputs]
        if all(isinstance(e, XTCTensorExpr) and e.type.is_constant() for e in exprs):
            graph.forward_types([e.type for e in exprs])  # type: ignore[attr-defined]
        return graph


class XTCGraphScopes(threading.local):
    def __init__(self) -> None:
        self._scopes = [XTCGraphScope()]

    def push(self, **graph_kwargs: Any) -> None:
        self._scopes.append(XTCGraphScope(**graph_kwargs))

    def pop(self) -> XTCGraphScope:
        if len(self._scopes) <= 1:
            raise RuntimeError("no graph scope to close")
        return self._scopes.pop()

    @property
    def current(self) -> XTCGraphScope:
        return self._scopes[-1]

    def append(self, expr: XTCExpr, name: str | None = None) -> XTCExpr:
        for scope in self._scopes:
            scope.add_expr(expr, name)
        return expr

    def inputs(self, *exprs: XTCExpr) -> None:
        self.current.add_inputs(*exprs)

    def outputs(self, *exprs: XTCExpr) -> None:
        self.current.add_outputs(*exprs)

    def name(self, name: str) -> None:
        self.current.graph_kwargs["name"] = name


XTCGraphContext = XTCGraphScopes()
