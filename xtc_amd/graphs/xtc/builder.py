# SPDX-License-Identifier: BSD-3-Clause
"""`with O.graph(name=...) as gb:` and graph (de)serialisation
(src/xtc/graphs/xtc/builder.py:16-87)."""

from __future__ import annotations

from pathlib import Path
from typing import Any

import yaml

from .context import XTCGraphContext
from .expr import OP_EXPRS, XTCExpr, XTCTensorExpr
from .graph import XTCGraph
from .operators import XTCOperator

__all__ = ["graph_builder"]


def _tuplify(obj: Any) -> Any:
    if isinstance(obj, dict):
        return {k: _tuplify(v) for k, v in obj.items()}
    if isinstance(obj, list):
        return tuple(_tuplify(v) for v in obj)
    return obj


class graph_builder:
    def __init__(self, **graph_kwargs: Any) -> None:
        self._graph_kwargs = graph_kwargs
        self._graph: XTCGraph | None = None

    def __enter__(self) -> "graph_builder":
        XTCGraphContext.push(**self._graph_kwargs)
        return self

    def __exit__(self, *_: Any) -> None:
        self._graph = XTCGraphContext.pop().graph

    @property
    def graph(self) -> XTCGraph:
        if self._graph is None:
            raise RuntimeError("the graph is only available after the builder block")
        return self._graph

    def set_outputs(self, *outs: XTCExpr) -> None:
        XTCGraphContext.current.set_outputs(*outs)

    def set_inputs(self, *inps: XTCExpr) -> None:
        XTCGraphContext.current.set_inputs(*inps)

    @classmethod
    def from_dict(cls, graph_dict: dict[str, Any]) -> dict[str, Any]:
        """Replays a serialised graph into the current scope."""
        from . import op_factory

        if "name" in graph_dict:
            XTCGraphContext.name(graph_dict["name"])
        exprs: dict[str, XTCExpr] = {}
        for inp in graph_dict["inputs"]:
            exprs[inp["uid"]] = XTCTensorExpr.from_dict(inp["expr"])
        XTCGraphContext.inputs(*exprs.values())
        for node in graph_dict["nodes"]:
            spec = node["expr"]
            op_name = spec["op"]["name"]
            if op_name not in OP_EXPRS:
                mismatch = (
                    "version mismatch detected, "
                    if graph_dict.get("ops_version") != XTCOperator.version_string()
                    else ""
                )
                raise ValueError(f"{mismatch}serialized op {op_name} is not implemented.")
            args = [exprs[a] for a in spec["args"]]
            fn = getattr(op_factory, op_name)
            exprs[node["uid"]] = fn(*args, name=node.get("name"), **_tuplify(spec["op"]["attrs"]))
        XTCGraphContext.outputs(*[exprs[o["uid"]] for o in graph_dict["outputs"]])
        return graph_dict

    @classmethod
    def loads(cls, text: str) -> None:
        cls.from_dict(yaml.safe_load(text))

    @classmethod
    def load(cls, file_name: str | Path) -> None:
        with open(file_name) as f:
            cls.from_dict(yaml.safe_load(f))
