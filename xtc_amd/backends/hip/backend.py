# SPDX-License-Identifier: BSD-3-Clause
"""HipBackend: the XTC Backend of the MI355X kernels.

Drop-in for `xtc.backends.<name>.Backend(graph, **kwargs)`
(src/xtc/itf/back/backend.py:13-56, instantiated by name in
src/xtc/search/explore.py:262-268 with `use_tensor_dialect=`).  The graph is
lowered once to a kernel-launch plan (lowering.py); the Scheduler records
transformations per operator node; the Compiler maps them onto kernel
template parameters and emits the payload.
"""

from __future__ import annotations

from typing import Any

from ...itf.back import Backend
from .compiler import HipCompiler
from .lowering import Plan, UnsupportedGraph, lower_graph
from .scheduler import HipScheduler

__all__ = ["HipBackend"]


class HipBackend(Backend):
    def __init__(self, graph: Any, **kwargs: Any) -> None:
        # kwargs of other backends (use_tensor_dialect, always_vectorize, ...)
        # have no meaning here and are accepted for call-site compatibility.
        self._graph = graph
        self._kwargs = dict(kwargs)
        if graph.outputs_types is None and graph.inputs_types is None:
            raise UnsupportedGraph("graph input types are unknown: build it from typed O.tensor inputs")
        self._plan = lower_graph(graph)
        self._ops: dict[str, Any] = {}
        for uid, node in graph.nodes.items():
            if uid in graph.inputs:
                continue
            self._ops[node.name] = node

    @property
    def graph(self) -> Any:
        return self._graph

    @property
    def plan(self) -> Plan:
        return self._plan

    @property
    def payload_name(self) -> str:
        name = self._graph.name or "payload"
        if not name.replace("_", "a").isalnum() or name[0].isdigit():
            raise UnsupportedGraph(f"graph name {name!r} is not a valid C identifier")
        return name

    @property
    def node_names(self) -> list[str]:
        return list(self._ops)

    def node_operation(self, name: str) -> Any:
        return self._ops[name].operation

    @property
    def default_node(self) -> str:
        """The node whose kernel writes the first graph output."""
        out = self._graph.outputs[0]
        for ln in reversed(self._plan.launches):
            if ln.output == out or ln.output.split(".")[0] == out:
                return ln.node
        return self.node_names[-1]

    def get_scheduler(self, **kwargs: Any) -> HipScheduler:
        return HipScheduler(
            self,
            nodes=kwargs.get("nodes"),
            default_node=kwargs.get("default_node"),
            nodes_schedulers=kwargs.get("nodes_schedulers"),
        )

    def get_compiler(self, **kwargs: Any) -> HipCompiler:
        return HipCompiler(self, **kwargs)
