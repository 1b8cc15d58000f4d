# SPDX-License-Identifier: BSD-3-Clause
"""Dataflow graph of the DSL (src/xtc/graphs/xtc/graph.py, utils.py).

The printed form and the YAML dictionary layout are interfaces: the
reference's golden tests and `--graph-file` inputs use them.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from pathlib import Path
from typing import Any

import yaml

from ...itf.data import Tensor, TensorType
from ...itf.graph import Graph
from .data import XTCTensor, XTCTensorType
from .node import XTCNode
from .operators import XTCOperator

__all__ = ["XTCGraph", "topological_order"]


def topological_order(nodes: Sequence[XTCNode], seeds: Sequence[XTCNode] | None = None) -> list[XTCNode]:
    """Post-order walk from `seeds` (default: nodes no other node uses),
    restricted to `nodes`; predecessors come before their users."""
    members = {n.uid: n for n in nodes}
    if len(members) != len(nodes):
        raise ValueError("duplicate nodes in graph")
    if seeds is None:
        used = {p for n in nodes for p in n.preds}
        seeds = [n for n in nodes if n.uid not in used]
    order: list[XTCNode] = []
    seen: set[str] = set()

    def visit(node: XTCNode) -> None:
        stack: list[tuple[XTCNode, bool]] = [(node, False)]
        while stack:
            cur, done = stack.pop()
            if done:
                order.append(cur)
                continue
            if cur.uid in seen or cur.uid not in members:
                continue
            seen.add(cur.uid)
            stack.append((cur, True))
            for pred in reversed(cur.preds_nodes):
                if pred.uid not in seen:
                    stack.append((pred, False))

    for s in seeds:
        visit(s)
    return order


class XTCGraph(Graph):
    def __init__(self, name: str | None = None) -> None:
        self._name = name
        self._nodes: list[XTCNode] = []
        self._inputs: list[XTCNode] = []
        self._outputs: list[XTCNode] = []
        self._inputs_types: list[XTCTensorType] | None = None
        self._outputs_types: list[XTCTensorType] | None = None

    @property
    def name(self) -> str:
        return self._name or ""

    @property
    def nodes(self) -> Mapping[str, XTCNode]:
        return {n.uid: n for n in self._nodes}

    @property
    def inputs(self) -> Sequence[str]:
        return [n.uid for n in self._inputs]

    @property
    def outputs(self) -> Sequence[str]:
        return [n.uid for n in self._outputs]

    @property
    def inputs_nodes(self) -> Sequence[XTCNode]:
        return self._inputs

    @property
    def outputs_nodes(self) -> Sequence[XTCNode]:
        return self._outputs

    @property
    def inputs_types(self) -> Sequence[XTCTensorType] | None:
        return self._inputs_types

    @property
    def outputs_types(self) -> Sequence[XTCTensorType] | None:
        return self._outputs_types

    def add_nodes(self, nodes: Sequence[XTCNode]) -> None:
        self._nodes.extend(nodes)

    def set_inputs(self, inputs: Sequence[XTCNode]) -> None:
        self._inputs = list(inputs)

    def set_outputs(self, outputs: Sequence[XTCNode]) -> None:
        self._outputs = list(outputs)

    def sorted_nodes(self) -> list[XTCNode]:
        """Nodes in a topological order."""
        return topological_order(self._nodes)

    def forward_types(self, inputs_types: Sequence[TensorType]) -> Sequence[XTCTensorType]:
        if len(inputs_types) != len(self._inputs):
            raise ValueError(f"forward types inputs size mismatch: {len(inputs_types)} != {len(self._inputs)}")
        self._inputs_types = list(inputs_types)  # type: ignore[arg-type]
        env: dict[str, Any] = dict(zip(self.inputs, self._inputs_types))
        for node in self.sorted_nodes():
            if node.uid in env and node.is_tensor():
                node.forward_types([])
                continue
            env[node.uid] = node.forward_types([env[u] for u in node.inputs])[0]
        self._outputs_types = [env[u] for u in self.outputs]
        return self._outputs_types

    def forward(self, inputs: Sequence[Tensor]) -> Sequence[XTCTensor]:
        if len(inputs) != len(self._inputs):
            raise ValueError(f"forward inputs size mismatch: {len(inputs)} != {len(self._inputs)}")
        env: dict[str, Any] = dict(zip(self.inputs, inputs))
        for node in self.sorted_nodes():
            if node.uid in env and node.is_tensor():
                continue
            env[node.uid] = node.forward([env[u] for u in node.inputs])[0]
        return [env[u] for u in self.outputs]

    def ops_dtype(self) -> str:
        """dtype of the first node's operation (graph.py:201-205)."""
        return self._nodes[0].operation.ops_dtype if self._nodes else "float32"

    def ops_count(self) -> int:
        """Sum of ops counts of nodes whose dtype is ops_dtype (graph.py:190-199)."""
        dtype = self.ops_dtype()
        return sum(n.operation.ops_count for n in self._nodes if n.operation.ops_dtype == dtype)

    def __str__(self) -> str:
        lines = ["graph:"]
        if self.name:
            lines.append(f"  name: {self._name}")
        for title, nodes, types in (
            ("inputs", self._inputs, self._inputs_types),
            ("outputs", self._outputs, self._outputs_types),
        ):
            if not nodes:
                lines.append(f"  {title}: []")
                continue
            lines.append(f"  {title}:")
            for idx, node in enumerate(nodes):
                suffix = f" : {types[idx]}" if types else ""
                lines.append(f"  - {node.uid}{suffix}")
        if self._nodes:
            lines.append("  nodes:")
            for node in topological_order(self._nodes, self._outputs):
                lines.append(f"  - {node.uid}: {node}")
        else:
            lines.append("  nodes: {}")
        return "\n".join(lines) + "\n"

    def to_dict(self) -> dict[str, Any]:
        """Serialisable form with uids renumbered from the first input."""
        data: dict[str, Any] = {}
        if self._name:
            data["name"] = self._name
        data["inputs"] = [{"uid": n.uid, "expr": n.expr.to_dict()} for n in self._inputs]
        data["outputs"] = [{"uid": n.uid} for n in self._outputs]
        data["nodes"] = [n.to_dict() for n in self._nodes if not (n.is_tensor() and n in self._inputs)]
        data["ops_version"] = XTCOperator.version_string()
        base = int(data["inputs"][0]["uid"][1:]) if data["inputs"] else 0

        def renumber(obj: Any) -> Any:
            if isinstance(obj, dict):
                return {k: renumber(v) for k, v in obj.items()}
            if isinstance(obj, list):
                return [renumber(v) for v in obj]
            if isinstance(obj, str) and obj.startswith("%") and obj[1:].isdigit():
                return f"%{int(obj[1:]) - base}"
            return obj

        return renumber(data)  # type: ignore[no-any-return]

    def dumps(self) -> str:
        return yaml.safe_dump(self.to_dict(), sort_keys=False)

    def dump(self, file_name: str | Path) -> None:
        path = Path(file_name)
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(self.dumps())
