# SPDX-License-Identifier: BSD-3-Clause
"""Loop-nest view of a node schedule (what `Scheduler.get_loop_nest` returns,
src/xtc/itf/schd/scheduler.py:293-307, src/xtc/schedules/loop_nest.py:78-459).

A LoopNest holds one root node per loop root ("." plus one per split
segment); each records the loop order, tile extents per dimension and the
vectorize/parallelize/unroll annotations, and prints as an indented nest.
"""

from __future__ import annotations

from dataclasses import dataclass, field

__all__ = ["LoopNest", "LoopNestNode", "SplitOrigin"]


@dataclass
class SplitOrigin:
    axis: str
    start: int
    end: int | None


@dataclass
class LoopNestNode:
    root: str
    tiles: dict[str, dict[str, int]] = field(default_factory=dict)
    interchange: list[str] = field(default_factory=list)
    vectorize: list[str] = field(default_factory=list)
    parallelize: list[str] = field(default_factory=list)
    unroll: dict[str, int] = field(default_factory=dict)
    splits: dict[str, dict[str, int]] = field(default_factory=dict)
    split_origin: SplitOrigin | None = None
    children: list["LoopNestNode"] = field(default_factory=list)
    parent: "LoopNestNode | None" = None

    def is_root(self) -> bool:
        return self.parent is None

    def add_child(self, child: "LoopNestNode") -> None:
        child.parent = self
        self.children.append(child)

    def descendants_dfs(self) -> list["LoopNestNode"]:
        out = [self]
        for c in self.children:
            out.extend(c.descendants_dfs())
        return out

    def _extent(self, loop: str, dims: dict[str, int]) -> str:
        for dim, levels in self.tiles.items():
            if loop in levels:
                return f"{levels[loop]}"
        return f"{dims.get(loop, '?')}"

    def pretty_print(self, dims: dict[str, int] | None = None, indent: int = 0) -> str:
        dims = dims or {}
        lines = []
        pad = "  " * indent
        head = f"{pad}loop nest {self.root}"
        if self.split_origin is not None:
            o = self.split_origin
            head += f" ({o.axis}[{o.start}:{'' if o.end is None else o.end}])"
        lines.append(head + ":")
        for depth, loop in enumerate(self.interchange):
            notes = []
            if loop in self.parallelize:
                notes.append("parallel")
            if loop in self.vectorize:
                notes.append("vectorized")
            if loop in self.unroll:
                notes.append(f"unroll={self.unroll[loop]}")
            note = f"  // {', '.join(notes)}" if notes else ""
            lines.append(f"{pad}{'  ' * (depth + 1)}for {loop} ({self._extent(loop, dims)}){note}")
        for c in self.children:
            lines.append(c.pretty_print(dims, indent + 1))
        return "\n".join(lines)


@dataclass
class LoopNest:
    abstract_dims: list[str]
    sizes: dict[str, int] = field(default_factory=dict)
    root_node: LoopNestNode | None = None

    def build_root_node(self, root: str) -> LoopNestNode:
        self.root_node = LoopNestNode(root=root, tiles={d: {} for d in self.abstract_dims})
        return self.root_node

    @property
    def nodes(self) -> list[LoopNestNode]:
        return [] if self.root_node is None else self.root_node.descendants_dfs()

    def __str__(self) -> str:
        return "" if self.root_node is None else self.root_node.pretty_print(self.sizes)
