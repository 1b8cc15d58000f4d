# SPDX-License-Identifier: BSD-3-Clause
"""Loop-nest description of a node schedule: what `Scheduler.get_loop_nest`
returns and what the descript interpreter builds
(src/xtc/itf/schd/scheduler.py:293-307, src/xtc/schedules/loop_nest.py:78-459).

A LoopNestNode holds the loops of one root (the operation, or one segment of
a split): tiles per axis (tile loop -> size), splits per axis (segment loop
-> start), the loop order and the loop annotations.  Split segments are
child nodes.  `pretty_print` renders the nest one loop per line
(`loop X`, `tile(X, n)`, `split(X, start, end)`, `// annotations`, `...` for
the body) and `LoopNest.check` rejects inconsistent nests.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

from .exceptions import ScheduleValidationError

__all__ = ["SplitOrigin", "LoopNestNode", "LoopInfo", "LoopNest"]


@dataclass
class SplitOrigin:
    """The axis segment [start, end) a split child covers (end None: to the end)."""

    axis: str
    start: Any
    end: Any


@dataclass
class LoopNestNode:
    root: str
    tiles: dict[str, dict[str, Any]] = field(default_factory=dict)
    splits: dict[str, dict[str, Any]] = field(default_factory=dict)
    interchange: list[str] = field(default_factory=list)
    vectorize: list[str] = field(default_factory=list)
    parallelize: list[str] = field(default_factory=list)
    unroll: dict[str, Any] = field(default_factory=dict)
    buffer_at: dict[str, str | None] = field(default_factory=dict)
    pack_at: dict[str, tuple[Any, str | None, Any]] = field(default_factory=dict)
    split_origin: SplitOrigin | None = None
    children: list["LoopNestNode"] = field(default_factory=list)
    parent: "LoopNestNode | None" = field(default=None, repr=False)

    @property
    def is_root(self) -> bool:
        return self.parent is None

    def add_child(self, child: "LoopNestNode") -> None:
        child.parent = self
        self.children.append(child)

    def ancestors(self) -> list["LoopNestNode"]:
        out, cur = [], self.parent
        while cur is not None:
            out.append(cur)
            cur = cur.parent
        return out

    def descendants_dfs(self) -> list["LoopNestNode"]:
        out: list[LoopNestNode] = []
        for c in self.children:
            out.append(c)
            out.extend(c.descendants_dfs())
        return out

    # ------------------------------------------------------------ printing
    def _notes(self, loop: str) -> str:
        notes = []
        if loop in self.parallelize:
            notes.append("parallelized")
        if loop in self.vectorize:
            notes.append("vectorized")
        if loop in self.unroll:
            notes.append(f"unroll({self.unroll[loop]})")
        if loop in self.buffer_at:
            mtype = self.buffer_at[loop]
            notes.append("buffer" if mtype is None else f"buffer({mtype})")
        if loop in self.pack_at:
            idx, mtype, pad = self.pack_at[loop]
            parts = [str(idx)] + ([mtype] if mtype is not None else []) + (["pad"] if pad else [])
            notes.append(f"pack({', '.join(parts)})")
        return ("  // " + ", ".join(notes)) if notes else ""

    def own_tiles(self) -> dict[str, tuple[str, Any]]:
        """Tile loop -> (axis, size) of this node (tile names restart in
        each split segment, so they are looked up per node)."""
        return {name: (axis, size) for axis, loops in self.tiles.items() for name, size in loops.items()}

    def pretty_print(self, indent: int = 0) -> str:
        info = LoopInfo.build_from_node(self)
        info.tiles_info.update(self.own_tiles())
        child_of: dict[str, LoopNestNode] = {}
        for child in self.children:
            o = child.split_origin
            if o is not None:
                for name, start in self.splits.get(o.axis, {}).items():
                    if start == o.start:
                        child_of[name] = child
                        break
        lines: list[str] = []
        depth = indent
        printed_splits: set[str] = set()
        for loop in self.interchange:
            if loop in printed_splits:
                continue
            if loop in info.splits_info:
                axis = info.splits_info[loop][0]
                # every segment of the axis at the same depth, in loop order
                segs = [l for l in self.interchange if l in info.splits_info and info.splits_info[l][0] == axis]
                printed_splits.update(segs)
                for seg in segs:
                    _, start, end = info.splits_info[seg]
                    lines.append(" " * depth + f"split({axis}, {start}, {'...' if end is None else end})" + self._notes(seg))
                    if seg in child_of:
                        lines.append(child_of[seg].pretty_print(depth + 2))
                    else:
                        lines.append(" " * (depth + 2) + "...")
                continue
            if loop in info.tiles_info:
                axis, size = info.tiles_info[loop]
                text = f"tile({axis}, {size})"
            else:
                text = f"loop {loop.split('/')[-1]}"
            lines.append(" " * depth + text + self._notes(loop))
            depth += 2
        if not printed_splits:
            lines.append(" " * depth + "...")
        return "\n".join(lines)


@dataclass
class LoopInfo:
    """Loop name -> axis tables of a node and its descendants."""

    dims: list[str]
    tiles_info: dict[str, tuple[str, Any]] = field(default_factory=dict)
    splits_info: dict[str, tuple[str, Any, Any]] = field(default_factory=dict)

    @property
    def loops_to_axis(self) -> dict[str, str]:
        out = {d: d for d in self.dims}
        out.update({n: a for n, (a, _) in self.tiles_info.items()})
        out.update({n: a for n, (a, _, _) in self.splits_info.items()})
        return out

    @property
    def splits_to_sizes(self) -> dict[str, int]:
        return {n: e - s for n, (_, s, e) in self.splits_info.items()
                if isinstance(s, int) and isinstance(e, int)}

    @staticmethod
    def build_from_node(node: LoopNestNode) -> "LoopInfo":
        tiles: dict[str, tuple[str, Any]] = {}
        splits: dict[str, tuple[str, Any, Any]] = {}
        dims: dict[str, None] = {}

        def visit(n: LoopNestNode) -> None:
            for axis, loops in n.tiles.items():
                for name, size in loops.items():
                    tiles[name] = (axis, size)
            for axis, segs in n.splits.items():
                ordered = list(segs.items())
                if all(isinstance(s, int) for _, s in ordered):
                    ordered.sort(key=lambda kv: kv[1])
                for i, (name, start) in enumerate(ordered):
                    splits[name] = (axis, start, ordered[i + 1][1] if i + 1 < len(ordered) else None)
            refined = set(tiles) | set(splits)
            for loop in n.interchange:
                if loop not in refined:
                    dims[loop] = None
            for axis, _ in tiles.values():
                dims[axis] = None
            for axis, _, _ in splits.values():
                dims[axis] = None
            for c in n.children:
                visit(c)

        visit(node)
        return LoopInfo(list(dims), tiles, splits)


@dataclass
class LoopNest:
    abstract_dims: list[str]
    root_node: LoopNestNode | None = None
    constraints: list[str] = field(default_factory=list)

    @property
    def nodes(self) -> list[LoopNestNode]:
        return [] if self.root_node is None else [self.root_node] + self.root_node.descendants_dfs()

    def build_root_node(self, root: str) -> LoopNestNode:
        self.root_node = LoopNestNode(root=root, tiles={a: {} for a in self.abstract_dims})
        return self.root_node

    def __str__(self) -> str:
        return "" if self.root_node is None else self.root_node.pretty_print()

    # ---------------------------------------------------------- validation
    def check(self) -> None:
        """Raises ScheduleValidationError for the inconsistencies the
        reference rejects (loop_nest.py:347-459): a declared axis no loop
        uses, a non-vectorized loop inside a vectorized one, a tile placed
        before its axis, and an inner tile or segment larger than the loop
        around it (or an unroll larger than its loop)."""
        if self.root_node is None:
            raise ScheduleValidationError("empty loop nest")
        info = LoopInfo.build_from_node(self.root_node)
        for dim in self.abstract_dims:
            if dim not in info.dims:
                raise ScheduleValidationError(f"{dim} defined but never used")
        for node in self.nodes:
            vect = False
            for loop in node.interchange:
                if loop in node.vectorize:
                    vect = True
                elif vect:
                    raise ScheduleValidationError(f"Inner loop {loop} isn't vectorized but an outer one is.")
        seen: set[str] = set()
        for node in self.nodes:
            own = node.own_tiles()
            for loop in node.interchange:
                if loop in own:
                    axis, size = own[loop]
                    if axis not in seen:
                        raise ScheduleValidationError(f"`{axis}#{size}`: {axis} has not been materialized yet.")
                elif loop in info.splits_info:
                    seen.add(info.splits_info[loop][0])
                else:
                    seen.add(loop)
        split_size: dict[str, int | None] = {}
        for node in self.nodes:
            tile_size: dict[str, int] = {}
            o = node.split_origin
            if o is not None:
                split_size[o.axis] = o.end - o.start if isinstance(o.start, int) and isinstance(o.end, int) else None
            own = node.own_tiles()
            for loop in node.interchange:
                axis = own[loop][0] if loop in own else info.loops_to_axis.get(loop, loop)
                current = tile_size.get(axis, split_size.get(axis))
                size = None
                if loop in own:
                    size = own[loop][1]
                    tile_size[axis] = size
                elif loop in info.splits_to_sizes:
                    size = info.splits_to_sizes[loop]
                    split_size[axis] = size
                if size is not None and current is not None and size > current:
                    raise ScheduleValidationError(f"Inner loop {loop} on axis {axis} must be smaller than outer loop.")
                if loop in node.unroll and size and size < node.unroll[loop]:
                    raise ScheduleValidationError(
                        f'`{{"unroll" = {node.unroll[loop]}}}`: unroll factor should be smaller than {size}.'
                    )
