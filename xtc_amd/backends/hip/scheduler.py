# SPDX-License-Identifier: BSD-3-Clause
"""Scheduler of the HIP backend.

Same surface and recording semantics as the reference's MLIR scheduler
(src/xtc/backends/mlir/MlirScheduler.py:21-288,
src/xtc/backends/mlir/MlirNodeScheduler.py:17-232): one node scheduler per
operator node, transformations recorded under loop names "<root>/<name>",
the default interchange being the base dims then tile levels, and
`get_scheduler(default_node=..., nodes=...)` selecting the target node.
Where the MLIR backend defaults to the last node, this backend defaults to
the node whose kernel produces the graph output (a relu fused into a matmul
epilogue is not a kernel of its own).

The recorded schedule is turned into kernel template parameters by
`mapping.py` at compile time.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, field
from pprint import pformat
from typing import TYPE_CHECKING, Any

from ...itf.schd import DEFAULT_ROOT, Schedule, Scheduler
from ...schedules.loop_nest import LoopNest, LoopNestNode, SplitOrigin

if TYPE_CHECKING:
    from .backend import HipBackend

__all__ = ["HipScheduler", "HipSchedule", "HipNodeSchedule", "HipSegment", "ScheduleError"]

_SEP = "/"


class ScheduleError(ValueError):
    """A transformation the HIP backend cannot express."""


def loop_name(root: str, name: str) -> str:
    return f"{root}{_SEP}{name}"


def basename(name: str) -> str:
    return name.split(_SEP)[-1]


def parent_of(name: str) -> str:
    """The root a qualified loop or segment name lives in."""
    return name.rsplit(_SEP, 1)[0]


@dataclass(frozen=True)
class HipSegment:
    """One segment of a split() axis: [start, end) of `dim`, with the
    schedule its root carries (re-rooted so its loops read as top-level)."""

    dim: str
    start: int
    end: int
    schedule: "HipNodeSchedule"


@dataclass(frozen=True)
class HipNodeSchedule:
    node_name: str
    dims: list[str]
    sizes: dict[str, int]
    splits: dict[str, dict[str, int]]
    tiles: dict[str, dict[str, int]]
    permutation: dict[str, list[str]]
    vectorization: list[str]
    parallelization: list[str]
    unrolling: dict[str, int]
    packed_buffers: dict[str, list[int]]
    buffers: list[str]
    fused: list[tuple[str, int]]
    # segments of the splits at the root, in axis order (empty without split)
    segments: tuple[HipSegment, ...] = ()

    def levels(self, dim: str) -> list[int]:
        """Tile extents of `dim`, outer to inner (empty if untiled)."""
        return list(self.tiles.get(dim, {}).values())

    def base_order(self, root: str = DEFAULT_ROOT) -> list[str]:
        """Base dims in the order they appear in the root's permutation."""
        perm = [basename(p) for p in self.permutation.get(root, [])]
        return [p for p in perm if p in self.dims]

    def is_parallel(self, dim: str, root: str = DEFAULT_ROOT) -> bool:
        return loop_name(root, dim) in self.parallelization

    def __str__(self) -> str:
        return pformat(asdict(self), sort_dicts=False)


class _NodeScheduler:
    def __init__(self, node_name: str, dims: list[str], sizes: dict[str, int]) -> None:
        self.node_name = node_name
        self.dims = list(dims)
        self.sizes = dict(sizes)
        # (root, dim) -> qualified segment name -> start
        self.splits: dict[tuple[str, str], dict[str, int]] = {}
        self.tiles: dict[str, dict[str, int]] = {d: {} for d in self.dims}
        self.permutation: dict[str, list[str]] = {}
        self.vectorization: list[str] = []
        self.parallelization: list[str] = []
        self.unrolling: dict[str, int] = {}
        self.packed_buffers: dict[str, list[int]] = {}
        self.buffers: list[str] = []
        self.fused: list[tuple[str, int]] = []
        self.buffer_at: dict[str, str | None] = {}
        self.pack_at: dict[str, tuple[int, str | None, bool]] = {}

    def _dim_of(self, name: str) -> str:
        if name in self.dims:
            return name
        for d, lv in self.tiles.items():
            if name in lv:
                return d
        raise ScheduleError(f"{self.node_name}: unknown loop {name!r}")

    def default_interchange(self, root: str) -> list[str]:
        order = [loop_name(root, d) for d in self.dims]
        depth = max((len(v) for v in self.tiles.values()), default=0)
        for lvl in range(depth):
            for d in self.dims:
                names = list(self.tiles.get(d, {}))
                if lvl < len(names):
                    order.append(loop_name(root, names[lvl]))
        return order

    def freeze(self) -> HipNodeSchedule:
        if not self.permutation:
            self.permutation[DEFAULT_ROOT] = self.default_interchange(DEFAULT_ROOT)
        return self._frozen_view(DEFAULT_ROOT, dict(self.sizes))

    def _frozen_view(self, root: str, sizes: dict[str, int]) -> HipNodeSchedule:
        """The schedule of the loops under `root`, renamed as if `root` were
        the top level; the segments of the splits made at `root` carry the
        views of their own roots."""

        def under(name: str) -> bool:
            return parent_of(name) == root

        def rerooted(name: str) -> str:
            return loop_name(DEFAULT_ROOT, basename(name))

        splits = {d: v for (r, d), v in self.splits.items() if r == root and v}
        segments: list[HipSegment] = []
        for dim, segs in splits.items():
            names = list(segs)
            for idx, seg in enumerate(names):
                start = segs[seg]
                end = segs[names[idx + 1]] if idx + 1 < len(names) else sizes[dim]
                sub_sizes = dict(sizes)
                sub_sizes[dim] = end - start
                segments.append(HipSegment(dim, start, end, self._frozen_view(seg, sub_sizes)))
        perm = self.permutation.get(root)
        if perm is None:
            perm = self.default_interchange(root) if root == DEFAULT_ROOT else []
        return HipNodeSchedule(
            node_name=self.node_name,
            dims=list(self.dims),
            sizes=dict(sizes),
            splits={k: {basename(n): v for n, v in seg.items()} for k, seg in splits.items()},
            tiles={k: {basename(n): s for n, s in v.items() if under(n)} for k, v in self.tiles.items()
                   if k in self.dims},
            permutation={DEFAULT_ROOT: [rerooted(p) for p in perm]},
            vectorization=[rerooted(v) for v in self.vectorization if under(v)],
            parallelization=[rerooted(v) for v in self.parallelization if under(v)],
            unrolling={rerooted(k): v for k, v in self.unrolling.items() if under(k)},
            packed_buffers={rerooted(k): list(v) for k, v in self.packed_buffers.items() if under(k)},
            buffers=[rerooted(b) for b in self.buffers if under(b)],
            fused=[(rerooted(a), i) for a, i in self.fused if under(a)],
            segments=tuple(segments),
        )


class HipScheduler(Scheduler):
    def __init__(
        self,
        backend: "HipBackend",
        nodes: list[str] | None = None,
        default_node: str | None = None,
        nodes_schedulers: dict[str, "_NodeScheduler"] | None = None,
    ) -> None:
        self._backend = backend
        if nodes_schedulers is not None:
            # shares the node states of another scheduler
            # (MlirScheduler's nodes_schedulers, MlirScheduler.py:22-45)
            self._schedulers = nodes_schedulers
        else:
            names = nodes if nodes is not None else backend.node_names
            self._schedulers = {}
            for name in names:
                op = backend.node_operation(name)
                dims = list(op.dims)
                self._schedulers[name] = _NodeScheduler(name, dims, {d: int(v) for d, v in op.dims.items()})
        target = default_node if default_node is not None else backend.default_node
        if target not in self._schedulers:
            raise ScheduleError(f"no schedulable node named {target!r} (nodes: {list(self._schedulers)})")
        self._current = self._schedulers[target]

    @property
    def backend(self) -> "HipBackend":
        return self._backend

    @property
    def node_name(self) -> str:
        return self._current.node_name

    @property
    def nodes_schedulers(self) -> dict[str, "_NodeScheduler"]:
        return self._schedulers

    def for_node(self, name: str) -> "HipScheduler":
        """A scheduler over the same node states whose primitives apply to
        node `name`: schedules several nodes of one graph."""
        return HipScheduler(self._backend, default_node=name, nodes_schedulers=self._schedulers)

    def schedule(self) -> "HipSchedule":
        return HipSchedule(self, [s.freeze() for s in self._schedulers.values()])

    def set_dims(self, dims: list[str]) -> None:
        cur = self._current
        if len(dims) != len(cur.dims):
            raise ScheduleError(f"set_dims: {len(dims)} names for {len(cur.dims)} dims")
        cur.sizes = {new: cur.sizes[old] for new, old in zip(dims, cur.dims)}
        cur.dims = list(dims)
        cur.tiles = {d: {} for d in cur.dims}

    def split(self, dim: str, segments: dict[str, int], root: str = DEFAULT_ROOT) -> None:
        cur = self._current
        cur._dim_of(dim)
        renamed = {loop_name(root, k): int(v) for k, v in segments.items()}
        cur.splits[(root, dim)] = renamed
        for seg in renamed:
            cur.tiles.setdefault(seg, {})

    def tile(self, dim: str, tiles: dict[str, int], root: str = DEFAULT_ROOT) -> None:
        cur = self._current
        if dim not in cur.tiles:
            raise ScheduleError(f"{cur.node_name}: cannot tile unknown dim {dim!r} (dims: {cur.dims})")
        for name, size in tiles.items():
            if int(size) <= 0:
                raise ScheduleError(f"{cur.node_name}: tile {name}={size} must be positive")
            cur.tiles[dim][loop_name(root, name)] = int(size)

    def interchange(self, permutation: list[str], root: str = DEFAULT_ROOT) -> None:
        self._current.permutation[root] = [loop_name(root, a) for a in permutation]

    def vectorize(self, axes: list[str], root: str = DEFAULT_ROOT) -> None:
        self._current.vectorization += [loop_name(root, a) for a in axes]

    def parallelize(self, axes: list[str], root: str = DEFAULT_ROOT) -> None:
        self._current.parallelization = [loop_name(root, a) for a in axes]

    def unroll(self, unrolls: dict[str, int], root: str = DEFAULT_ROOT) -> None:
        for name, factor in unrolls.items():
            self._current.unrolling[loop_name(root, name)] = int(factor)

    def buffer_at(self, axis: str, mtype: str | None = None, root: str = DEFAULT_ROOT) -> None:
        if mtype not in (None, "global", "local", "shared"):
            raise ScheduleError(f"buffer_at: unknown memory type {mtype!r}")
        self._current.buffers.append(loop_name(root, axis))
        self._current.buffer_at[loop_name(root, axis)] = mtype

    def pack_at(
        self,
        axis: str,
        input_idx: int,
        mtype: str | None = None,
        pad: bool = False,
        root: str = DEFAULT_ROOT,
    ) -> None:
        if mtype not in (None, "global", "local", "shared"):
            raise ScheduleError(f"pack_at: unknown memory type {mtype!r}")
        self._current.packed_buffers.setdefault(loop_name(root, axis), []).append(int(input_idx))
        self._current.pack_at[loop_name(root, axis)] = (int(input_idx), mtype, pad)

    def fuse_producer_at(self, axis: str, input_idx: int, root: str = DEFAULT_ROOT) -> None:
        self._current._dim_of(axis)  # raises on an unknown loop
        self._current.fused.append((loop_name(root, axis), int(input_idx)))

    def _single_gpu(self, what: str) -> None:
        raise ScheduleError(
            f"{what}: the HIP backend runs one kernel on one GPU per process; "
            "multi-device meshes are not supported"
        )

    def define_memory_mesh(self, axes: dict[str, int]) -> None:
        self._single_gpu("define_memory_mesh")

    def define_processor_mesh(self, axes: dict[str, int]) -> None:
        self._single_gpu("define_processor_mesh")

    def distribute(self, axis: str, processor_axis: str, root: str = DEFAULT_ROOT) -> None:
        self._single_gpu("distribute")

    def distributed_buffer_at(
        self, axis: str, input_idx: int, memory_axes: list[str], root: str = DEFAULT_ROOT
    ) -> None:
        self._single_gpu("distributed_buffer_at")

    def get_loop_nest(self) -> LoopNest:
        """The current node's schedule as a LoopNest: the root "." and one
        child per split segment, each with its own tiles, loop order and
        annotations, loop names without their root prefix."""
        cur = self._current
        sched = cur.freeze()
        nest = LoopNest(abstract_dims=list(sched.dims))
        root = nest.build_root_node(DEFAULT_ROOT)
        segments: dict[str, tuple[str, SplitOrigin]] = {}  # qualified segment -> (dim, origin)
        for (_, dim), segs in cur.splits.items():
            names = list(segs)
            for idx, seg in enumerate(names):
                end = segs[names[idx + 1]] if idx + 1 < len(names) else None
                segments[seg] = (dim, SplitOrigin(axis=dim, start=segs[seg], end=end))

        def fill(node: LoopNestNode, root_name: str) -> None:
            perm = cur.permutation.get(root_name)
            if perm is None:
                perm = cur.default_interchange(root_name) if root_name == DEFAULT_ROOT else []
            members = set(perm)
            node.interchange = [basename(p) for p in perm]
            for dim, levels in cur.tiles.items():
                if dim not in sched.dims:
                    continue
                for name, size in levels.items():
                    if parent_of(name) == root_name:
                        node.tiles.setdefault(dim, {})[basename(name)] = size
            for seg, (dim, _) in segments.items():
                if parent_of(seg) == root_name:
                    node.splits.setdefault(dim, {})[basename(seg)] = cur.splits[(parent_of(seg), dim)][seg]
            node.vectorize = [basename(v) for v in cur.vectorization if v in members]
            node.parallelize = [basename(v) for v in cur.parallelization if v in members]
            node.unroll = {basename(k): v for k, v in cur.unrolling.items() if k in members}
            node.buffer_at = {basename(k): v for k, v in cur.buffer_at.items() if k in members}
            node.pack_at = {basename(k): v for k, v in cur.pack_at.items() if k in members}
            for seg, (dim, origin) in segments.items():
                if parent_of(seg) == root_name:
                    child = LoopNestNode(root=seg, tiles={d: {} for d in sched.dims}, split_origin=origin)
                    node.add_child(child)
                    fill(child, seg)

        fill(root, DEFAULT_ROOT)
        return nest


class HipSchedule(Schedule):
    def __init__(self, scheduler: HipScheduler, nodes_schedules: list[HipNodeSchedule]) -> None:
        self._scheduler = scheduler
        self._nodes = {s.node_name: s for s in nodes_schedules}

    @property
    def scheduler(self) -> HipScheduler:
        return self._scheduler

    @property
    def schedule_impl(self) -> list[HipNodeSchedule]:
        return list(self._nodes.values())

    def node(self, name: str) -> HipNodeSchedule | None:
        return self._nodes.get(name)

    def __str__(self) -> str:
        return str([str(s) for s in self._nodes.values()])
