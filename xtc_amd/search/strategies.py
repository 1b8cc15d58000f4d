# SPDX-License-Identifier: BSD-3-Clause
"""Schedule search spaces (src/xtc/search/strategies.py:42-1283).

A strategy turns a point of an integer sample space into Scheduler calls.
The spaces, their enumeration order, filters and seeded random draws follow
the reference so that a seed gives the same samples (the transcripts of
tests/filecheck/search/test_*.py are replayed by tests/test_strategies.py):

  * PRT schemes ("OO", "PRP", "PPRPRP", "PPWRPRP", "PFPWRPRP" ...): a
    sequence of items, P = parallel axes, R = reduction axes, T = all axes,
    O = first P axis then R axes then remaining P axes, W = write buffer at
    the preceding axis, F = producer fusion at the preceding axis.  Each axis
    occurrence after the first is a new tile level; a sample holds the tile
    factors of every axis (outer to inner), then one boolean per W and F.
    The innermost tile of the last P axis is vectorised, the trailing tiled
    axes are unrolled, and with threads > 1 the leading base P axes are
    parallelised.
  * P1: one tile level with a permutation of the inner tiles (matmul).
  * GOTO: the Goto/BLIS blocking of matmul.

Extension: `tile_hip`, whose samples are exactly the GEMM kernel instances
compiled into libxtc_hip (block tile, wave tile, K slab, split-K), so every
sample runs on the GPU; and a `sample_filter` keyword on every strategy
(the HIP explorer uses it to keep only samples that map exactly onto a
kernel instance).
"""

from __future__ import annotations

import itertools
from collections.abc import Callable, Iterator, Mapping, Sequence
from dataclasses import dataclass, field
from math import prod
from typing import Any

import numpy as np

from ..itf.search import Sample, Strategy, VecSample
from ..utils.algorithms import sample_uniques
from ..utils.math import factors_enumeration, factors_to_sizes

__all__ = ["Strategies", "BaseStrategy", "BaseStrategyPRTScheme", "Strategy_HIP"]


def _node_of(graph: Any, node: str | None) -> Any:
    if node is None:
        return graph.outputs_nodes[0]
    for n in graph.nodes.values():
        if n.name == node or n.uid == node:
            return n
    raise ValueError(f"no node {node!r} in graph")


def _operation_of(graph: Any, node: str | None) -> Any:
    return _node_of(graph, node).operation


class BaseStrategy(Strategy):
    """Common machinery: product enumeration, unroll filter, seeded draws."""

    def __init__(
        self,
        graph: Any,
        sample_names: list[str] | None = None,
        vec_size: int = 16,
        max_unroll: int = 256,
        threads: int = 1,
        max_parallelize: int = -1,
        **kwargs: Any,
    ) -> None:
        self._graph = graph
        self._sample_names = sample_names
        self._vec_size = vec_size
        self._max_unroll = max_unroll
        self._threads = threads
        self._max_parallelize = max_parallelize
        self._op = _operation_of(graph, kwargs.get("node"))
        self._stats: dict[str, int] = {}
        self._parallelize = threads > 1
        self._vectorize = vec_size > 1
        self._unroll = max_unroll != 0
        self._arch_vreg_num = kwargs.get("vreg_num", 32)
        self._arch_l1_size = kwargs.get("l1_size", 32 * 1024)
        self._arch_l2_size = kwargs.get("l2_size", 1024 * 1024)
        self._sample_filter: Callable[[list[int]], bool] | None = kwargs.get("sample_filter")

    # ---- Strategy interface
    @property
    def graph(self) -> Any:
        return self._graph

    @property
    def sample_names(self) -> list[str]:
        assert self._sample_names is not None
        return self._sample_names

    @property
    def stats(self) -> Mapping[str, int]:
        return self._stats

    def generate(self, scheduler: Any, sample: Sample) -> None:
        self._generate(scheduler, list(sample))

    def exhaustive(self) -> Iterator[VecSample]:
        samples = self._filter(self._iter_product(self._independents(), stat="all"))
        return self._user_filter(samples)

    def default_schedule(self, opt_level: int = 2) -> VecSample:
        if opt_level < 0:
            raise ValueError("opt_level must be >= 0")
        return self._default_schedule(opt_level)

    def sample(self, num: int, seed: int | None = 0) -> Iterator[VecSample]:
        if num <= 0 or (seed is not None and seed < 0):
            raise ValueError("num must be > 0 and seed >= 0")
        rng = np.random.default_rng(seed=seed)
        inds = self._independents()

        def draw(n: int) -> Iterator[tuple[int, ...]]:
            cands = self._user_filter(self._filter(iter(self._sample_product(inds, n, rng))))
            return (tuple(s) for s in cands)

        return iter([list(s) for s in sample_uniques(draw, num)[:num]])  # type: ignore[arg-type]

    def dict_to_sample(self, sample: dict[str, Any]) -> Sample:
        return list(sample.values())

    def sample_to_dict(self, sample: Sample) -> dict[str, int]:
        return dict(zip(self.sample_names, sample))

    # ---- helpers
    def _user_filter(self, samples: Iterator[VecSample]) -> Iterator[VecSample]:
        if self._sample_filter is None:
            yield from samples
            return
        for x in samples:
            if self._sample_filter(list(x)):
                yield x

    def _constant_sizes(self) -> Mapping[str, int]:
        return {a: int(v) for a, v in self._op.dims.items() if isinstance(v, int)}

    def _iter_product(self, args: Sequence[Sequence[Sequence[int]]], stat: str | None = None) -> Iterator[VecSample]:
        if stat:
            self._stats[stat] = 0
        for combo in itertools.product(*args):
            if stat:
                self._stats[stat] += 1
            yield list(itertools.chain(*combo))

    def _vector_axis(self) -> str | None:
        p = list(self._op.dims_kind("P"))
        return p[-1] if p else None

    def _filter_unroll(
        self, indexes: list[int], v_index: int | None, samples: Iterator[VecSample], stat: str | None = None
    ) -> Iterator[VecSample]:
        """Keeps samples whose inner unrolled volume, divided by the vector
        width actually used, is at most max_unroll."""
        if stat:
            self._stats[stat] = 0
        if self._max_unroll < 0:
            yield from samples
            return
        for x in samples:
            volume = prod(x[i] for i in indexes)
            vec = min(x[v_index] if v_index is not None else 1, self._vec_size)
            if volume / vec <= self._max_unroll:
                if stat:
                    self._stats[stat] += 1
                yield x

    @staticmethod
    def _sample_product(inds: list[list[list[int]]], num: int, rng: np.random.Generator) -> list[VecSample]:
        # one rng.integers call per independent variable, in order: the
        # reference's draw sequence
        cols = [np.array(var, dtype="int")[rng.integers(len(var), size=num)] for var in inds]
        return np.hstack(cols).tolist()

    # ---- to implement
    def _generate(self, sch: Any, in_x: list[int]) -> None:
        raise NotImplementedError

    def _default_schedule(self, opt_level: int) -> list[int]:
        raise NotImplementedError

    def _independents(self) -> list[list[list[int]]]:
        raise NotImplementedError

    def _filter(self, samples: Iterator[VecSample]) -> Iterator[VecSample]:
        raise NotImplementedError


class BaseStrategyPRTScheme(BaseStrategy):
    """Tiling sequences built from P/R/T/O items with W/F markers."""

    def __init__(self, graph: Any, scheme: str, **kwargs: Any) -> None:
        super().__init__(graph, [], **kwargs)
        self._scheme = scheme
        self._axes = list(self._op.dims)
        self._sizes = self._constant_sizes()
        self._p_axes = list(self._op.dims_kind("P"))
        self._r_axes = list(self._op.dims_kind("R"))
        self._build_order()
        self._tiles_idx = self._build_tiles_index()
        self._x_size = sum(levels - 1 for levels in self._tiles_levels.values())
        self._parallel = self._build_parallel()
        self._unrolled = self._build_unrolled()
        self._vectorized = self._build_vectorized()
        self._sample_names = (
            [f"x{i}" for i in range(self._x_size)]
            + [f"w{i}" for i in range(len(self._w_axes))]
            + [f"f{i}" for i in range(len(self._f_axes))]
        )
        self._out_dtype = self._op.outputs_types[0].dtype
        assert len(self._vectorized) <= 1

    def _build_order(self) -> None:
        levels = {axis: 0 for axis in self._axes}
        self._order: list[str] = []
        self._base_axis: dict[str, str] = {}
        self._item_map: dict[int, list[str]] = {}
        self._w_axes: list[str] = []
        self._f_axes: list[str] = []
        previous = ""
        for idx, item in enumerate(self._scheme):
            if item == "P":
                axes = self._p_axes
            elif item == "R":
                axes = self._r_axes
            elif item == "T":
                axes = self._axes
            elif item == "O":
                axes = [*self._p_axes[:1], *self._r_axes, *self._p_axes[1:]]
            elif item in "WF":
                if not previous:
                    raise ValueError(f"scheme {self._scheme}: {item} needs a preceding axis")
                (self._w_axes if item == "W" else self._f_axes).append(previous)
                axes = []
            else:
                raise ValueError(f"unknown scheme item {item!r}")
            names = []
            for axis in axes:
                name = axis if levels[axis] == 0 else f"{axis}{levels[axis]}"
                levels[axis] += 1
                self._base_axis[name] = axis
                names.append(name)
            self._order.extend(names)
            self._item_map[idx] = names
            previous = names[-1] if names else ""
        self._tiles_levels = levels

    def _build_tiles_index(self) -> dict[str, int]:
        out: dict[str, int] = {}
        idx = 0
        for axis in self._axes:
            if self._tiles_levels[axis] < 1:
                raise ValueError(f"no tile level specified for axis: {axis}")
            out[axis] = idx
            for level in range(self._tiles_levels[axis] - 1):
                out[f"{axis}{level + 1}"] = idx
                idx += 1
        return out

    def _build_unrolled(self) -> list[str]:
        if not self._unroll:
            return []
        s = self._scheme
        if s[-1:] in ("T", "O") or s[-2:] in ("PR", "RP"):
            limit = len(self._axes)
        elif s[-1:] == "P":
            limit = len(self._p_axes)
        elif s[-1:] == "R":
            limit = len(self._r_axes)
        else:
            limit = 0
        out = []
        for idx, axis in enumerate(reversed(self._order)):
            if idx >= limit or axis == self._base_axis[axis]:
                break
            out.append(axis)
        return out

    def _build_vectorized(self) -> list[str]:
        if not self._vectorize or not self._order:
            return []
        inner = self._order[-1]
        if inner == self._base_axis[inner] or self._base_axis[inner] != self._vector_axis():
            return []
        return [inner]

    def _build_parallel(self) -> list[str]:
        if not self._parallelize:
            return []
        out = []
        for idx, axis in enumerate(self._order):
            if self._max_parallelize >= 0 and idx >= self._max_parallelize:
                break
            if self._base_axis[axis] != axis or axis not in self._p_axes:
                break
            out.append(axis)
        return out

    def _inner_items_indexes(self, item_idx: int) -> list[int]:
        if item_idx < 0:
            item_idx += len(self._scheme)
        return [self._tiles_idx[a] for i in range(item_idx, len(self._scheme)) for a in self._item_map[i]]

    def _filter_vectorized(self, samples: Iterator[VecSample], stat: str | None = None) -> Iterator[VecSample]:
        """Keeps samples whose vectorised tile is at least vec_size."""
        if stat:
            self._stats[stat] = 0
        vaxis = self._vectorized[0] if self._vectorized else ""
        if not vaxis or self._sizes[self._base_axis[vaxis]] <= self._vec_size:
            yield from samples
            return
        vidx = self._tiles_idx[vaxis]
        for x in samples:
            if x[vidx] >= self._vec_size:
                if stat:
                    self._stats[stat] += 1
                yield x

    def _filter_volume(
        self, samples: Iterator[VecSample], inner_items: int, limit: float, stat: str | None
    ) -> Iterator[VecSample]:
        if stat:
            self._stats[stat] = 0
        idx = self._inner_items_indexes(-inner_items)
        for x in samples:
            if prod(x[i] for i in idx) <= limit:
                if stat:
                    self._stats[stat] += 1
                yield x

    def _filter_reg_num(self, samples: Iterator[VecSample], inner_items: int, stat: str | None = None):  # type: ignore[no-untyped-def]
        return self._filter_volume(samples, inner_items, self._vec_size * self._arch_vreg_num, stat)

    def _filter_l1_size(self, samples: Iterator[VecSample], inner_items: int, stat: str | None = None):  # type: ignore[no-untyped-def]
        return self._filter_volume(samples, inner_items, self._arch_l1_size / self._elt_size(), stat)

    def _filter_l2_size(self, samples: Iterator[VecSample], inner_items: int, stat: str | None = None):  # type: ignore[no-untyped-def]
        return self._filter_volume(samples, inner_items, self._arch_l2_size / self._elt_size(), stat)

    def _elt_size(self) -> int:
        from ..utils.bf16 import itemsize

        return itemsize(self._out_dtype)

    def _independents(self) -> list[list[list[int]]]:
        tiles = [factors_enumeration(self._sizes[a], lv - 1) for a, lv in self._tiles_levels.items()]
        return tiles + [[[0], [1]]] * len(self._w_axes) + [[[0], [1]]] * len(self._f_axes)

    def _filter(self, samples: Iterator[VecSample]) -> Iterator[VecSample]:
        idx = [self._tiles_idx[a] for a in self._unrolled]
        vidx = [self._tiles_idx[a] for a in self._vectorized]
        return self._filter_unroll(idx, vidx[0] if vidx else None, samples, stat="filtered")

    def _generate(self, sch: Any, in_x: list[int]) -> None:
        n_w, n_f = len(self._w_axes), len(self._f_axes)
        for axis in self._axes:
            idx = self._tiles_idx[axis]
            sizes = factors_to_sizes(in_x[idx : idx + self._tiles_levels[axis] - 1])
            sch.tile(axis, {f"{axis}{lvl + 1}": s for lvl, s in enumerate(sizes)})
        sch.interchange(self._order)
        sch.parallelize(self._parallel)
        sch.vectorize(self._vectorized)
        sch.unroll({a: in_x[self._tiles_idx[a]] for a in self._unrolled})
        flags = in_x[len(in_x) - (n_w + n_f) :] if n_w + n_f else []
        for axis, flag in zip(self._w_axes, flags[:n_w]):
            if flag:
                sch.buffer_at(axis)
        for axis, flag in zip(self._f_axes, flags[n_w:]):
            if flag:
                sch.fuse_producer_at(axis, 0)

    def _max_factor(self, axis: str, bound: int) -> int:
        return [f[0] for f in factors_enumeration(self._sizes[self._base_axis[axis]], 1) if f[0] <= bound][-1]

    def _default_schedule(self, opt_level: int) -> list[int]:
        def tiled(v_unroll: int, p_unroll: int, r_unroll: int) -> list[int] | None:
            vaxes = self._vectorized[:1]
            paxes = [a for a in self._unrolled if self._base_axis[a] in self._p_axes][:2]
            raxes = [a for a in self._unrolled if self._base_axis[a] in self._r_axes][:1]
            vt = {a: self._max_factor(a, max(p_unroll, v_unroll)) for a in vaxes}
            pt = {a: self._max_factor(a, p_unroll) for a in paxes if a not in vt}
            rt = {a: self._max_factor(a, r_unroll) for a in raxes}
            tiles = {**pt, **rt, **vt}
            for a, t in tiles.items():
                size = self._sizes[self._base_axis[a]]
                if not (t > 0 and size >= t and size % t == 0):
                    return None
            out = [1] * self._x_size
            for a, t in tiles.items():
                out[self._tiles_idx[a]] = t
            return out

        sched = [1] * self._x_size
        w = [0] * len(self._w_axes)
        if opt_level >= 2:
            if w:
                w[-1] = 1
            sched = tiled(self._vec_size, 2, 1) or sched
        if opt_level >= 3:
            w = [1] * len(self._w_axes)
            sched = tiled(self._vec_size, 4, 16) or sched
        return sched + w


def _scheme_class(name: str, scheme: str, filters: str = "") -> type[BaseStrategyPRTScheme]:
    """A PRT strategy class for `scheme`; filters "v" adds the vector-width
    filter, "vr" the vector, register, L1 and L2 volume filters."""

    def __init__(self: BaseStrategyPRTScheme, graph: Any, **kwargs: Any) -> None:
        BaseStrategyPRTScheme.__init__(self, graph, scheme=scheme, **kwargs)

    def _filter(self: BaseStrategyPRTScheme, samples: Iterator[VecSample]) -> Iterator[VecSample]:
        samples = BaseStrategyPRTScheme._filter(self, samples)
        if "v" in filters:
            samples = self._filter_vectorized(samples, "filtered_vec")
        if "r" in filters:
            samples = self._filter_reg_num(samples, 1, "filtered_reg")
            samples = self._filter_l1_size(samples, 2, "filtered_l1")
            samples = self._filter_l2_size(samples, 3, "filtered_l2")
        return samples

    body: dict[str, Any] = {"__init__": __init__, "__doc__": f"Tiling scheme {scheme}{' (' + filters + ')' if filters else ''}."}
    if filters:
        body["_filter"] = _filter
    return type(name, (BaseStrategyPRTScheme,), body)


Strategy_OO = _scheme_class("Strategy_OO", "OO")
Strategy_PRP = _scheme_class("Strategy_PRP", "PRP")
Strategy_PPRPRP = _scheme_class("Strategy_PPRPRP", "PPRPRP")
Strategy_PPRPRPv = _scheme_class("Strategy_PPRPRPv", "PPRPRP", "v")
Strategy_PPRPRPvr = _scheme_class("Strategy_PPRPRPvr", "PPRPRP", "vr")
Strategy_PPWRPRP = _scheme_class("Strategy_PPWRPRP", "PPWRPRP")
Strategy_PPWRPRPv = _scheme_class("Strategy_PPWRPRPv", "PPWRPRP", "v")
Strategy_PPWRPRPvr = _scheme_class("Strategy_PPWRPRPvr", "PPWRPRP", "vr")
Strategy_PFPWRPRP = _scheme_class("Strategy_PFPWRPRP", "PFPWRPRP")
Strategy_PFPWRPRPv = _scheme_class("Strategy_PFPWRPRPv", "PFPWRPRP", "v")
Strategy_PFPWRPRPvr = _scheme_class("Strategy_PFPWRPRPvr", "PFPWRPRP", "vr")


class Strategy_P1(BaseStrategy):
    """One tile level on i, j, k plus a permutation of the inner tiles
    (matmul only).  Sample: [ti, tj, tk, order]."""

    def __init__(self, graph: Any, **kwargs: Any) -> None:
        super().__init__(graph, ["ti", "tj", "tk", "order"], **kwargs)
        if tuple(self._op.dims) != ("i", "j", "k"):
            raise ValueError("tile_p1 applies to matmul (dims i, j, k)")
        self._perms = list(itertools.permutations(["i1", "j1", "k1"]))
        self._vector_perms = [i for i, p in enumerate(self._perms) if p[-1] == "j1"]

    def _generate(self, sch: Any, in_x: list[int]) -> None:
        ti, tj, tk, order = in_x[:4]
        perm = list(self._perms[order])
        tiles = {"i1": ti, "j1": tj, "k1": tk}
        axes = ["i", "j", "k"] + perm
        parallel = [a for a in axes[:2] if a in ("i", "j")] if self._threads > 1 else []
        sch.tile("i", {"i1": ti})
        sch.tile("j", {"j1": tj})
        sch.tile("k", {"k1": tk})
        sch.interchange(axes)
        sch.parallelize(parallel)
        sch.vectorize(["j1"] if axes[-1] == "j1" else [])
        sch.unroll({a: tiles[a] for a in reversed(perm)})

    def _filter_unroll(self, indexes, v_index, samples, stat=None):  # type: ignore[no-untyped-def,override]
        if stat:
            self._stats[stat] = 0
        if self._max_unroll < 0:
            yield from samples
            return
        for x in samples:
            vsize = x[v_index] if v_index is not None and x[-1] in self._vector_perms else 1
            if prod(x[i] for i in indexes) / min(vsize, self._vec_size) <= self._max_unroll:
                if stat:
                    self._stats[stat] += 1
                yield x

    def _independents(self) -> list[list[list[int]]]:
        i, j, k = self._constant_sizes().values()
        return [factors_enumeration(i, 1), factors_enumeration(j, 1), factors_enumeration(k, 1),
                [[x] for x in range(len(self._perms))]]

    def _filter(self, samples: Iterator[VecSample]) -> Iterator[VecSample]:
        return self._filter_unroll([0, 1, 2], 1, samples, stat="filtered")

    def _default_schedule(self, opt_level: int) -> list[int]:
        i, j, k = self._constant_sizes().values()
        sched = [1, 1, 1, 1 if opt_level >= 2 else 0]
        if opt_level >= 3:
            it, jt, kt = 2, self._vec_size, 1
            if all(n >= t and n % t == 0 for n, t in ((i, it), (j, jt), (k, kt))):
                sched = [it, jt, kt, 1]
        return sched


class Strategy_P1v(Strategy_P1):
    """tile_p1 restricted to vectorised permutations with tj >= vec_size."""

    def _filter(self, samples: Iterator[VecSample]) -> Iterator[VecSample]:
        for x in super()._filter(samples):
            if x[-1] in self._vector_perms and x[1] >= self._vec_size:
                yield x


class Strategy_GOTO(BaseStrategy):
    """Goto blocking of matmul: sample [iL2, iR, jL3, jR, kL1, unroll_k,
    pack_B, pack_A]; order j, k, i, j1, i1, k1, i2, j2 with j2 vectorised."""

    def __init__(self, graph: Any, **kwargs: Any) -> None:
        super().__init__(graph, ["iL2", "iR", "jL3", "jR", "kL1", "unroll_k", "pack_B", "pack_A"], **kwargs)

    def _generate(self, sch: Any, in_x: list[int]) -> None:
        iL2, iR, jL3, jR, kL1, unroll_k, pack_b, pack_a = in_x[:8]
        if pack_b:
            sch.pack_at("k", 1, pad=True)
        if pack_a:
            sch.pack_at("i", 0, pad=True)
        sch.tile("i", {"i1": iR * iL2, "i2": iR})
        sch.tile("j", {"j1": jR * jL3, "j2": jR})
        sch.tile("k", {"k1": kL1})
        sch.interchange(["j", "k", "i", "j1", "i1", "k1", "i2", "j2"])
        sch.parallelize(["j"] if self._threads > 1 else [])
        sch.vectorize(["j2"])
        sch.unroll({"i2": iR, "k1": unroll_k})

    def _independents(self) -> list[list[list[int]]]:
        i, j, k = self._constant_sizes().values()
        b = [[0], [1]]
        return [factors_enumeration(i, 2), factors_enumeration(j, 2), factors_enumeration(k, 2), b, b]

    def _filter(self, samples: Iterator[VecSample]) -> Iterator[VecSample]:
        return self._filter_unroll([1, 3, 5], 3, samples, stat="filtered")

    def _default_schedule(self, opt_level: int) -> list[int]:
        i, j, k = self._constant_sizes().values()
        sched = [1, 1, 1, 1, 1, 0, 0, 0]
        if opt_level >= 3:
            it, jt, kt = 2, self._vec_size, 1
            if all(n >= t and n % t == 0 for n, t in ((i, it), (j, jt), (k, kt))):
                sched = [1, it, 1, jt, kt, 2, 1, 1]
        return sched


class Strategy_GOTO_R(Strategy_GOTO):
    """GOTO with small register tiles and k unrolls, 1 < outer blocks < 128."""

    def _filter(self, samples: Iterator[VecSample]) -> Iterator[VecSample]:
        reg = self._vec_size * self._arch_vreg_num
        for x in super()._filter(samples):
            io, ii, jo, ji, _, uk = x[:6]
            if ii * ji < reg // 2 and ii < 4 and uk < 4 and 128 > io > 1 and 128 > jo > 1:
                yield x


class Strategy_HIP(BaseStrategy):
    """GPU space: every compiled GEMM kernel instance of the graph's dtype.

    Sample [bm, wm, bn, wn, bk, split_k, stages] (sizes, not factors); the
    mapping of xtc_amd/backends/hip/mapping.py read backwards:
      * matmul (i, j, k): tile(i, {i1: bm, i2: wm}), tile(j, {j1: bn, j2: wn}),
        and on k either {k1: bk} or, with split_k > 1, {k1: K/split_k, k2: bk}
        plus parallelize(k);
      * conv2d (b, h, w, f, r, s, c): the implicit-GEMM rows are b*h*w, so
        the block and wave heights are split over h and w (w takes up to 8),
        f carries the block and wave widths and c the slab depth, {c1: bk};
        with split_k > 1, {c1: K/split_k, c2: bk} plus parallelize(c), for
        the splits whose slice K/split_k is at most C;
      * stages: unroll of the slab loop (k, or k1 under split-K; c or c1 for conv)
        by the pipeline depth, one of the depths the tile's kernel is
        compiled for on this shape (the default first).

    Its default sample is the library's own choice for the shape, and the
    iterative search evaluates it in its first batch (starts_from_default).
    """

    starts_from_default = True

    def __init__(self, graph: Any, **kwargs: Any) -> None:
        super().__init__(graph, ["bm", "wm", "bn", "wn", "bk", "split_k", "stages"], **kwargs)
        dims = list(self._op.dims)
        kinds = [d for d in dims if d in self._op.dims_kind("R")]
        dtype = str(self._op.inputs_types[0].dtype)
        from ..backends.hip.mapping import legal_tiles

        if len(dims) == 3 and kinds == [dims[2]]:
            self._conv = False
            self._M, self._N, self._K = (int(self._op.dims[d]) for d in dims)
        elif len(dims) == 7 and kinds == dims[4:]:
            self._conv = True
            size = {d: int(self._op.dims[d]) for d in dims}
            self._M = size[dims[0]] * size[dims[1]] * size[dims[2]]
            self._N = size[dims[3]]
            self._K = size[dims[4]] * size[dims[5]] * size[dims[6]]
            self._C = size[dims[6]]
        else:
            raise ValueError("tile_hip applies to matmul (P, P, R) and conv2d (P, P, P, P, R, R, R) operations")
        self._dims = dims
        self._attrs = self._launch_attrs(graph, _node_of(graph, kwargs.get("node")).name)
        tiles = sorted(set(legal_tiles(dtype, self._conv)))
        self._tiles = [t for t in tiles if t[0] <= max(16, self._M) * 2 and t[1] <= max(16, self._N) * 2]
        splits = (1, 2, 4, 8, 16, 32)
        if self._conv:
            self._tiles = [t for t in self._tiles if t[2] <= self._C]
            # a split's K slice is a tile of c (c1 = K / split), so it is at
            # most C: splits of at least R*S, each slice within one tap's channels
            self._splits = [s for s in splits
                            if s == 1 or (self._K % s == 0 and 64 <= self._K // s <= self._C)]
        else:
            self._splits = [s for s in splits if s == 1 or (self._K % s == 0 and self._K // s >= 64)]
        self._dtype = dtype

    @staticmethod
    def _launch_attrs(graph: Any, node: str) -> dict[str, Any]:
        """The HIP lowering's attributes of node `node`'s kernel launch."""
        from ..backends.hip import Backend

        for ln in Backend(graph).plan.launches:
            if ln.kind in ("matmul", "conv2d") and ln.node == node:
                return ln.attrs
        raise ValueError(f"tile_hip: node {node} has no matmul/conv2d kernel launch")

    def _depths(self, tile: tuple[int, int, int, int, int], split: int) -> list[int]:
        from ..backends.hip.mapping import pipeline_depths

        return pipeline_depths(self._attrs, self._conv, tile, split)

    def _points(self) -> list[list[int]]:
        from ..runtimes.hip import capi

        out = []
        for tile in self._tiles:
            bm, bn, bk, wgm, wgn = tile
            for s in self._splits:
                if s > 1 and (self._K // s) % bk:
                    continue
                try:
                    depths = self._depths(tile, s)
                except capi.HipError:  # a tile with no kernel for this shape
                    continue
                for depth in depths:
                    out.append([bm, bm // wgm, bn, bn // wgn, bk, s, depth])
        return out

    def _independents(self) -> list[list[list[int]]]:
        return [self._points()]

    def _filter(self, samples: Iterator[VecSample]) -> Iterator[VecSample]:
        self._stats["filtered"] = 0
        for x in samples:
            self._stats["filtered"] += 1
            yield x

    def _generate(self, sch: Any, in_x: list[int]) -> None:
        bm, wm, bn, wn, bk, split = in_x[:6]
        depth = in_x[6] if len(in_x) > 6 else None
        if self._conv:
            b, h, w, f, r, s, c = self._dims
            # the block's pixels as h x w tiles: w the largest divisor up to 8
            # (8 for the power-of-two tiles and 112 = 14 x 8, 7 for 98 = 14 x 7)
            w1 = max(d for d in range(1, min(bm, 8) + 1) if bm % d == 0)
            w2 = max(d for d in range(1, min(wm, 8) + 1) if wm % d == 0)
            sch.tile(b, {f"{b}1": 1, f"{b}2": 1})
            sch.tile(h, {f"{h}1": bm // w1, f"{h}2": wm // w2})
            sch.tile(w, {f"{w}1": w1, f"{w}2": w2})
            sch.tile(f, {f"{f}1": bn, f"{f}2": wn})
            if split > 1:
                # split-K: parallel slices of K / split reduction elements
                sch.tile(c, {f"{c}1": self._K // split, f"{c}2": bk})
                sch.parallelize([b, h, w, f, c])
                slab = f"{c}1"
            else:
                sch.tile(c, {f"{c}1": bk})
                sch.parallelize([b, h, w, f])
                slab = c
            if depth is not None:
                sch.unroll({slab: depth})  # the slab loop: `depth` slabs in flight
            return
        i, j, k = self._dims
        sch.tile(i, {f"{i}1": bm, f"{i}2": wm})
        sch.tile(j, {f"{j}1": bn, f"{j}2": wn})
        if split > 1:
            sch.tile(k, {f"{k}1": self._K // split, f"{k}2": bk})
            sch.interchange([i, j, k, f"{i}1", f"{j}1", f"{k}1", f"{k}2", f"{i}2", f"{j}2"])
            sch.parallelize([i, j, k])
            slab_loop = f"{k}1"
        else:
            sch.tile(k, {f"{k}1": bk})
            sch.interchange([i, j, k, f"{i}1", f"{j}1", f"{k}1", f"{i}2", f"{j}2"])
            sch.parallelize([i, j])
            slab_loop = k
        if depth is not None:
            sch.unroll({slab_loop: depth})  # `depth` slabs in flight through LDS

    def _default_schedule(self, opt_level: int) -> list[int]:
        from ..runtimes.hip import capi

        if self._conv:
            from ..backends.hip.mapping import default_conv_tile

            tile, split = default_conv_tile(self._attrs)
        else:
            tile, split = capi.default_tile(self._dtype, self._conv, self._M, self._N, self._K)
        bm, bn, bk, wgm, wgn = tile
        split = max(1, split)
        if split not in self._splits:
            # a library split this space cannot name (a conv slice wider than C)
            split = max(s for s in self._splits if s <= split and (s == 1 or (self._K // s) % bk == 0))
        return [bm, bm // wgm, bn, bn // wgn, bk, split, self._depths(tile, split)[0]]


@dataclass
class StrategyRegistration:
    cls: type[Strategy]
    default_args: list[Any] = field(default_factory=list)
    default_kwargs: dict[str, Any] = field(default_factory=dict)


class Strategies:
    """Name -> strategy class registry (src/xtc/search/strategies.py:1190-1283)."""

    _map: dict[str, StrategyRegistration] = {}
    _aliases: dict[str, str] = {}

    @classmethod
    def register(
        cls,
        name: str,
        strategy_cls: type[Strategy],
        *,
        default_args: Sequence[Any] | None = None,
        default_kwargs: Mapping[str, Any] | None = None,
        aliases: Sequence[str] = (),
    ) -> None:
        cls._map[name] = StrategyRegistration(strategy_cls, list(default_args or []), dict(default_kwargs or {}))
        for alias in aliases:
            cls.register_alias(alias, name)

    @classmethod
    def register_alias(cls, alias: str, name: str) -> None:
        cls._aliases[alias] = name

    @classmethod
    def names(cls, *, include_aliases: bool = False) -> list[str]:
        return list(cls._map) + (list(cls._aliases) if include_aliases else [])

    @classmethod
    def resolve_name(cls, name: str) -> str:
        """Follows aliases to a registered name; an alias loop is an error."""
        chain = [name]
        while chain[-1] in cls._aliases:
            target = cls._aliases[chain[-1]]
            if target in chain:
                raise ValueError(f"aliases loop without reaching a strategy: {' -> '.join(chain + [target])}")
            chain.append(target)
        return chain[-1]

    @classmethod
    def registration(cls, name: str) -> StrategyRegistration:
        resolved = cls.resolve_name(name)
        reg = cls._map.get(resolved)
        if reg is None:
            raise ValueError(f"no strategy is registered as {resolved!r} (known: {', '.join(sorted(cls._map))})")
        return reg

    @classmethod
    def from_name(cls, name: str) -> type[Strategy]:
        return cls.registration(name).cls

    @classmethod
    def create(cls, name: str, graph: Any, *args: Any, **kwargs: Any) -> Strategy:
        reg = cls.registration(name)
        return reg.cls(graph, *reg.default_args, *args, **{**reg.default_kwargs, **kwargs})


Strategies.register("tile_p1", Strategy_P1)
Strategies.register("tile_p1_v", Strategy_P1v)
Strategies.register("tile_oo", Strategy_OO, aliases=("tile1d", "tile3d"))
Strategies.register("tile_prp", Strategy_PRP)
Strategies.register("tile_pprprp", Strategy_PPRPRP, aliases=("tile7d",))
Strategies.register("tile_pprprp_v", Strategy_PPRPRPv, aliases=("tile7dv",))
Strategies.register("tile_pprprp_vr", Strategy_PPRPRPvr, aliases=("tile7dvr",))
Strategies.register("tile_ppwrprp", Strategy_PPWRPRP, aliases=("tile8d",))
Strategies.register("tile_ppwrprp_v", Strategy_PPWRPRPv, aliases=("tile8dv",))
Strategies.register("tile_ppwrprp_vr", Strategy_PPWRPRPvr, aliases=("tile8dvr",))
Strategies.register("tile_pfpwrprp", Strategy_PFPWRPRP, aliases=("tile9d",))
Strategies.register("tile_pfpwrprp_v", Strategy_PFPWRPRPv, aliases=("tile9dv",))
Strategies.register("tile_pfpwrprp_vr", Strategy_PFPWRPRPvr, aliases=("tile9dvr",))
Strategies.register("tile_goto", Strategy_GOTO)
Strategies.register("tile_goto_r", Strategy_GOTO_R)
Strategies.register("prt", BaseStrategyPRTScheme)
Strategies.register("tile_hip", Strategy_HIP, aliases=("tile_gpu",))
Strategies.register_alias("tile4d", "tile_p1")
Strategies.register_alias("tile4dv", "tile_p1_v")


def __getattr__(name: str) -> Any:
    # the descript strategies live in descript_strategy.py (which imports
    # this module); they are also reachable here, as in the reference
    if name in ("Strategy_Descript", "Strategy_Descript_Explore"):
        from . import descript_strategy

        return getattr(descript_strategy, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
