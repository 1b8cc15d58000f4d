# SPDX-License-Identifier: BSD-3-Clause
"""Schedule -> GEMM kernel template parameters.

A matmul/conv2d launch runs one instance of the MFMA GEMM template
(xtc_amd/csrc/gemm.hpp): a workgroup computes a BM x BN output tile with
WGM x WGN waves, walking K in BK slabs through LDS.  XTC's loop knobs map
onto it as follows (dims of matmul: i, j, k; of conv2d: b, h, w, f, r, s, c,
where (b,h,w) form GEMM-M, f GEMM-N and (r,s,c) GEMM-K):

  * first tile level of the M dims   -> BM (product over b,h,w for conv)
  * first tile level of the N dim    -> BN
  * second tile level of M / N       -> wave tile WM / WN, so WGM = BM/WM,
                                        WGN = BN/WN (absent: library choice)
  * first tile level of the K dims   -> BK (LDS slab depth)
  * parallelize(k)                   -> split-K: K / (first k level) slices,
                                        summed inside the launch; BK is then
                                        the second k level
  * interchange with N's base loop outside M's -> column-major tile raster;
    otherwise tiles are rastered in groups of 8 tile-rows (L2 reuse)
  * unroll of the loop that walks the K slabs (k without split-K, k1 with
    it; c for conv) by S -> pipeline depth S: S slabs in flight through S
    LDS stages.  It must be a depth the kernel is compiled for
    (xtc_hip_matmul_pipeline_depths: 3-6 for the fp32 LDS-DMA BK-16 tiles,
    2-3 for its BK-32 256-wide tiles, 2-4 for 128x128, 3-5 for the bf16
    ping-pong kernel, 2-4 for the skinny bf16 kernel, 2 for the generic
    template and 4 on its 64x64 tiles, which keep three slabs of loads in
    flight in registers); absent, the kernel's default.  Unroll factors of
    the other loops are recorded: the MFMA loop over a slab and the wave's
    sub-tiles are always fully unrolled, and the block and wave tiles are
    spread over waves and lanes
  * vectorize(loop) -> the 16-byte loads and stores of every kernel (4 fp32,
    2 fp64 or 8 bf16 elements): the vectorized loop's extent must be a multiple of
    that width, or the schedule is rejected
  * pack_at(local), buffer_at, fuse_producer_at -> always on in these
    kernels (LDS staging of both operands, register-resident output tile,
    pad folded into the conv loader); recorded, no further effect.
  * split(i or j, segments) of a matmul -> one launch per segment on the
    strided sub-view of A (rows) or B (columns), C and bias, each mapped from
    its own root's tiles and knobs (src/xtc/itf/schd/scheduler.py:65-81); a
    split made inside a segment cuts that segment, its cut points counted
    from the segment's start; a split on the reduction axis, or on a
    conv2d, is rejected: the kernels overwrite C rather than accumulate
    into it.

Tile semantics follow the reference: a tile size is the extent of the
sub-loop (src/xtc/backends/mlir/MlirCompilerPasses.py:414-457).

A request that matches no compiled instance is either rejected with
ScheduleError (policy "strict", the default) or mapped to the nearest
instance in log2 distance (policy "nearest", opt-in); the result records
which happened.  The compiler's default policy "report" maps with "strict"
and turns the error into a module that fails when evaluated (compiler.py).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from functools import lru_cache
from math import prod
from typing import Any

from .scheduler import HipNodeSchedule, ScheduleError

__all__ = ["GemmConfig", "SplitConfig", "map_gemm", "map_node", "gemm_instances", "legal_tiles", "pipeline_depths"]

DEFAULT_GROUP_M = 8


@dataclass(frozen=True)
class GemmConfig:
    dtype: str
    conv: bool
    bm: int
    bn: int
    bk: int
    wgm: int
    wgn: int
    split_k: int = 1
    group_m: int = DEFAULT_GROUP_M
    xcd_remap: int = 1
    exact: bool = True
    source: str = "schedule"  # "schedule" | "nearest" | "default"
    stages: int = 0  # pipeline depth, 0 = the kernel's default

    @property
    def tile(self) -> tuple[int, int, int, int, int]:
        return (self.bm, self.bn, self.bk, self.wgm, self.wgn)

    def describe(self) -> str:
        depth = f" stages={self.stages}" if self.stages else ""
        return (
            f"{'conv' if self.conv else 'gemm'}<{self.dtype}> BMxBNxBK={self.bm}x{self.bn}x{self.bk} "
            f"waves={self.wgm}x{self.wgn} split_k={self.split_k}{depth} group_m={self.group_m} ({self.source})"
        )


@dataclass(frozen=True)
class SplitPiece:
    """One launch of a split matmul: output rows [m0, m0 + M) and columns
    [n0, n0 + N) on the kernel instance `config`."""

    m0: int
    M: int
    n0: int
    N: int
    config: GemmConfig


@dataclass(frozen=True)
class SplitConfig:
    """A matmul whose schedule splits i or j: one launch per piece."""

    pieces: tuple[SplitPiece, ...]

    @property
    def exact(self) -> bool:
        return all(p.config.exact for p in self.pieces)

    def describe(self) -> str:
        return "; ".join(f"rows {p.m0}+{p.M} cols {p.n0}+{p.N}: {p.config.describe()}" for p in self.pieces)


@lru_cache(maxsize=None)
def gemm_instances() -> tuple[tuple[str, bool, tuple[int, int, int, int, int]], ...]:
    """(dtype, conv, tile) of every kernel instance compiled into libxtc_hip."""
    from ...runtimes.hip import capi

    return tuple((i["dtype"], bool(i["conv"]), tuple(i["tile"])) for i in capi.gemm_instances())  # type: ignore[misc]


def legal_tiles(dtype: str, conv: bool) -> list[tuple[int, int, int, int, int]]:
    return [t for d, c, t in gemm_instances() if d == dtype and c == conv]


def _dims_roles(sched: HipNodeSchedule, conv: bool) -> tuple[list[str], list[str], list[str]]:
    d = sched.dims
    if conv:
        return d[0:3], [d[3]], d[4:7]
    return [d[0]], [d[1]], [d[2]]


def _level(sched: HipNodeSchedule, dims: list[str], level: int) -> int | None:
    """Product over `dims` of the tile extent at `level` (a dim with fewer
    levels contributes its innermost extent, an untiled dim 1); None if no
    dim reaches that level."""
    if not any(len(sched.levels(d)) > level for d in dims):
        return None
    out = 1
    for d in dims:
        lv = sched.levels(d)
        out *= lv[min(level, len(lv) - 1)] if lv else 1
    return out


def _default(dtype: str, conv: bool, M: int, N: int, K: int,
             attrs: dict[str, Any] | None = None) -> tuple[tuple[int, int, int, int, int], int]:
    from ...runtimes.hip import capi

    if conv and attrs is not None:
        return default_conv_tile(attrs)
    return capi.default_tile(dtype, conv, M, N, K)


def default_conv_tile(attrs: dict[str, Any]) -> tuple[tuple[int, int, int, int, int], int]:
    """The library's default (tile, split_k) for a conv2d launch: it sees the
    window and strides (xtc_hip_conv2d_default_tile)."""
    from ...runtimes.hip import capi

    _, nb, h, w, c, f, r, s, (sh, sw), (pt, pb, pl, pr) = _attrs_key(attrs, True)
    dt = capi.DTYPE_IDS[attrs["dtype"]]
    cd = capi.Conv2dDesc(dtype=dt, N=nb, H=h, W=w, C=c, F=f, R=r, S=s, stride_h=sh, stride_w=sw, pad_top=pt,
                         pad_bottom=pb, pad_left=pl, pad_right=pr)
    return capi.conv2d_default_tile(cd)


def _attrs_key(attrs: dict[str, Any], conv: bool) -> tuple[Any, ...]:
    if conv:
        return (attrs["dtype"], attrs["NB"], attrs["H"], attrs["W"], attrs["C"], attrs["F"], attrs["R"], attrs["S"],
                tuple(attrs["stride"]), tuple(attrs["pads"]))
    return (attrs["dtype"], attrs["M"], attrs["N"], attrs["K"], bool(attrs.get("trans_a")),
            bool(attrs.get("trans_b")))


@lru_cache(maxsize=4096)
def _depths(key: tuple[Any, ...], conv: bool, tile: tuple[int, int, int, int, int], split_k: int) -> tuple[int, ...]:
    from ...runtimes.hip import capi

    dt = capi.DTYPE_IDS[key[0]]
    if conv:
        _, nb, h, w, c, f, r, s, (sh, sw), (pt, pb, pl, pr) = key
        cd = capi.Conv2dDesc(dtype=dt, N=nb, H=h, W=w, C=c, F=f, R=r, S=s, stride_h=sh, stride_w=sw, pad_top=pt,
                             pad_bottom=pb, pad_left=pl, pad_right=pr, tile=capi.Tile(*tile), split_k=split_k)
        return tuple(capi.conv2d_pipeline_depths(cd))
    _, m, n, k, ta, tb = key
    md = capi.MatmulDesc(dtype=dt, M=m, N=n, K=k, tile=capi.Tile(*tile), split_k=split_k, trans_a=int(ta),
                         trans_b=int(tb))
    return tuple(capi.matmul_pipeline_depths(md))


def pipeline_depths(attrs: dict[str, Any], conv: bool, tile: tuple[int, int, int, int, int], split_k: int) -> list[int]:
    """Pipeline depths of the kernel that runs this launch with `tile` and
    `split_k`, its default first (xtc_hip_*_pipeline_depths)."""
    return list(_depths(_attrs_key(attrs, conv), conv, tuple(tile), int(split_k)))


def _slab_loop(sched: HipNodeSchedule, k_dims: list[str], split: bool) -> str:
    """Name of the loop that walks the K slabs: the loop just outside the
    slab level (the K dim itself without split-K, its first tile level with
    it; for conv, the innermost reduction dim c)."""
    dim = k_dims[-1]
    names = list(sched.tiles.get(dim, {}))
    return names[0] if split and names else dim


def _requested_depth(sched: HipNodeSchedule, k_dims: list[str], split: bool) -> int | None:
    from ...itf.schd import DEFAULT_ROOT
    from .scheduler import loop_name

    return sched.unrolling.get(loop_name(DEFAULT_ROOT, _slab_loop(sched, k_dims, split)))


def _check_vectorize(sched: HipNodeSchedule, dtype: str) -> None:
    from .scheduler import basename

    width = {"float32": 4, "float64": 2}.get(dtype, 8)
    for qualified in sched.vectorization:
        name = basename(qualified)
        extent = None
        if name in sched.dims:
            extent = sched.sizes.get(name)
        else:
            for levels in sched.tiles.values():
                if name in levels:
                    extent = levels[name]
        if extent is not None and extent % width:
            raise ScheduleError(
                f"{sched.node_name}: vectorize({name}): extent {extent} is not a multiple of the {width}-element "
                f"(16-byte) vectors the {dtype} kernels load and store"
            )


def _nearest(req: dict[str, int | None], cands: list[tuple[int, int, int, int, int]]) -> tuple[int, int, int, int, int]:
    def cost(t: tuple[int, int, int, int, int]) -> tuple[float, int]:
        bm, bn, bk, wgm, wgn = t
        have = {"bm": bm, "bn": bn, "bk": bk, "wm": bm // wgm, "wn": bn // wgn}
        c = 0.0
        for k, v in req.items():
            if v:
                c += abs(math.log2(have[k]) - math.log2(v))
        return (c, -(wgm * wgn))

    return min(cands, key=cost)


def map_gemm(
    launch_attrs: dict[str, Any],
    conv: bool,
    sched: HipNodeSchedule | None,
    policy: str = "strict",
) -> GemmConfig:
    dtype = launch_attrs["dtype"]
    M, N, K = launch_attrs["M"], launch_attrs["N"], launch_attrs["K"]
    cands = legal_tiles(dtype, conv)
    if not cands:
        raise ScheduleError(f"no compiled {'conv' if conv else 'matmul'} instance for {dtype}")
    if sched is not None and sched.segments:
        raise ScheduleError(f"{sched.node_name}: split() maps to several launches (map_node)")
    if sched is None or not any(sched.levels(d) for d in sched.dims) and not sched.parallelization:
        tile, split = _default(dtype, conv, M, N, K, launch_attrs)
        return GemmConfig(dtype, conv, *tile, split_k=split, exact=True, source="default")
    m_dims, n_dims, k_dims = _dims_roles(sched, conv)
    bm = _level(sched, m_dims, 0)
    bn = _level(sched, n_dims, 0)
    wm = _level(sched, m_dims, 1)
    wn = _level(sched, n_dims, 1)
    k_parallel = any(sched.is_parallel(d) for d in k_dims)
    split_k = 1
    if k_parallel:
        kslice = _level(sched, k_dims, 0)
        if kslice is None:
            raise ScheduleError(f"{sched.node_name}: parallelize on K needs a K tile (the slice per split)")
        if K % kslice:
            raise ScheduleError(f"{sched.node_name}: K={K} is not a multiple of the split-K slice {kslice}")
        split_k = K // kslice
        bk = _level(sched, k_dims, 1)
    else:
        bk = _level(sched, k_dims, 0)
    order = sched.base_order()
    col_major = bool(order) and order.index(n_dims[0]) < min(order.index(d) for d in m_dims if d in order)
    group_m = (M + (bm or 64) - 1) // (bm or 64) if col_major else DEFAULT_GROUP_M

    dflt_tile, dflt_split = _default(dtype, conv, M, N, K, launch_attrs)
    req_bm = bm or dflt_tile[0]
    req_bn = bn or dflt_tile[1]
    req_bk = bk or dflt_tile[2]
    matches = [
        t
        for t in cands
        if t[0] == req_bm
        and t[1] == req_bn
        and t[2] == req_bk
        and (wm is None or t[0] // t[3] == wm)
        and (wn is None or t[1] // t[4] == wn)
    ]
    _check_vectorize(sched, dtype)
    depth = _requested_depth(sched, k_dims, k_parallel)
    if conv:
        # some conv tiles exist only in the direct kernel, for the shapes it takes
        from ...runtimes.hip import capi

        runnable = []
        for t in matches:
            try:
                pipeline_depths(launch_attrs, conv, t, split_k)
                runnable.append(t)
            except capi.HipError:
                pass
        if matches and not runnable and policy == "strict":
            raise ScheduleError(f"{sched.node_name}: conv tile {matches[0]} has no kernel for this shape "
                                "(it exists only in the direct conv kernel)")
        matches = runnable
    if matches:
        # unspecified wave split: the instance with the most waves
        tile = max(matches, key=lambda t: (t[3] * t[4], t[3]))
        stages = 0
        if depth is not None:
            depths = pipeline_depths(launch_attrs, conv, tile, split_k)
            if depth not in depths:
                if policy == "strict":
                    raise ScheduleError(
                        f"{sched.node_name}: unroll({_slab_loop(sched, k_dims, k_parallel)}: {depth}) asks for a "
                        f"{depth}-slab pipeline; the kernel of tile {tile} runs {depths} (default {depths[0]})"
                    )
                return GemmConfig(dtype, conv, *tile, split_k=split_k, group_m=group_m, exact=False,
                                  source="nearest")
            stages = 0 if depth == depths[0] else depth
        return GemmConfig(dtype, conv, *tile, split_k=split_k, group_m=group_m, exact=True, source="schedule",
                          stages=stages)
    if policy == "strict":
        wave = "" if wm is None and wn is None else f" wave tile {wm}x{wn}"
        raise ScheduleError(
            f"{sched.node_name}: no {dtype} {'conv' if conv else 'matmul'} kernel for block tile "
            f"{req_bm}x{req_bn}x{req_bk}{wave}; compiled tiles (BM,BN,BK,WGM,WGN): "
            f"{sorted(set(cands))[:12]}..."
        )
    tile = _nearest({"bm": req_bm, "bn": req_bn, "bk": req_bk, "wm": wm, "wn": wn}, cands)
    return GemmConfig(dtype, conv, *tile, split_k=split_k, group_m=group_m, exact=False, source="nearest")


def map_node(
    launch_attrs: dict[str, Any],
    conv: bool,
    sched: HipNodeSchedule | None,
    policy: str = "strict",
) -> GemmConfig | SplitConfig:
    """map_gemm, plus split() of a matmul's i or j axis into one launch per
    segment (nested splits of a segment's own root included)."""
    if sched is None or not sched.segments:
        return map_gemm(launch_attrs, conv, sched, policy)
    pieces = _split_pieces(launch_attrs, conv, sched, policy, 0, 0)
    return SplitConfig(tuple(pieces))


def _split_pieces(attrs: dict[str, Any], conv: bool, sched: HipNodeSchedule, policy: str, m0: int,
                  n0: int) -> list[SplitPiece]:
    if not sched.segments:
        return [SplitPiece(m0, attrs["M"], n0, attrs["N"], map_gemm(attrs, conv, sched, policy))]
    where = f"{sched.node_name}: split()"
    if conv:
        raise ScheduleError(f"{where} has no HIP mapping for conv2d (one launch covers the whole tensor)")
    dims = {seg.dim for seg in sched.segments}
    if len(dims) != 1:
        raise ScheduleError(f"{where} of several axes at one root ({sorted(dims)}) has no HIP mapping")
    (dim,) = dims
    m_dim, n_dim, k_dim = sched.dims[0], sched.dims[1], sched.dims[2]
    if dim == k_dim:
        raise ScheduleError(f"{where} on the reduction axis {dim!r} has no HIP mapping: the kernels overwrite C "
                            "rather than accumulate into it")
    if sched.levels(dim):
        # the split then cuts every tile of the axis, so each segment is a
        # strided set of rows or columns rather than one sub-matrix
        raise ScheduleError(f"{where} of {dim!r} inside its tiles ({sched.levels(dim)}) has no HIP mapping: only a "
                            "split of the untiled axis becomes one launch per segment")
    extent = attrs["M"] if dim == m_dim else attrs["N"]
    segs = list(sched.segments)
    if segs[0].start != 0:
        raise ScheduleError(f"{where}: the first segment of {dim!r} starts at {segs[0].start}, not 0")
    out: list[SplitPiece] = []
    for seg in segs:
        if not 0 <= seg.start < seg.end <= extent:
            raise ScheduleError(f"{where}: segment [{seg.start}, {seg.end}) of {dim!r} is empty or outside "
                                f"[0, {extent})")
        sub = dict(attrs)
        if dim == m_dim:
            sub["M"] = seg.end - seg.start
            out += _split_pieces(sub, conv, seg.schedule, policy, m0 + seg.start, n0)
        else:
            sub["N"] = seg.end - seg.start
            out += _split_pieces(sub, conv, seg.schedule, policy, m0, n0 + seg.start)
    return out


def schedule_is_legal(sched: HipNodeSchedule, launch_attrs: dict[str, Any], conv: bool) -> bool:
    """True if `sched` maps exactly onto a compiled instance."""
    try:
        return map_node(launch_attrs, conv, sched, policy="strict").exact
    except ScheduleError:
        return False


def gemm_flops(attrs: dict[str, Any]) -> int:
    return 2 * prod((attrs["M"], attrs["N"], attrs["K"]))
