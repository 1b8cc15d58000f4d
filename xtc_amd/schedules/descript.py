# SPDX-License-Identifier: BSD-3-Clause
"""descript: declarative schedule specifications (src/xtc/schedules/descript.py:36-542,
src/xtc/schedules/parsing.py:1-352).

A specification is a dict whose keys, in loop order, are
  * "i"            a loop over axis i (annotations in the value dict),
  * "i#32"         a tile of axis i of size 32 (a string size is a parameter),
  * "i[0:128]"     a segment of axis i (the value is the nested schedule of
    "i[128:]"      the segment; "i[:n:]" is a segment of size n),
and whose values hold the annotations
  unroll (True | factor | parameter), vectorize, parallelize (True | parameter),
  buffer (memory type or "default"), pack ((input, memory type, pad)),
  partial / full (tile semantics of a parameter size).
The same can be written in YAML ("i": "parallelize", "j": {"size": 16, ...}).

The flow: parse (dict -> AST) -> interpret (AST -> LoopNest, with parameters
and constraints) -> instantiate (parameters from a sample) -> check ->
apply to a Scheduler (split / tile / interchange / vectorize / parallelize /
unroll / buffer_at / pack_at per node, children after their parent).  The
HIP backend then maps the resulting tiles onto kernel template parameters.
"""

from __future__ import annotations

import ast
import copy
import functools
import re
from dataclasses import dataclass, field
from typing import Any

import yaml

from .exceptions import ScheduleInterpretError, ScheduleParseError, ScheduleValidationError
from .loop_nest import LoopNest, LoopNestNode, SplitOrigin

__all__ = [
    "Annotations",
    "AxisDecl",
    "TileDecl",
    "SplitDecl",
    "ScheduleSpec",
    "ScheduleParser",
    "YAMLParser",
    "ScheduleInterpreter",
    "Descript",
    "descript_scheduler",
    "instantiate",
    "check_constraints",
]

Literal = int | str


def _literal(text: str) -> Literal:
    return int(text) if text.lstrip("-").isdigit() else text


# ------------------------------------------------------------------ AST


@dataclass(frozen=True)
class Annotations:
    unroll: Literal | None = None  # None with unroll_specified: the whole loop
    unroll_specified: bool = False
    vectorize: bool | str = False
    parallelize: bool | str = False
    buffer: str | None = None
    buffer_specified: bool = False
    pack: tuple[Literal, str | None, bool | str] | None = None
    pack_specified: bool = False
    partial: bool = False
    full: bool = False


@dataclass(frozen=True)
class AxisDecl:
    axis: str
    annotations: Annotations


@dataclass(frozen=True)
class TileDecl:
    axis: str
    size: Literal
    annotations: Annotations

    def __str__(self) -> str:
        return f"{self.axis}#{self.size}"


@dataclass(frozen=True)
class SplitDecl:
    axis: str
    start: Literal | None
    end: Literal | None
    size: Literal | None
    body: "ScheduleSpec"

    def __str__(self) -> str:
        if self.size is not None:
            return f"{self.axis}[:{self.size}:]"
        return f"{self.axis}[{'' if self.start is None else self.start}:{'' if self.end is None else self.end}]"


@dataclass(frozen=True)
class ScheduleSpec:
    items: tuple[AxisDecl | TileDecl | SplitDecl, ...]


# ------------------------------------------------------------------ parsing


class ScheduleParser:
    """dict -> ScheduleSpec."""

    _SEGMENT = re.compile(r"^(.*)\[(-\w+|\w*)?:(-\w+|\w*)?\]$")
    _SIZED_SEGMENT = re.compile(r"^(.*)\[:(\w*):\]$")

    def parse(self, spec: dict[str, Any]) -> ScheduleSpec:
        return ScheduleSpec(tuple(self._declaration(k, v) for k, v in spec.items()))

    def _declaration(self, key: str, value: Any) -> AxisDecl | TileDecl | SplitDecl:
        if not isinstance(value, dict):
            raise ScheduleParseError(f"`{key}`: the value of a declaration should be a dict, not {value!r}")
        if ":" in key:
            axis, start, end, size = self._segment(key)
            return SplitDecl(axis, start, end, size, self.parse(value))
        if "#" in key:
            parts = key.split("#")
            if len(parts) != 2:
                raise ScheduleParseError(f"`{key}`: invalid tile syntax, expected 'axis#size'")
            return TileDecl(parts[0], _literal(parts[1]), self._annotations(value, key))
        return AxisDecl(key, self._annotations(value, key))

    def _segment(self, key: str) -> tuple[str, Literal | None, Literal | None, Literal | None]:
        m = self._SEGMENT.match(key)
        if m:
            axis, a, b = m.groups()
            return axis, (_literal(a) if a else None), (_literal(b) if b else None), None
        m = self._SIZED_SEGMENT.match(key)
        if not m:
            raise ScheduleParseError(f"Wrong format {key}")
        return m.group(1), None, None, _literal(m.group(2))

    def _annotations(self, value: dict[str, Any], context: str) -> Annotations:
        kw: dict[str, Any] = {}
        for key, param in value.items():
            if key == "unroll":
                if param is True or param is None:
                    kw.update(unroll=None, unroll_specified=True)
                elif param is False:
                    pass
                elif isinstance(param, (int, str)):
                    kw.update(unroll=param, unroll_specified=True)
                else:
                    raise ScheduleParseError(
                        f'`{{"unroll" = {param}}}`: unroll parameter should be True, False, or a string or integer.'
                    )
            elif key == "vectorize":
                param = True if param is None else param
                if not isinstance(param, (bool, str)):
                    raise ScheduleParseError(
                        f'`{{"vectorize" = {param}}}`: vectorization parameter should be True, False or a string.'
                    )
                kw["vectorize"] = param
            elif key == "parallelize":
                param = True if param is None else param
                if not isinstance(param, (bool, str)):
                    raise ScheduleParseError(
                        f'`{{"parallelize" = {param}}}`: parallelization parameter should be True, False or a string.'
                    )
                kw["parallelize"] = param
            elif key == "buffer":
                if not isinstance(param, str):
                    raise ScheduleParseError(f'`{{"buffer" = {param}}}`: buffer parameter should be a string (mtype).')
                kw.update(buffer=None if param == "default" else param, buffer_specified=True)
            elif key == "pack":
                kw.update(pack=self._pack(param, context), pack_specified=True)
            elif key == "partial":
                kw["partial"] = True
            elif key == "full":
                kw["full"] = True
            else:
                raise ScheduleParseError(f"Unknown annotation on {context}: {key}")
        if kw.get("partial") and kw.get("full"):
            raise ScheduleParseError(f"{context} has both annotations full and partial")
        return Annotations(**kw)

    @staticmethod
    def _pack(param: Any, context: str) -> tuple[Literal, str | None, bool | str]:
        if param is None:
            return (context, None, False)
        if not isinstance(param, (list, tuple)) or len(param) != 3:
            raise ScheduleParseError(
                f'`{{"pack" = {param}}}` on {context}: pack parameter should be a tuple (input_idx, mtype, pad).'
            )
        idx, mtype, pad = param
        if not isinstance(idx, (int, str)):
            raise ScheduleParseError(f'`{{"pack" = {param}}}` on {context}: input_idx should be an integer.')
        if mtype is not None and not isinstance(mtype, str):
            raise ScheduleParseError(f'`{{"pack" = {param}}}` on {context}: mtype should be a string or None.')
        if not isinstance(pad, (bool, str)):
            raise ScheduleParseError(f'`{{"pack" = {param}}}` on {context}: pad should be a boolean.')
        return (idx, None if mtype == "default" else mtype, pad)


class YAMLParser:
    """YAML text -> dict specification.  A string value lists keywords
    ("parallelize unroll=4"); a "size" entry turns the key into a tile."""

    def parse(self, text: str) -> dict[str, Any]:
        data = yaml.safe_load(text)
        if not isinstance(data, dict):
            raise ScheduleParseError(f"Wrong format: YAML input parses to {type(data)}.")
        return self._convert(data)

    def _convert(self, spec: dict[str, Any]) -> dict[str, Any]:
        spec = dict(spec)
        constraints = spec.pop("constraints", [])
        out: dict[str, Any] = {}
        for key, value in spec.items():
            if value is None:
                d: dict[str, Any] = {}
            elif isinstance(value, str):
                d = self._keywords(value)
            elif isinstance(value, dict):
                d = dict(value)
            else:
                raise ScheduleParseError(f"Value {value} of key {key} is neither a string nor a dict.")
            size = d.pop("size", None)
            if size:
                key = f"{key}#{size}"
            out[str(key)] = self._convert(d) if ":" in str(key) else d
        if constraints:
            out["constraints"] = list(constraints)
        return out

    @staticmethod
    def _keywords(text: str) -> dict[str, Any]:
        d: dict[str, Any] = {}
        for word in text.split():
            if "=" not in word:
                d[word] = None
                continue
            k, v = word.split("=", 1)
            try:
                d[k] = yaml.safe_load(v)
            except yaml.YAMLError:
                d[k] = v
        return d


# ------------------------------------------------------------------ interpretation


@dataclass
class _NodeParams:
    """Parameterised annotations of a node, resolved by `instantiate`."""

    vectorize: dict[str, str] = field(default_factory=dict)
    parallelize: dict[str, str] = field(default_factory=dict)


class ScheduleInterpreter:
    """ScheduleSpec -> LoopNest (sizes may be parameter names; constraints on
    them accumulate in LoopNest.constraints)."""

    def __init__(
        self,
        abstract_dims: list[str],
        abstract_dim_sizes: dict[str, int] | None = None,
        abstract_matrix: list[str] | None = None,
        partial_tiles: bool = False,
        partial_unrolls: bool = False,
    ) -> None:
        self.abstract_dims = list(abstract_dims)
        self.abstract_dim_sizes = dict(abstract_dim_sizes or {})
        self.abstract_matrix = list(abstract_matrix or [])
        self.partial_tiles = partial_tiles
        self.partial_unrolls = partial_unrolls

    def interpret(self, spec: ScheduleSpec, root: str) -> LoopNest:
        nest = LoopNest(abstract_dims=list(self.abstract_dims))
        node = nest.build_root_node(root)
        self._params: dict[int, _NodeParams] = {}
        self._node(spec, node, root, [], {a: ([s] if (s := self.abstract_dim_sizes.get(a)) else []) for a in self.abstract_dims},
                   nest.constraints)
        nest.params = self._params  # type: ignore[attr-defined]
        return nest

    # extents: axis -> enclosing sizes, outermost first
    def _node(self, spec: ScheduleSpec, node: LoopNestNode, root: str, head: list[str],
              extents: dict[str, list[Literal]], constraints: list[str]) -> None:
        order = list(head)
        cut: dict[str, Literal | None] = {a: 0 for a in self.abstract_dims}
        sizes: dict[str, Literal] = {}
        sized_cuts: list[tuple[str, Literal | None]] = []
        loop = ""
        for item in spec.items:
            if isinstance(item, SplitDecl):
                self._segment(item, node, root, order, cut, extents, constraints, sized_cuts)
            elif isinstance(item, TileDecl):
                loop = self._tile(item, node, order, sizes, extents, constraints)
                self._annotate(item.annotations, loop, sizes, node, constraints)
            else:
                name = self._axis(item, order)
                if name:
                    loop = name
                self._annotate(item.annotations, loop, sizes, node, constraints)
        # a segment of variable size that ends the axis ends at its extent:
        # its cut placeholder is replaced by that extent
        for name, total in sized_cuts:
            axis = next((a for a, c in cut.items() if c == name), None)
            if axis is None or total is None:
                continue
            word = re.compile(rf"\b{re.escape(name)}\b")
            constraints[:] = [word.sub(str(total), c) for c in constraints]
            for child in node.children:
                origin = child.split_origin
                if origin is not None and origin.end == name:
                    child.split_origin = SplitOrigin(axis=origin.axis, start=origin.start, end=total)
            cut[axis] = total
        for axis, c in cut.items():
            full = extents[axis][-1] if extents.get(axis) else None
            if isinstance(c, int) and c not in (0, full):
                raise ScheduleInterpretError(f"Splitting of {axis} unachieved (stops at {c}).")
        node.interchange = order

    def _segment(self, item: SplitDecl, node: LoopNestNode, root: str, order: list[str],
                 cut: dict[str, Literal | None], extents: dict[str, list[Literal]], constraints: list[str],
                 sized_cuts: list[tuple[str, Literal | None]]) -> None:
        axis = item.axis
        self._known(axis)
        prev = cut[axis]
        total = extents[axis][-1] if extents[axis] else None
        start = item.start if item.start is not None else prev
        if item.size is None:
            self._contiguous(item, prev, start)
        segs = node.splits.setdefault(axis, {})
        name = f"{axis}[{len(segs)}]"
        segs[name] = prev if item.size is not None else start
        order.append(name)
        if item.size is None:
            end = item.end
            cut[axis] = end
            stop = total if end is None else end
            inner: Literal | None = None
            if isinstance(start, int):
                if start == 0:
                    inner = stop
                elif isinstance(stop, int):
                    inner = stop - start
            if inner is None:
                inner = (root.lstrip(".").lstrip("/") + name).replace("[", "_").replace("]", "_").replace("/", "")
                constraints.append(f"{inner} <= {stop}")
                if isinstance(start, str):
                    constraints.append(f"{start} <= {stop}")
                constraints.append(f"{inner} + {start} == {stop}")
            seg_start, seg_end = start, end
        else:
            seg_start, seg_end = prev, None
            if isinstance(item.size, int) and isinstance(prev, int):
                cut[axis] = prev + item.size
                seg_end = prev + item.size
            elif prev == 0:
                cut[axis] = item.size
                seg_end = item.size
            else:
                new_cut = (root.lstrip(".").lstrip("/") + name).replace("[", "_").replace("]", "_").replace("/", "")
                if sized_cuts:
                    # an earlier variable cut lies within the extent
                    constraints.append(f"{sized_cuts[-1][0]} <= {sized_cuts[-1][1]}")
                sized_cuts.append((new_cut, total))
                cut[axis] = new_cut
                constraints.append(f"{item.size} + {prev} == {new_cut}")
                seg_end = new_cut
            if total is not None and not isinstance(total, int):
                constraints.append(f"{cut[axis]} <= {total}")
        child = LoopNestNode(root=f"{root}/{name}", tiles={a: {} for a in self.abstract_dims},
                             split_origin=SplitOrigin(axis=axis, start=seg_start, end=seg_end))
        node.add_child(child)
        child_extents = copy.deepcopy(extents)
        self._node(item.body, child, f"{root}/{name}", [axis], child_extents, constraints)

    def _tile(self, item: TileDecl, node: LoopNestNode, order: list[str], sizes: dict[str, Literal],
              extents: dict[str, list[Literal]], constraints: list[str]) -> str:
        self._known(item.axis)
        if isinstance(item.size, int) and item.size <= 0:
            raise ScheduleInterpretError(f"`{item}`: tile sizes should be strictly positive.")
        name = f"{item.axis}{len(node.tiles[item.axis])}"
        node.tiles[item.axis][name] = item.size
        sizes[name] = item.size
        order.append(name)
        outer = extents.setdefault(item.axis, [])
        if isinstance(item.size, str):
            if item.annotations.partial or (not item.annotations.full and self.partial_tiles):
                if not outer:
                    raise ScheduleInterpretError(f"`{item}`: {item.size} is a partial tile, but its range cannot be computed.")
                constraints.append(f"{item.size} <= {outer[-1]}")
            else:
                if not self.abstract_dim_sizes:
                    raise ScheduleInterpretError(f"`{item}` is a full tile, but the axis sizes are unknown.")
                constraints.append(f"{item.size} || {{{', '.join(map(str, outer))}}}")
        outer.append(item.size)
        return name

    def _axis(self, item: AxisDecl, order: list[str]) -> str:
        if item.axis in self.abstract_matrix:
            return ""
        self._known(item.axis)
        if item.axis in order:
            raise ScheduleInterpretError(f"Axis {item.axis} is scheduled twice (or more).")
        order.append(item.axis)
        return item.axis

    def _annotate(self, ann: Annotations, loop: str, sizes: dict[str, Literal], node: LoopNestNode,
                  constraints: list[str]) -> None:
        params = self._params.setdefault(id(node), _NodeParams())
        if ann.unroll_specified:
            factor = ann.unroll
            if factor is None:
                if loop not in sizes:
                    raise ScheduleInterpretError(f"{loop}'s size being unknown, an unroll factor is needed.")
                factor = sizes[loop]
            elif isinstance(factor, int) and factor <= 0:
                raise ScheduleInterpretError(f'`{{"unroll" = {factor}}}`: unroll parameter should be strictly positive.')
            elif isinstance(factor, str) and loop in sizes:
                op = "<=" if self.partial_unrolls else "||"
                constraints.append(f"{factor} {op} {sizes[loop]}")
            node.unroll[loop] = factor
        for kind, value, target, table in (
            ("vectorize", ann.vectorize, node.vectorize, params.vectorize),
            ("parallelize", ann.parallelize, node.parallelize, params.parallelize),
        ):
            if isinstance(value, str):
                table[loop] = value
                constraints.append(f"{value} in {{0, 1}}")
            elif value:
                target.append(loop)
        if ann.buffer_specified:
            node.buffer_at[loop] = ann.buffer
        if ann.pack_specified and ann.pack is not None:
            idx, mtype, pad = ann.pack
            if isinstance(idx, str):
                pos = self.abstract_matrix.index(idx)
                if pos == len(self.abstract_matrix) - 1:
                    node.buffer_at[loop] = mtype
                else:
                    node.pack_at[loop] = (pos, mtype, pad)
            else:
                node.pack_at[loop] = (idx, mtype, pad)

    def _known(self, axis: str) -> None:
        if axis not in self.abstract_dims:
            raise ScheduleInterpretError(f"Axis {axis} is not a defined axis (defined axis: {self.abstract_dims}).")

    @staticmethod
    def _contiguous(item: SplitDecl, prev: Literal | None, start: Literal) -> None:
        if prev is None:
            raise ScheduleInterpretError(f"{item}: {item.axis} already covered.")
        if isinstance(start, int) and isinstance(prev, int):
            if start > prev:
                raise ScheduleInterpretError(f"{item}: splitting doesn't fully cover {item.axis} (jumps from {prev} to {start}).")
            if start < prev:
                raise ScheduleInterpretError(f"{item}: the segment begins at {start} but the previous one ends at {prev}.")
        elif start != prev:
            raise ScheduleInterpretError(f"{item}: Splitting ends at {prev} and begins at {start}. These need to be the same.")
        if isinstance(start, int) and isinstance(item.end, int) and start >= item.end:
            raise ScheduleInterpretError(f"{item}: the ending point should be greater than the starting point.")


# ------------------------------------------------------------------ parameters


_EXPR_NODES = (ast.Expression, ast.BinOp, ast.UnaryOp, ast.Add, ast.Sub, ast.Mult, ast.FloorDiv, ast.USub,
               ast.UAdd, ast.Constant, ast.Name, ast.Load)
_COMPARE_NODES = (ast.Compare, ast.LtE, ast.GtE, ast.Lt, ast.Gt, ast.Eq, ast.NotEq)


@functools.lru_cache(maxsize=4096)
def compile_expr(text: str, compare: bool = False) -> tuple[Any, tuple[str, ...]]:
    """An integer expression over parameters (+, -, *, //, parentheses), or
    with `compare` a chain of comparisons of such expressions, as
    (code object, parameter names).  Anything else is refused."""
    try:
        tree = ast.parse(text.strip(), mode="eval")
    except SyntaxError as err:
        raise ScheduleValidationError(f"cannot parse `{text}`: {err.msg}") from None
    allowed = _EXPR_NODES + (_COMPARE_NODES if compare else ())
    for n in ast.walk(tree):
        if not isinstance(n, allowed) or (isinstance(n, ast.Constant) and type(n.value) is not int):
            raise ScheduleValidationError(f"unsupported expression `{text}`")
    if compare and not isinstance(tree.body, ast.Compare):
        raise ScheduleValidationError(f"unsupported constraint `{text}`")
    names = tuple(dict.fromkeys(n.id for n in ast.walk(tree) if isinstance(n, ast.Name)))
    return compile(tree, "<descript>", "eval"), names


def _eval(text: str, sample: dict[str, int], compare: bool = False) -> int:
    code, names = compile_expr(text, compare)
    env = {}
    for n in names:
        if n not in sample:
            raise ScheduleValidationError(f"parameter {n} has no value in the sample")
        env[n] = int(sample[n])
    return eval(code, {"__builtins__": {}}, env)  # noqa: S307 - whitelisted integer AST


def _value(token: str, sample: dict[str, int]) -> int:
    return int(_eval(token, sample))


def _expr(text: str, sample: dict[str, int]) -> int:
    return int(_eval(text, sample))


def _members(text: str) -> list[str]:
    return [v for v in text.strip().strip("{}").split(",") if v.strip()]


def check_constraints(constraints: list[str], sample: dict[str, int]) -> None:
    """Evaluates the constraint forms of descript specs and their
    interpreter: comparisons of integer expressions (`a <= b`,
    `a * b >= 8`, `a == b + c`, ...), `a in {x, y}`, and `a || {b, c}` /
    `a || b` (a divides every listed size)."""
    for c in constraints:
        if " in " in c:
            lhs, rhs = c.split(" in ", 1)
            ok = _expr(lhs, sample) in {_expr(v, sample) for v in _members(rhs)}
        elif "||" in c:
            lhs, rhs = c.split("||", 1)
            a = _expr(lhs, sample)
            ok = a > 0 and all(_expr(v, sample) % a == 0 for v in _members(rhs))
        else:
            ok = bool(_eval(c, sample, compare=True))
        if not ok:
            raise ScheduleValidationError(f"constraint `{c}` does not hold for {sample}")


def instantiate(nest: LoopNest, sample: dict[str, int]) -> LoopNest:
    """A copy of `nest` with every parameter replaced by its sample value;
    parameterised vectorize/parallelize apply when their value is 1."""
    check_constraints(nest.constraints, sample)
    params: dict[int, _NodeParams] = getattr(nest, "params", {})

    def val(v: Any) -> Any:
        return _expr(v, sample) if isinstance(v, str) else v

    out = LoopNest(abstract_dims=list(nest.abstract_dims))

    def copy_node(src: LoopNestNode) -> LoopNestNode:
        dst = LoopNestNode(
            root=src.root,
            tiles={a: {n: val(s) for n, s in t.items()} for a, t in src.tiles.items()},
            splits={a: {n: val(s) for n, s in t.items()} for a, t in src.splits.items()},
            interchange=list(src.interchange),
            vectorize=list(src.vectorize),
            parallelize=list(src.parallelize),
            unroll={n: val(f) for n, f in src.unroll.items()},
            buffer_at=dict(src.buffer_at),
            pack_at={n: (i, m, bool(val(p)) if isinstance(p, str) else p) for n, (i, m, p) in src.pack_at.items()},
            split_origin=None if src.split_origin is None else SplitOrigin(
                src.split_origin.axis, val(src.split_origin.start), val(src.split_origin.end)),
        )
        p = params.get(id(src))
        if p is not None:
            dst.vectorize += [l for l, name in p.vectorize.items() if _value(name, sample)]
            dst.parallelize += [l for l, name in p.parallelize.items() if _value(name, sample)]
        for child in src.children:
            dst.add_child(copy_node(child))
        return dst

    if nest.root_node is not None:
        out.root_node = copy_node(nest.root_node)
    return out


# ------------------------------------------------------------------ application


@dataclass(frozen=True)
class Descript:
    abstract_dims: list[str]
    abstract_dim_sizes: dict[str, int] = field(default_factory=dict)
    abstract_matrix: list[str] = field(default_factory=list)
    partial_tiles: bool = False
    partial_unrolls: bool = False

    def loop_nest(self, node_name: str, spec: dict[str, Any] | str) -> LoopNest:
        if isinstance(spec, str):
            spec = YAMLParser().parse(spec)
        spec = dict(spec)
        constraints = list(spec.pop("constraints", []))
        ast = ScheduleParser().parse(spec)
        nest = ScheduleInterpreter(
            self.abstract_dims, self.abstract_dim_sizes, self.abstract_matrix, self.partial_tiles, self.partial_unrolls
        ).interpret(ast, root=node_name)
        nest.constraints += constraints
        return nest

    def apply_sample(self, nest: LoopNest, sample: dict[str, int], scheduler: Any) -> None:
        concrete = instantiate(nest, sample)
        concrete.check()
        self._apply(concrete, scheduler)

    def apply(self, node_name: str, spec: dict[str, Any] | str, scheduler: Any, sample: dict[str, int] | None = None) -> None:
        self.apply_sample(self.loop_nest(node_name, spec), dict(sample or {}), scheduler)

    def _apply(self, nest: LoopNest, scheduler: Any) -> None:
        scheduler.set_dims(list(self.abstract_dims))
        if nest.root_node is not None:
            self._apply_node(nest.root_node, scheduler, ".")

    def _apply_node(self, node: LoopNestNode, scheduler: Any, root: str) -> None:
        for axis, segs in node.splits.items():
            scheduler.split(axis, dict(segs), root=root)
        for axis, tiles in node.tiles.items():
            if tiles:
                scheduler.tile(axis, dict(tiles), root=root)
        scheduler.interchange(list(node.interchange), root=root)
        scheduler.vectorize(list(node.vectorize), root=root)
        scheduler.parallelize(list(node.parallelize), root=root)
        scheduler.unroll(dict(node.unroll), root=root)
        for loop, mtype in node.buffer_at.items():
            scheduler.buffer_at(loop, mtype=mtype, root=root)
        for loop, (idx, mtype, pad) in node.pack_at.items():
            scheduler.pack_at(loop, idx, mtype=mtype, pad=pad, root=root)
        for child in node.children:
            seg = next(n for n, s in node.splits.get(child.split_origin.axis, {}).items()
                       if s == child.split_origin.start) if child.split_origin else None
            self._apply_node(child, scheduler, f"{root}/{seg}" if seg else root)


def descript_scheduler(
    scheduler: Any,
    node_name: str,
    abstract_dims: list[str],
    spec: dict[str, Any] | str,
    abstract_dim_sizes: dict[str, int] | None = None,
    abstract_matrix: list[str] | None = None,
    sample: dict[str, int] | None = None,
) -> None:
    """Applies a descript specification to `scheduler` for node `node_name`
    whose axes are named `abstract_dims` (descript.py:36-60)."""
    Descript(list(abstract_dims), dict(abstract_dim_sizes or {}), list(abstract_matrix or [])).apply(
        node_name, spec, scheduler, sample
    )
