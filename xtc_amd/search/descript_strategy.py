# SPDX-License-Identifier: BSD-3-Clause
"""A search strategy over the free parameters of a descript schedule spec:
`loop-explore --descript spec.yaml`
(Strategy_Descript / Strategy_Descript_Explore,
src/xtc/search/strategies.py:1031-1185).

The spec is interpreted once into a parametric loop nest
(xtc_amd.schedules.descript).  Its parameters are the names the spec uses for
tile sizes, unroll factors, split points and annotation switches, plus the
spec's own `constraints:`; the interpreter emits the constraints that make a
sample legal (a tile divides the sizes it tiles, an unroll divides its loop,
a switch is 0 or 1, split cuts are ordered and cover the axis): `a || {x, y}`
(a divides x and y), `a in {x, y}`, and comparisons of integer expressions
(`a <= b`, `i_1_ + iS == iL2`, `nvr * mr * kr <= 256`).  A sample is one
integer per parameter, in the order the parameters first appear in those
constraints; `generate` instantiates the nest with it and applies it to the
scheduler.

The reference solves the constraints with xvs and z3 (neither installed
here).  This module solves them by depth-first search: each parameter's
domain comes from the constraints that bound it directly (an `in` set, the
divisors of the literal sizes it divides, else 1 up to its literal bound or
the largest dimension); parameters with small domains are assigned first; an
equation with one unknown left assigns it; a comparison or divisibility with
one unknown left narrows that unknown's candidates; and a comparison whose
sum-and-product side already exceeds its bound at the parameters' least
values cuts the branch.  A space of up to ENUMERATION_BUDGET search steps is
enumerated and sampled uniformly without replacement; a larger one is
sampled by randomised depth-first draws.  The legal set is the reference's
(the constraint lists and the counts of distinct samples match its tests);
the order of the seeded draws is this module's own, so it is parity unpinned.
"""

from __future__ import annotations

import ast
from bisect import bisect_left, bisect_right
from collections.abc import Callable, Iterator, Mapping
from math import gcd
from typing import Any

import numpy as np

from ..itf.schd import DEFAULT_ROOT
from ..itf.search import Sample, Strategy, VecSample
from ..schedules.descript import Descript, compile_expr
from ..utils.algorithms import sample_uniques

__all__ = ["Strategy_Descript", "Strategy_Descript_Explore"]

# a complete enumeration is attempted up to this many solver steps; above
# it, samples come from randomised depth-first draws
ENUMERATION_BUDGET = 20_000
DRAW_BUDGET = 2_000


def _divisors(n: int) -> list[int]:
    return [d for d in range(1, n + 1) if n % d == 0] if n > 0 else [1]


def _monotone(text: str) -> bool:
    """True when the expression only adds and multiplies: it then grows with
    every parameter over non-negative values."""
    tree = ast.parse(text, mode="eval")
    return not any(isinstance(n, (ast.Sub, ast.USub, ast.FloorDiv)) for n in ast.walk(tree)) and not any(
        isinstance(n, ast.Constant) and n.value < 0 for n in ast.walk(tree)
    )


class _Expr:
    """A compiled integer expression and its parameters."""

    __slots__ = ("text", "code", "names", "monotone")

    def __init__(self, text: str) -> None:
        self.text = text.strip()
        self.code, names = compile_expr(self.text)
        self.names = frozenset(names)
        self.monotone = _monotone(self.text)

    def __call__(self, env: Mapping[str, int]) -> int:
        return eval(self.code, {"__builtins__": {}}, env)  # noqa: S307 - whitelisted integer AST


class _Con:
    """One constraint, prepared for checks on partial assignments."""

    def __init__(self, text: str) -> None:
        self.text = text
        self.op = ""
        if " in " in text or "||" in text:
            sep = " in " if " in " in text else "||"
            lhs, rhs = text.split(sep, 1)
            self.kind = "in" if sep == " in " else "div"
            self.lhs = _Expr(lhs)
            self.members = [_Expr(v) for v in rhs.strip().strip("{}").split(",") if v.strip()]
            self.rhs = None
        else:
            compile_expr(text, compare=True)
            tree = ast.parse(text.strip(), mode="eval").body
            assert isinstance(tree, ast.Compare)
            self.kind = "cmp"
            self.members = []
            if len(tree.ops) == 1:
                ops = {ast.LtE: "<=", ast.GtE: ">=", ast.Lt: "<", ast.Gt: ">", ast.Eq: "==", ast.NotEq: "!="}
                self.op = ops[type(tree.ops[0])]
                self.lhs, self.rhs = _Expr(ast.unparse(tree.left)), _Expr(ast.unparse(tree.comparators[0]))
            else:
                self.lhs = self.rhs = None
        if self.lhs is None:
            self.names = frozenset(compile_expr(text, compare=True)[1])
        else:
            self.names = self.lhs.names.union(*(m.names for m in self.members),
                                              self.rhs.names if self.rhs is not None else ())

    def holds(self, env: Mapping[str, int]) -> bool:
        """Evaluated with every parameter assigned."""
        if self.kind == "in":
            return self.lhs(env) in {m(env) for m in self.members}
        if self.kind == "div":
            a = self.lhs(env)
            return a > 0 and all(m(env) % a == 0 for m in self.members)
        if self.lhs is None:
            code, names = compile_expr(self.text, compare=True)
            return bool(eval(code, {"__builtins__": {}}, {n: env[n] for n in names}))  # noqa: S307
        a, b = self.lhs(env), self.rhs(env)
        return {"<=": a <= b, "<": a < b, ">=": a >= b, ">": a > b, "==": a == b, "!=": a != b}[self.op]

    def refutes(self, env: Mapping[str, int], low: Mapping[str, int]) -> bool:
        """True when no completion of the partial assignment `env` can
        satisfy the constraint; `low` holds each parameter's least value."""
        if self.names <= env.keys():
            return not self.holds(env)
        if self.kind == "div":
            if self.lhs.names <= env.keys():
                a = self.lhs(env)
                if a <= 0:
                    return True
                return any(m.names <= env.keys() and m(env) % a for m in self.members)
            return False
        if self.op in ("<=", "<", ">=", ">"):
            small, big = (self.lhs, self.rhs) if self.op in ("<=", "<") else (self.rhs, self.lhs)
            if big.names <= env.keys() and small.monotone:
                least = small({**low, **env})
                bound = big(env)
                return least > bound or (self.op in ("<", ">") and least == bound)
        return False

    def derive(self, env: Mapping[str, int]) -> tuple[str, int | None] | None:
        """For `a == b` with one parameter unassigned, in which the equation
        is linear: (parameter, its value, or None when no integer fits)."""
        if self.op != "==":
            return None
        missing = self.names.difference(env)
        if len(missing) != 1:
            return None
        (v,) = missing
        e = dict(env)

        def f(x: int) -> int:
            e[v] = x
            return self.lhs(e) - self.rhs(e)

        f0, f1, f2 = f(0), f(1), f(2)
        slope = f1 - f0
        if slope == 0 or f2 - f1 != slope:
            return None
        if f0 % slope:
            return v, None
        x = -f0 // slope
        return (v, x) if f(x) == 0 else (v, None)


class Strategy_Descript(Strategy):
    def __init__(
        self,
        graph: Any,
        spec: dict[str, Any] | str,
        constraints: list[str] | None = None,
        partial_tiles: bool = False,
        partial_unrolls: bool = False,
        sample_filter: Callable[[list[int]], bool] | None = None,
        node: str | None = None,
        **kwargs: Any,
    ) -> None:
        from .strategies import _operation_of

        self._graph = graph
        op = _operation_of(graph, node)
        self._axes = list(op.dims)
        self._sizes = {a: int(v) for a, v in op.dims.items() if isinstance(v, int)}
        self._descript = Descript(
            abstract_dims=self._axes,
            abstract_dim_sizes=dict(self._sizes),
            abstract_matrix=["A", "B", "C"],
            partial_tiles=partial_tiles,
            partial_unrolls=partial_unrolls,
        )
        self._nest = self._descript.loop_nest(DEFAULT_ROOT, spec)
        self._constraints = list(constraints or []) + list(self._nest.constraints)
        self._cons = [_Con(c) for c in self._constraints]
        self._eqs = [c for c in self._cons if c.op == "=="]
        # parameters in order of first appearance in the constraints
        self._params: list[str] = []
        for c in self._constraints:
            for n in ast.walk(ast.parse(c.replace("||", "<=").replace(" in ", "==").replace("{", "(")
                                         .replace("}", ")"), mode="eval")):
                if isinstance(n, ast.Name) and n.id not in self._params:
                    self._params.append(n.id)
        self._domains = {p: self._domain(p) for p in self._params}
        self._low = {p: min(d) for p, d in self._domains.items()}
        self._members = {p: set(d) for p, d in self._domains.items()}
        self._by_param = {p: [c for c in self._cons if p in c.names] for p in self._params}
        # the search assigns small domains first: divisor and switch
        # parameters settle the equations and bounds that prune the ranges
        self._order = sorted(self._params, key=lambda p: len(self._domains[p]))
        self._sample_filter = sample_filter
        self._stats: dict[str, int] = {"enumerated": 0, "draws": 0, "filtered": 0}
        self._solutions: list[tuple[int, ...]] | None = None
        self._complete = False

    # ---- domains
    def _domain(self, p: str) -> list[int]:
        top = max(self._sizes.values(), default=1)

        def literal(e: _Expr) -> bool:
            return not e.names

        for c in self._cons:
            if c.kind == "in" and c.lhs.text == p and all(literal(m) for m in c.members):
                return sorted({m({}) for m in c.members})
        for c in self._cons:
            if c.kind == "div" and c.lhs.text == p and any(literal(m) for m in c.members):
                g = 0
                for m in c.members:
                    if literal(m):
                        g = gcd(g, abs(m({})))
                return _divisors(g)
        # a literal upper bound, else the largest dimension
        bounds = [c.rhs({}) - (c.op == "<") for c in self._cons
                  if c.kind == "cmp" and c.op in ("<=", "<") and c.lhs is not None and c.lhs.text == p
                  and literal(c.rhs)]
        return list(range(1, max(1, min(bounds) if bounds else top) + 1))

    # ---- solver
    def _consistent(self, env: dict[str, int], changed: str) -> bool:
        return not any(c.refutes(env, self._low) for c in self._by_param[changed])

    def _propagate(self, env: dict[str, int], trail: list[str]) -> bool:
        """Assigns every parameter an equation fixes; False on a conflict."""
        progress = True
        while progress:
            progress = False
            for c in self._eqs:
                got = c.derive(env)
                if got is None:
                    continue
                v, x = got
                if x is None or x not in self._members[v]:
                    return False
                env[v] = x
                trail.append(v)
                if not self._consistent(env, v):
                    return False
                progress = True
        return True

    def _candidates(self, v: str, env: dict[str, int]) -> list[int]:
        """The values of `v`'s domain that the constraints whose only
        unassigned parameter is `v` leave: bounds from linear comparisons,
        multiples and divisors from `||`."""
        lo, hi, mult = None, None, 1
        divides: list[int] = []
        e = dict(env)
        for c in self._by_param[v]:
            if len(c.names) - len(c.names & env.keys()) != 1:
                continue
            if c.kind == "div":
                if c.lhs.text == v:
                    divides += [m(env) for m in c.members]
                elif c.lhs.names <= env.keys() and any(m.text == v for m in c.members):
                    a = c.lhs(env)
                    mult = mult * a // gcd(mult, a) if a > 0 else mult
                continue
            if c.op not in ("<=", "<", ">=", ">") or c.lhs is None:
                continue

            def f(x: int) -> int:
                e[v] = x
                return c.lhs(e) - c.rhs(e)

            f0, f1, f2 = f(0), f(1), f(2)
            slope = f1 - f0
            if slope == 0 or f2 - f1 != slope:
                continue
            # f0 + slope * x <= t  (or >= t)
            le = c.op in ("<=", "<")
            t = -1 if c.op == "<" else (1 if c.op == ">" else 0)
            if (slope > 0) == le:  # an upper bound on x
                b = (t - f0) // slope if slope > 0 else -((t - f0) // -slope)
                hi = b if hi is None else min(hi, b)
            else:
                b = -((f0 - t) // slope) if slope > 0 else (f0 - t) // -slope
                lo = b if lo is None else max(lo, b)
        dom = self._domains[v]
        i = bisect_left(dom, lo) if lo is not None else 0
        j = bisect_right(dom, hi) if hi is not None else len(dom)
        return [x for x in dom[i:j] if x % mult == 0 and all(d % x == 0 for d in divides)]

    def _search(self, order: Callable[[list[int]], list[int]], budget: int) -> Iterator[tuple[int, ...]]:
        """Depth-first solutions, each parameter's candidates taken in
        `order`, within `budget` steps (self._exhausted says whether the
        space was covered)."""
        env: dict[str, int] = {}
        steps = 0
        self._exhausted = True

        def rec() -> Iterator[tuple[int, ...]]:
            nonlocal steps
            free = next((p for p in self._order if p not in env), None)
            if free is None:
                yield tuple(env[p] for p in self._params)
                return
            for x in order(self._candidates(free, env)):
                steps += 1
                if steps > budget:
                    self._exhausted = False
                    return
                trail = [free]
                env[free] = x
                if self._consistent(env, free) and self._propagate(env, trail):
                    yield from rec()
                for v in trail:
                    env.pop(v, None)
                if steps > budget:
                    return

        if self._propagate(env, []):
            yield from rec()

    def _accept(self, x: tuple[int, ...]) -> bool:
        if self._sample_filter is None or self._sample_filter(list(x)):
            return True
        self._stats["filtered"] += 1
        return False

    def _enumerate(self) -> list[tuple[int, ...]] | None:
        """Every solution, or None when the space exceeds the budget."""
        if self._solutions is None:
            sols = list(self._search(lambda c: c, ENUMERATION_BUDGET))
            self._complete = self._exhausted
            self._solutions = sols
            self._stats["enumerated"] = len(sols)
        return self._solutions if self._complete else None

    # ---- Strategy interface
    @property
    def graph(self) -> Any:
        return self._graph

    @property
    def sample_names(self) -> list[str]:
        return list(self._params)

    @property
    def stats(self) -> Mapping[str, int]:
        return self._stats

    def generate(self, scheduler: Any, sample: Sample | Mapping[str, int]) -> None:
        """Applies a sample: a list in `sample_names` order, or a mapping
        from parameter to value (the reference's Strategy_Descript form)."""
        env = dict(sample) if isinstance(sample, Mapping) else dict(zip(self._params, sample))
        self._descript.apply_sample(self._nest, env, scheduler)

    def exhaustive(self) -> Iterator[VecSample]:
        sols = self._enumerate()
        it = iter(sols) if sols is not None else self._search(lambda c: c, 1 << 62)
        for x in it:
            if self._accept(x):
                yield list(x)

    def default_schedule(self, opt_level: int = 2) -> VecSample:
        """The first legal sample in enumeration order (the spec fixes the
        schedule's shape; opt_level does not change it)."""
        if opt_level < 0:
            raise ValueError("opt_level must be >= 0")
        for x in self.exhaustive():
            return x
        raise ValueError("the descript spec has no legal sample")

    def sample(self, num: int, seed: int | None = 0) -> Iterator[VecSample]:
        """`num` distinct legal samples (fewer when fewer exist), seeded.  A
        space small enough to enumerate is drawn from uniformly without
        replacement; a larger one by randomised depth-first draws."""
        if num <= 0 or (seed is not None and seed < 0):
            raise ValueError("num must be > 0 and seed >= 0")
        rng = np.random.default_rng(seed=seed)
        sols = self._enumerate()
        if sols is not None:
            out = []
            for i in rng.permutation(len(sols)):
                if len(out) == num:
                    break
                if self._accept(sols[i]):
                    out.append(list(sols[i]))
            return iter(out)

        def shuffled(c: list[int]) -> list[int]:
            return [c[i] for i in rng.permutation(len(c))]

        def draw(n: int) -> Iterator[tuple[int, ...]]:
            for _ in range(n):
                self._stats["draws"] += 1
                for x in self._search(shuffled, DRAW_BUDGET):
                    if self._accept(x):
                        yield x
                        break

        return iter([list(s) for s in sample_uniques(draw, num)[:num]])  # type: ignore[arg-type]

    def dict_to_sample(self, sample: dict[str, Any]) -> Sample:
        return [sample[p] for p in self._params]

    def sample_to_dict(self, sample: Sample) -> dict[str, int]:
        return dict(zip(self._params, sample))


# the reference's explorer-facing name (src/xtc/search/strategies.py:1156-1183):
# samples as lists in a fixed parameter order, which Strategy_Descript does
Strategy_Descript_Explore = Strategy_Descript
