# SPDX-License-Identifier: BSD-3-Clause
"""Integer helpers of the tiling search (src/xtc/utils/math.py:13-95)."""

from __future__ import annotations

from functools import lru_cache
from math import isqrt, prod

__all__ = [
    "divisors_list",
    "factors_enumeration",
    "factors_to_sizes",
    "sizes_to_factors",
    "mulall",
    "pow2divisor",
]


@lru_cache(maxsize=None)
def _divisors(n: int) -> tuple[int, ...]:
    small = [d for d in range(1, isqrt(n) + 1) if n % d == 0]
    large = [n // d for d in reversed(small) if d * d != n]
    return tuple(small + large)


def divisors_list(n: int) -> list[int]:
    """Divisors of n in increasing order (1 and n included)."""
    return list(_divisors(n))


@lru_cache(maxsize=None)
def _factor_tuples(n: int, count: int) -> tuple[tuple[int, ...], ...]:
    if count == 0:
        return ((),)
    out: list[tuple[int, ...]] = []
    for d in _divisors(n):
        for rest in _factor_tuples(n // d, count - 1):
            out.append((d, *rest))
    return tuple(out)


def factors_enumeration(n: int, n_factors: int) -> list[list[int]]:
    """All `n_factors`-tuples of positive integers whose product divides n,
    in lexicographic order of increasing factors.

    Same enumeration order as the reference's sampler relies on
    (src/xtc/utils/math.py:39-68): e.g. for (28, 2) the list starts
    [1,1],[1,2],[1,4],[1,7],[1,14],[1,28],[2,1],...
    """
    return [list(t) for t in _factor_tuples(n, n_factors)]


def factors_to_sizes(factors: list[int]) -> list[int]:
    """Outer-to-inner factors -> outer-to-inner tile extents.

    [4, 1, 2, 2] -> [16, 4, 4, 2]: each extent is the product of its own
    factor and all inner ones.
    """
    sizes: list[int] = []
    acc = 1
    for f in reversed(factors):
        acc *= f
        sizes.append(acc)
    return sizes[::-1]


def sizes_to_factors(sizes: list[int]) -> list[int]:
    """Inverse of factors_to_sizes: [16, 4, 4, 2] -> [4, 1, 2, 2]."""
    out = []
    for idx, s in enumerate(sizes):
        inner = sizes[idx + 1] if idx + 1 < len(sizes) else 1
        out.append(s // inner)
    return out


def mulall(args: list[int]) -> int:
    return prod(args)


def pow2divisor(value: int) -> int:
    """Largest power of two dividing value."""
    return value & -value
