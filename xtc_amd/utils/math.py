# SPDX-License-Identifier: BSD-3-Clause
"""Integer helpers of the tiling search (src/xtc/utils/math.py:13-95) and
the sample-space estimators of its unique sampling (math.py:103-158)."""

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
    "estimate_count_prob_smooth",
    "estimate_unique_prob_good_turing",
    "estimate_unique_num_chao1",
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


def estimate_count_prob_smooth(count: int, sample_size: int, alpha: float = 1.0) -> float:
    """Additive (Laplace) smoothing of the frequency count / sample_size:
    (count + alpha) / (sample_size + alpha), and 0 for alpha = 0 with no
    samples (math.py:141-158)."""
    if not 0 <= count <= sample_size or alpha < 0:
        raise ValueError(f"need 0 <= count <= sample_size and alpha >= 0: {count}, {sample_size}, {alpha}")
    if alpha == 0 and sample_size == 0:
        return 0.0
    return (count + alpha) / (sample_size + alpha)


def estimate_unique_prob_good_turing(sample_size: int, once_num: int) -> float:
    """Good-Turing estimate of the chance that the next draw is a value not
    seen yet: the share of draws seen exactly once, smoothed as above so
    that empty or small samples give a usable value (math.py:126-138)."""
    if not 0 <= once_num <= sample_size:
        raise ValueError(f"need 0 <= once_num <= sample_size: {once_num}, {sample_size}")
    return estimate_count_prob_smooth(once_num, sample_size)


def estimate_unique_num_chao1(unique_num: int, once_num: int, twice_num: int) -> int:
    """Bias-corrected Chao1 lower bound on the number of distinct values of a
    space, from the distinct values drawn so far and those seen exactly once
    (f1) and twice (f2): S_obs + f1 (f1 - 1) / (2 (f2 + 1)), rounded to the
    nearest integer (Chao's estimator as the SpadeR guide states it;
    math.py:103-123)."""
    if once_num < 0 or twice_num < 0 or unique_num < once_num + twice_num:
        raise ValueError(f"need f1, f2 >= 0 and unique_num >= f1 + f2: {unique_num}, {once_num}, {twice_num}")
    return int(unique_num + once_num * (once_num - 1) / (2 * (twice_num + 1)) + 0.5)
