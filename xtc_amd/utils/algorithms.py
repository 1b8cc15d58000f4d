# SPDX-License-Identifier: BSD-3-Clause
"""Unique sampling from a space of unknown size (src/xtc/utils/algorithms.py:20-120)."""

from __future__ import annotations

from collections.abc import Callable, Hashable, Iterator

from .math import estimate_unique_prob_good_turing

__all__ = ["sample_uniques"]


def sample_uniques(draw: Callable[[int], Iterator[Hashable]], num: int, prob: float = 1 / 1000) -> list[Hashable]:
    """Draws rounds of candidates until `num` unique ones are found or a new
    unique becomes unlikely.

    Each round asks `draw` for `round_num` candidates (doubling after an empty
    round).  The stop test estimates the chance that the next request yields
    a new unique sample as P(valid) * P(unseen), with P(valid) the fraction
    of requests that produced a candidate and P(unseen) the smoothed
    Good-Turing estimate (singletons + 1) / (draws + 1)
    (estimate_unique_prob_good_turing).  The stream of
    accepted samples is the reference's, so seeded explorations agree.
    """
    round_num = num
    samples: list[Hashable] = []
    seen: set[Hashable] = set()
    once: set[Hashable] = set()
    twice: set[Hashable] = set()
    draws = requests = 0
    p_next = 1.0
    while len(samples) < num and p_next > prob:
        got = list(draw(round_num))
        requests += round_num
        draws += len(got)
        for s in got:
            if s not in seen:
                samples.append(s)
                seen.add(s)
                once.add(s)
            elif s in once:
                once.remove(s)
                twice.add(s)
            elif s in twice:
                twice.remove(s)
        p_valid = max(1 / (requests + 1), draws / requests)
        p_unseen = estimate_unique_prob_good_turing(draws, len(once))
        p_next = p_valid * p_unseen
        if not got:
            round_num *= 2
    return samples[:num]
