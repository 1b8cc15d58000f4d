# SPDX-License-Identifier: BSD-3-Clause
"""Strategy interface (src/xtc/itf/search/strategy.py:22-164)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from collections.abc import Iterator
from typing import TYPE_CHECKING, Any, TypeAlias

if TYPE_CHECKING:
    from ..graph.graph import Graph
    from ..schd.scheduler import Scheduler

__all__ = ["Sample", "Strategy"]

Sample: TypeAlias = Any


class Strategy(ABC):
    """A schedule search space over one graph.

    A sample is a point of the space; `generate(scheduler, sample)` applies
    the corresponding transformations to a Scheduler.
    """

    @property
    @abstractmethod
    def graph(self) -> "Graph": ...

    @abstractmethod
    def generate(self, scheduler: "Scheduler", sample: Sample) -> None: ...

    @abstractmethod
    def exhaustive(self) -> Iterator[Sample]: ...

    @abstractmethod
    def sample(self, num: int, seed: int | None = 0) -> Iterator[Sample]: ...

    @abstractmethod
    def default_schedule(self, opt_level: int = 2) -> Sample: ...

    @property
    @abstractmethod
    def sample_names(self) -> list[str]: ...

    @abstractmethod
    def dict_to_sample(self, sample: dict[str, Any]) -> Sample: ...

    @abstractmethod
    def sample_to_dict(self, sample: Sample) -> dict[str, int]: ...
