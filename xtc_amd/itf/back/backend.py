# SPDX-License-Identifier: BSD-3-Clause
"""Backend interface (src/xtc/itf/back/backend.py:13-56)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING, Any

if TYPE_CHECKING:
    from ..comp.compiler import Compiler
    from ..graph.graph import Graph
    from ..schd.scheduler import Scheduler


class Backend(ABC):
    """Implementation of a Graph for one target.

    Built as `Backend(graph, **kwargs)`; hands out the Scheduler that records
    transformations and the Compiler that turns the resulting Schedule into a
    Module.
    """

    @abstractmethod
    def get_scheduler(self, **kwargs: Any) -> "Scheduler": ...

    @abstractmethod
    def get_compiler(self, **kwargs: Any) -> "Compiler": ...

    @property
    @abstractmethod
    def graph(self) -> "Graph": ...
