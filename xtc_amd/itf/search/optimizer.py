# SPDX-License-Identifier: BSD-3-Clause
"""Optimizer interface (src/xtc/itf/search/optimizer.py)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TypeAlias

__all__ = ["VecSample", "Optimizer"]

VecSample: TypeAlias = "list[int]"


class Optimizer(ABC):
    """Suggest/observe loop of an iterative search."""

    @abstractmethod
    def suggest(self) -> list[VecSample]: ...

    @abstractmethod
    def observe(self, x: list[VecSample], y: list[float]) -> None: ...

    @abstractmethod
    def finished(self) -> bool: ...
