# SPDX-License-Identifier: BSD-3-Clause
"""Executor interface (src/xtc/itf/exec/executor.py:10-38)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from ..comp.module import Module

__all__ = ["Executor"]


class Executor(ABC):
    """Runs a Module once; `execute()` returns 0 on success."""

    @abstractmethod
    def execute(self) -> int: ...

    @property
    @abstractmethod
    def module(self) -> "Module": ...
