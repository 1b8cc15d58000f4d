# SPDX-License-Identifier: BSD-3-Clause
"""Evaluator and Executor interfaces (src/xtc/itf/exec/evaluator.py:10-42,
src/xtc/itf/exec/executor.py:10-38)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from ..comp.module import Module

__all__ = ["Evaluator", "Executor"]


class Evaluator(ABC):
    """Runs a Module repeatedly, optionally validating it first.

    `evaluate()` returns `(results, code, message)`: per-repeat measurements
    (seconds per call, or counter values), 0 on success, and an error text.
    """

    @abstractmethod
    def evaluate(self) -> tuple[list[float], int, str]: ...

    @property
    @abstractmethod
    def module(self) -> "Module": ...


class Executor(ABC):
    """Runs a Module once; `execute()` returns 0 on success."""

    @abstractmethod
    def execute(self) -> int: ...

    @property
    @abstractmethod
    def module(self) -> "Module": ...
