# SPDX-License-Identifier: BSD-3-Clause
"""Evaluator interface (src/xtc/itf/exec/evaluator.py:10-42)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from ..comp.module import Module

__all__ = ["Evaluator"]


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
