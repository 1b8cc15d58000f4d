# SPDX-License-Identifier: BSD-3-Clause
"""Compiler interface (src/xtc/itf/comp/compiler.py:19-39)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from ..back.backend import Backend
    from ..schd.schedule import Schedule
    from .module import Module


class Compiler(ABC):
    """Turns a Schedule of a Backend into an executable Module."""

    @abstractmethod
    def compile(self, schedule: "Schedule") -> "Module": ...

    @property
    @abstractmethod
    def backend(self) -> "Backend": ...
