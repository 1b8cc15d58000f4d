# SPDX-License-Identifier: BSD-3-Clause
"""Schedule interface (src/xtc/itf/schd/schedule.py:11-35)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from .scheduler import Scheduler


class Schedule(ABC):
    """Frozen result of the transformations recorded by a Scheduler."""

    @property
    @abstractmethod
    def scheduler(self) -> "Scheduler": ...
