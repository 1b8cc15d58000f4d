# SPDX-License-Identifier: BSD-3-Clause
"""Errors of the schedule description layer (src/xtc/schedules/exceptions.py)."""

from __future__ import annotations

__all__ = ["ScheduleError", "ScheduleParseError", "ScheduleInterpretError", "ScheduleValidationError"]


class ScheduleError(Exception):
    """Base class of schedule description errors."""


class ScheduleParseError(ScheduleError):
    """The specification does not follow the descript syntax."""


class ScheduleInterpretError(ScheduleError):
    """The specification is well formed but cannot describe a loop nest."""


class ScheduleValidationError(ScheduleError):
    """The loop nest is inconsistent (unused axis, tile order, sizes, ...)."""
