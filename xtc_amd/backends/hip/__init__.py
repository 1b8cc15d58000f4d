# SPDX-License-Identifier: BSD-3-Clause
"""`from xtc_amd.backends.hip import Backend` -- the MI355X backend, under the
name XTC's explorer expects (`xtc.backends.<name>.Backend`,
src/xtc/search/explore.py:262-268)."""

from .backend import HipBackend
from .scheduler import HipSchedule, HipScheduler, ScheduleError

Backend = HipBackend

__all__ = ["Backend", "HipBackend", "HipScheduler", "HipSchedule", "ScheduleError"]
