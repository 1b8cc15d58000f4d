# SPDX-License-Identifier: BSD-3-Clause
from .schedule import Schedule
from .scheduler import DEFAULT_ROOT, Scheduler

__all__ = ["DEFAULT_ROOT", "Schedule", "Scheduler"]
