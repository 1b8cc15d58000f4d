# SPDX-License-Identifier: BSD-3-Clause
"""Evaluator and Executor interfaces (src/xtc/itf/exec/)."""

from .evaluator import Evaluator
from .executor import Executor

__all__ = ["Evaluator", "Executor"]
