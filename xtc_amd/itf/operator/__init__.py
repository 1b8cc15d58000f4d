# SPDX-License-Identifier: BSD-3-Clause
"""Operator interface (src/xtc/itf/operator/)."""

from .operator import Operator

__all__ = ["Operator"]
