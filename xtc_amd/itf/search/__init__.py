# SPDX-License-Identifier: BSD-3-Clause
"""Strategy and Optimizer interfaces (src/xtc/itf/search/)."""

from .optimizer import Optimizer, VecSample
from .strategy import Sample, Strategy

__all__ = ["Sample", "VecSample", "Strategy", "Optimizer"]
