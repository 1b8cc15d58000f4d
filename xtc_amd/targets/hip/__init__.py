# SPDX-License-Identifier: BSD-3-Clause
from .module import HipModule

__all__ = ["HipModule"]
