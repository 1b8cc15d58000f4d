# SPDX-License-Identifier: BSD-3-Clause
from .backend import Backend

__all__ = ["Backend"]
