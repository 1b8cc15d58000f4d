# SPDX-License-Identifier: BSD-3-Clause
from .compiler import Compiler
from .module import Module

__all__ = ["Compiler", "Module"]
