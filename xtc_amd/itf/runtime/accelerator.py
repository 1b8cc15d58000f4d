# SPDX-License-Identifier: BSD-3-Clause
"""Accelerator device interface (src/xtc/itf/runtime/accelerator.py:12-135)."""

from __future__ import annotations

import ctypes
from abc import abstractmethod
from collections.abc import Callable
from typing import TYPE_CHECKING, Any

from .common import CommonRuntimeInterface

if TYPE_CHECKING:
    from ..comp.module import Module


class AcceleratorDevice(CommonRuntimeInterface):
    @abstractmethod
    def detect_accelerator(self) -> bool: ...

    @abstractmethod
    def init_device(self) -> None: ...

    @abstractmethod
    def deinit_device(self) -> None: ...

    @abstractmethod
    def load_module(self, module: "Module") -> None: ...

    @abstractmethod
    def get_module_function(self, module: "Module", function_name: str) -> Callable: ...

    @abstractmethod
    def unload_module(self, module: "Module") -> None: ...

    @abstractmethod
    def memory_allocate(self, size_bytes: int) -> Any: ...

    @abstractmethod
    def memory_free(self, handle: Any) -> None: ...

    @abstractmethod
    def memory_copy_to(self, acc_handle: Any, src: ctypes.c_void_p, size_bytes: int) -> None: ...

    @abstractmethod
    def memory_copy_from(self, acc_handle: Any, dst: ctypes.c_void_p, size_bytes: int) -> None: ...

    @abstractmethod
    def memory_fill_zero(self, acc_handle: Any, size_bytes: int) -> None: ...

    @abstractmethod
    def memory_data_pointer(self, acc_handle: Any) -> ctypes.c_void_p: ...
