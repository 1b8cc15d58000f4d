# SPDX-License-Identifier: BSD-3-Clause
"""Runtime interface shared by host and accelerator runtimes
(src/xtc/itf/runtime/common.py:11-210)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Any


class CommonRuntimeInterface(ABC):
    @abstractmethod
    def target_name(self) -> str: ...

    @abstractmethod
    def device_name(self) -> str: ...

    @abstractmethod
    def device_arch(self) -> str: ...

    @abstractmethod
    def device_id(self) -> int: ...

    @abstractmethod
    def evaluate(self, results: Any, repeat: int, number: int, nargs: int, cfunc: Any, args: Any) -> None:
        """Times `cfunc(*args)` without counters; fills `results[repeat]`."""

    @abstractmethod
    def evaluate_perf(
        self,
        pmu_events: list[str],
        repeat: int,
        number: int,
        min_repeat_ms: int,
        cfunc: Any,
        args: Any,
        nargs: int,
    ) -> list[float]:
        """Returns `repeat * max(1, len(pmu_events))` values: seconds per call,
        or per-call counter values when events are given."""

    @abstractmethod
    def evaluate_packed(
        self, results: Any, repeat: int, number: int, min_repeat_ms: int, cfunc: Any, args: Any, codes: Any, nargs: int
    ) -> None: ...

    @abstractmethod
    def evaluate_packed_perf(
        self,
        results: Any,
        pmu_events: list[str],
        repeat: int,
        number: int,
        min_repeat_ms: int,
        cfunc: Any,
        args: Any,
        codes: Any,
        nargs: int,
    ) -> None: ...

    @abstractmethod
    def cndarray_new(self, ndim: int, shape: Any, dtype: Any, device: Any) -> Any: ...

    @abstractmethod
    def cndarray_del(self, handle: Any) -> None: ...

    @abstractmethod
    def cndarray_copy_from_data(self, handle: Any, data_handle: Any) -> None: ...

    @abstractmethod
    def cndarray_copy_to_data(self, handle: Any, data_handle: Any) -> None: ...

    @abstractmethod
    def evaluate_flops(self, dtype_name: str | bytes) -> float:
        """Peak ops (FMA) per second for `dtype_name`."""
