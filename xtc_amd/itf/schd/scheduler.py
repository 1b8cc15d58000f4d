# SPDX-License-Identifier: BSD-3-Clause
"""Scheduler interface (src/xtc/itf/schd/scheduler.py:10-307).

Every transformation takes a loop `root` (default ".") and names loops by the
tile names the caller chose.  A tile size is the extent of the sub-loop; the
parent loop steps by it (src/xtc/backends/mlir/MlirCompilerPasses.py:414-457).
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from ...schedules.loop_nest import LoopNest
    from ..back.backend import Backend
    from .schedule import Schedule

DEFAULT_ROOT = "."


class Scheduler(ABC):
    @abstractmethod
    def schedule(self) -> "Schedule": ...

    @property
    @abstractmethod
    def backend(self) -> "Backend": ...

    @abstractmethod
    def set_dims(self, dims: list[str]) -> None:
        """Renames the operation's dimensions (same count, same order)."""

    @abstractmethod
    def split(self, dim: str, segments: dict[str, int], root: str = DEFAULT_ROOT) -> None:
        """Cuts `dim` into consecutive segments, each a new loop root."""

    def strip_mine(self, dim: str, tiles: dict[str, int], root: str = DEFAULT_ROOT) -> None:
        """Strip-mining without reordering; by default the same as `tile`."""
        self.tile(dim, tiles, root=root)

    @abstractmethod
    def tile(self, dim: str, tiles: dict[str, int], root: str = DEFAULT_ROOT) -> None:
        """Adds tile levels of `dim`, outer to inner: {name: extent}."""

    @abstractmethod
    def interchange(self, permutation: list[str], root: str = DEFAULT_ROOT) -> None: ...

    @abstractmethod
    def vectorize(self, axes: list[str], root: str = DEFAULT_ROOT) -> None: ...

    @abstractmethod
    def parallelize(self, axes: list[str], root: str = DEFAULT_ROOT) -> None: ...

    @abstractmethod
    def unroll(self, unrolls: dict[str, int], root: str = DEFAULT_ROOT) -> None: ...

    @abstractmethod
    def buffer_at(self, axis: str, mtype: str | None = None, root: str = DEFAULT_ROOT) -> None: ...

    @abstractmethod
    def pack_at(
        self,
        axis: str,
        input_idx: int,
        mtype: str | None = None,
        pad: bool = False,
        root: str = DEFAULT_ROOT,
    ) -> None: ...

    @abstractmethod
    def fuse_producer_at(self, axis: str, input_idx: int, root: str = DEFAULT_ROOT) -> None: ...

    @abstractmethod
    def define_memory_mesh(self, axes: dict[str, int]) -> None: ...

    @abstractmethod
    def define_processor_mesh(self, axes: dict[str, int]) -> None: ...

    @abstractmethod
    def distribute(self, axis: str, processor_axis: str, root: str = DEFAULT_ROOT) -> None: ...

    @abstractmethod
    def distributed_buffer_at(
        self,
        axis: str,
        input_idx: int,
        memory_axes: list[str],
        root: str = DEFAULT_ROOT,
    ) -> None: ...

    @abstractmethod
    def get_loop_nest(self) -> "LoopNest": ...
