# SPDX-License-Identifier: BSD-3-Clause
"""Operation interface (src/xtc/itf/graph/operation.py)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from collections.abc import Mapping, Sequence
from typing import TYPE_CHECKING, Any, TypeAlias

if TYPE_CHECKING:
    from ..data.tensor import TensorType

__all__ = ["Operation", "AccessesMaps"]

# (dims names, per-input index expressions, per-output index expressions)
AccessesMaps: TypeAlias = "tuple[tuple[str, ...], tuple[tuple[str, ...], ...], tuple[tuple[str, ...], ...]]"


class Operation(ABC):
    """The iteration space of one node: dims, their kinds and access maps.

    Kinds are "P" (parallel) and "R" (reduction).  `ops_count` is the product
    of the iteration space, one op per point (src/xtc/graphs/xtc/operation.py:76-82).
    """

    @property
    @abstractmethod
    def name(self) -> str: ...

    @property
    @abstractmethod
    def attrs(self) -> Mapping[str, Any]: ...

    @property
    @abstractmethod
    def inputs_types(self) -> Sequence["TensorType"]: ...

    @property
    @abstractmethod
    def outputs_types(self) -> Sequence["TensorType"]: ...

    @property
    @abstractmethod
    def dims(self) -> Mapping[str, int | str]: ...

    @abstractmethod
    def dims_kind(self, kind: str) -> Sequence[str]: ...

    @property
    @abstractmethod
    def accesses_maps(self) -> AccessesMaps: ...

    @property
    @abstractmethod
    def ops_count(self) -> int: ...

    @property
    @abstractmethod
    def ops_dtype(self) -> str: ...

    @property
    @abstractmethod
    def signature(self) -> list[Any]: ...
