# SPDX-License-Identifier: BSD-3-Clause
"""Graph interface (src/xtc/itf/graph/graph.py)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from collections.abc import Mapping, Sequence
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from ..data.tensor import Tensor, TensorType
    from .node import Node

__all__ = ["Graph"]


class Graph(ABC):
    @property
    @abstractmethod
    def name(self) -> str: ...

    @property
    @abstractmethod
    def nodes(self) -> Mapping[str, Node]: ...

    @property
    @abstractmethod
    def inputs(self) -> Sequence[str]: ...

    @property
    @abstractmethod
    def outputs(self) -> Sequence[str]: ...

    @property
    @abstractmethod
    def inputs_types(self) -> "Sequence[TensorType] | None": ...

    @property
    def outputs_types(self) -> "Sequence[TensorType] | None":
        return None

    @property
    @abstractmethod
    def inputs_nodes(self) -> Sequence[Node]: ...

    @property
    @abstractmethod
    def outputs_nodes(self) -> Sequence[Node]: ...

    @abstractmethod
    def forward_types(self, inputs_types: Sequence["TensorType"]) -> Sequence["TensorType"]: ...

    @abstractmethod
    def forward(self, inputs: Sequence["Tensor"]) -> Sequence["Tensor"]: ...

    @abstractmethod
    def ops_count(self) -> int: ...

    @abstractmethod
    def ops_dtype(self) -> str: ...
