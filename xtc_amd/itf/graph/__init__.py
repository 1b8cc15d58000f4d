# SPDX-License-Identifier: BSD-3-Clause
"""Graph, Node and Operation interfaces (src/xtc/itf/graph/*.py)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from collections.abc import Mapping, Sequence
from typing import TYPE_CHECKING, Any, TypeAlias

if TYPE_CHECKING:
    from ..data import Tensor, TensorType
    from ..operator import Operator

__all__ = ["Graph", "Node", "Operation", "AccessesMaps"]

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


class Node(ABC):
    @property
    @abstractmethod
    def uid(self) -> str: ...

    @property
    @abstractmethod
    def name(self) -> str: ...

    @property
    @abstractmethod
    def inputs(self) -> list[str]: ...

    @property
    @abstractmethod
    def outputs(self) -> list[str]: ...

    @property
    @abstractmethod
    def inputs_types(self) -> "Sequence[TensorType] | None": ...

    @property
    def outputs_types(self) -> "Sequence[TensorType] | None":
        return None

    @property
    @abstractmethod
    def preds(self) -> Sequence[str]: ...

    @property
    @abstractmethod
    def preds_nodes(self) -> Sequence["Node"]: ...

    @property
    @abstractmethod
    def operator(self) -> "Operator": ...

    @property
    @abstractmethod
    def operation(self) -> Operation: ...

    @abstractmethod
    def forward_types(self, inputs_types: Sequence["TensorType"]) -> Sequence["TensorType"]: ...

    @abstractmethod
    def forward(self, inputs: Sequence["Tensor"]) -> Sequence["Tensor"]: ...

    @abstractmethod
    def to_dict(self) -> dict[str, Any]: ...


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
