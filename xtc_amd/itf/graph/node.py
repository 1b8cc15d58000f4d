# SPDX-License-Identifier: BSD-3-Clause
"""Node interface (src/xtc/itf/graph/node.py)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from collections.abc import Sequence
from typing import TYPE_CHECKING, Any

if TYPE_CHECKING:
    from ..data.tensor import Tensor, TensorType
    from ..operator.operator import Operator
    from .operation import Operation

__all__ = ["Node"]


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
