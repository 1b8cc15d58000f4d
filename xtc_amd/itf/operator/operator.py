# SPDX-License-Identifier: BSD-3-Clause
"""Operator interface (src/xtc/itf/operator/operator.py)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from collections.abc import Sequence
from typing import TYPE_CHECKING, Any

if TYPE_CHECKING:
    from ..data.tensor import Tensor, TensorType

__all__ = ["Operator"]


class Operator(ABC):
    @property
    @abstractmethod
    def name(self) -> str: ...

    @abstractmethod
    def forward_types(self, inputs_types: Sequence["TensorType"]) -> Sequence["TensorType"]: ...

    @abstractmethod
    def forward(self, inputs: Sequence["Tensor"]) -> Sequence["Tensor"]: ...

    @abstractmethod
    def to_dict(self) -> dict[str, Any]: ...
