# SPDX-License-Identifier: BSD-3-Clause
"""Tensor and tensor-type interfaces (src/xtc/itf/data/tensor.py)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING, Any, TypeAlias

import numpy.typing

if TYPE_CHECKING:
    from ..runtime.accelerator import AcceleratorDevice

__all__ = [
    "ShapeType",
    "DataType",
    "ConstantShapeType",
    "ConstantDataType",
    "TensorType",
    "ConstantTensorType",
    "Tensor",
]

ShapeType: TypeAlias = "tuple[int | str | None, ...] | None"
DataType: TypeAlias = "str | None"
ConstantShapeType: TypeAlias = "tuple[int, ...]"
ConstantDataType: TypeAlias = str


class TensorType(ABC):
    @property
    @abstractmethod
    def shape(self) -> Any: ...

    @property
    @abstractmethod
    def dtype(self) -> Any: ...

    @property
    @abstractmethod
    def device(self) -> "AcceleratorDevice | None": ...

    @property
    @abstractmethod
    def const(self) -> bool: ...

    @property
    @abstractmethod
    def layout(self) -> list[int] | None: ...

    @property
    @abstractmethod
    def ndim(self) -> int: ...

    @abstractmethod
    def to_dict(self) -> dict[str, Any]: ...


class ConstantTensorType(TensorType):
    """A tensor type whose shape and dtype are fully known."""


class Tensor(ABC):
    @property
    @abstractmethod
    def type(self) -> TensorType: ...

    @property
    @abstractmethod
    def data(self) -> Any: ...

    @abstractmethod
    def numpy(self) -> numpy.typing.NDArray: ...
