# SPDX-License-Identifier: BSD-3-Clause
"""Tensor types and host tensors of the graph DSL (src/xtc/graphs/xtc/data.py).

Printed forms (`5x3xfloat32`, `Tensor(type=..., data=a b c d...w x y z)`) are
part of the interface: the reference's own golden tests match them
(tests/filecheck/graphs/test_matmul.py:41-42).
"""

from __future__ import annotations

from math import prod
from typing import Any, Iterable

import numpy as np
import numpy.typing

from ...itf.data import ConstantTensorType, Tensor, TensorType
from ...utils.bf16 import host_dtype, is_bf16, itemsize, round_to_bf16

__all__ = ["XTCTensorType", "XTCConstantTensorType", "XTCTensor"]


class XTCTensorType(TensorType):
    """Shape/dtype/device/layout of a tensor; shape or dtype may be unknown."""

    def __init__(
        self,
        shape: Any = None,
        dtype: str | None = None,
        device: Any = None,
        const: bool = False,
        layout: list[int] | None = None,
    ) -> None:
        self._shape = None if shape is None else tuple(shape)
        self._dtype = dtype
        self._device = device
        self._const = const
        self._layout = layout

    @property
    def shape(self) -> Any:
        return self._shape

    @property
    def dtype(self) -> str | None:
        return self._dtype

    @property
    def device(self) -> Any:
        return self._device

    @property
    def const(self) -> bool:
        return self._const

    @property
    def layout(self) -> list[int] | None:
        return self._layout

    @property
    def ndim(self) -> int:
        return 0 if self._shape is None else len(self._shape)

    def is_constant_shape(self) -> bool:
        return self._shape is not None and all(isinstance(d, int) for d in self._shape)

    def is_constant_dtype(self) -> bool:
        return self._dtype is not None

    def is_constant(self) -> bool:
        return self.is_constant_shape() and self.is_constant_dtype()

    @property
    def size(self) -> int:
        if self._shape is None:
            return 0
        assert self.is_constant_shape(), "symbolic shapes are not supported"
        return prod(self._shape)

    @property
    def itemsize(self) -> int:
        assert self.is_constant_dtype(), "symbolic dtypes are not supported"
        return itemsize(self._dtype)

    @property
    def nbytes(self) -> int:
        return self.size * self.itemsize

    @property
    def constant_shape(self) -> tuple[int, ...]:
        assert self.is_constant_shape(), f"shape is not constant: {self._shape}"
        return tuple(int(d) for d in self._shape)  # type: ignore[union-attr]

    @property
    def constant_dtype(self) -> str:
        assert self.is_constant_dtype(), "dtype is not constant"
        return str(self._dtype)

    @property
    def constant(self) -> "XTCConstantTensorType":
        return XTCConstantTensorType(
            shape=self.constant_shape,
            dtype=self.constant_dtype,
            device=self._device,
            const=self._const,
            layout=self._layout,
        )

    def __repr__(self) -> str:
        dims = "??" if self._shape is None else "x".join(str(d) if d else "?" for d in self._shape)
        text = f"{dims}x{self._dtype if self._dtype else '?'}"
        if self._const:
            text += ", const"
        if self._layout is not None:
            ident = ",".join(str(i) for i in range(len(self._shape or ())))
            perm = ",".join(str(i) for i in self._layout)
            text += f", <({ident})->({perm})>"
        return text

    def __eq__(self, other: object) -> bool:
        if not isinstance(other, XTCTensorType):
            return NotImplemented
        return (
            self._shape == other._shape
            and self._dtype == other._dtype
            and self._const == other._const
            and self._layout == other._layout
        )

    def __hash__(self) -> int:
        return hash((self._shape, self._dtype, self._const))

    def to_dict(self) -> dict[str, Any]:
        out: dict[str, Any] = {}
        if self._shape:
            out["shape"] = list(self._shape)
        if self._dtype:
            out["dtype"] = self._dtype
        return out

    @classmethod
    def from_dict(cls, spec: dict[str, Any]) -> "XTCTensorType":
        shape = spec.get("shape")
        return cls(shape=None if shape is None else tuple(shape), dtype=spec.get("dtype"))


class XTCConstantTensorType(XTCTensorType, ConstantTensorType):
    """Tensor type with a known shape and dtype."""

    @property
    def shape(self) -> tuple[int, ...]:
        return self._shape  # type: ignore[return-value]

    @property
    def dtype(self) -> str:
        return str(self._dtype)


def _short(values: Iterable[Any], fmt: str) -> str:
    return " ".join(format(v, fmt) for v in values)


class XTCTensor(Tensor):
    """A host tensor: a numpy array plus its XTC type.

    For "bfloat16" the array is float32 holding bf16-representable values.
    """

    def __init__(self, data: Any | None = None, type: XTCTensorType | None = None, dtype: str | None = None) -> None:
        if data is None:
            self._data = None
            self._type = type if type is not None else XTCTensorType()
            return
        arr = np.array(data)
        if dtype is None and type is not None and type.dtype is not None:
            dtype = type.dtype
        if dtype is not None and is_bf16(dtype):
            arr = round_to_bf16(arr.astype(np.float32))
        elif dtype is not None:
            arr = arr.astype(host_dtype(dtype))
        self._data = arr
        self._type = XTCTensorType(arr.shape, dtype if dtype is not None else str(arr.dtype))

    @property
    def type(self) -> XTCTensorType:
        return self._type

    @property
    def data(self) -> Any:
        return self._data

    def numpy(self) -> numpy.typing.NDArray:
        assert self._data is not None, "tensor has no data"
        return np.array(self._data)

    def __repr__(self) -> str:
        if self._data is None:
            return f"Tensor(type={self._type}, data=None)"
        flat = self._data.reshape(-1)
        if flat.size > 8:
            text = f"{_short(flat[:4], '.4g')}...{_short(flat[-4:], '.4g')}"
        else:
            text = _short(flat, "g")
        return f"Tensor(type={self._type}, data={text})"
