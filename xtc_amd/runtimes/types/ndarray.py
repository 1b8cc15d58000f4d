# SPDX-License-Identifier: BSD-3-Clause
"""NDArray: a tensor owned by the runtime (src/xtc/runtimes/types/ndarray.py:23-237).

Built from a numpy array, it holds an aligned host copy (the alignment set
by NDArray.set_alloc_alignment, 256 bytes by default; loop-explore's huge
pages ask for 2 MiB) and, when given an accelerator device as `runtime`
(xtc_amd.runtimes.hip.HipDevice), moves it to device memory: `data` is then
the device pointer that payloads take.  `layout` [1, 0] stores a 2-D array
transposed, and numpy() gives back the logical array.  The dtypes are the
reference's (signed and unsigned integers of 8 to 64 bits, float32,
float64).

The host copy is a numpy buffer whose first element sits on the alignment
boundary, where the reference allocates a DLPack tensor in its C runtime.
"""

from __future__ import annotations

import ctypes
from enum import Enum
from typing import Any

import numpy as np

from ...itf.runtime.accelerator import AcceleratorDevice

__all__ = ["NDArray", "NDArrayLocation"]


class NDArrayLocation(Enum):
    HOST = 0
    DEVICE = 1


class NDArray:
    DTYPES = ("int8", "int16", "int32", "int64", "uint8", "uint16", "uint32", "uint64", "float32", "float64")
    _alignment = 256

    def __init__(self, array: Any, runtime: Any = None, layout: list[int] | None = None) -> None:
        if isinstance(array, NDArray):
            raise RuntimeError("an NDArray is built from a numpy array, not from another NDArray")
        if not isinstance(array, np.ndarray):
            raise TypeError(f"NDArray takes a numpy array, not {type(array).__name__}")
        if str(array.dtype) not in self.DTYPES:
            raise ValueError(f"NDArray dtype {array.dtype} is not one of {self.DTYPES}")
        self.runtime = runtime
        self.layout = list(layout) if layout is not None else None
        if self.layout is not None and (len(self.layout) != 2 or sorted(self.layout) != [0, 1]):
            raise ValueError(f"only 2-D layouts are implemented: {self.layout}")
        if self.is_transposed() and array.ndim != 2:
            raise ValueError("layout [1, 0] needs a 2-D array")
        self._logical_shape = tuple(array.shape)
        stored = np.ascontiguousarray(array.T if self.is_transposed() else array)
        self._host = self._aligned_empty(stored.shape, stored.dtype)
        np.copyto(self._host, stored)
        self.location = NDArrayLocation.HOST
        self.device_handle: Any = None
        if isinstance(runtime, AcceleratorDevice):
            self._to_device()

    @classmethod
    def set_alloc_alignment(cls, alignment: int) -> None:
        """Alignment in bytes of the host copies made from now on (a power of two)."""
        if alignment < 1 or alignment & (alignment - 1):
            raise ValueError(f"alignment must be a power of two: {alignment}")
        cls._alignment = int(alignment)

    @classmethod
    def _aligned_empty(cls, shape: tuple[int, ...], dtype: np.dtype) -> np.ndarray:
        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize
        raw = np.empty(nbytes + cls._alignment, dtype=np.uint8)
        skip = (-raw.ctypes.data) % cls._alignment
        return raw[skip : skip + nbytes].view(dtype).reshape(shape)

    def _to_device(self) -> None:
        nbytes = self._host.nbytes
        self.device_handle = self.runtime.memory_allocate(nbytes)
        self.runtime.memory_copy_to(self.device_handle, self._host.ctypes.data_as(ctypes.c_void_p), nbytes)
        self.location = NDArrayLocation.DEVICE

    def is_on_device(self) -> bool:
        return self.location == NDArrayLocation.DEVICE

    def is_transposed(self) -> bool:
        return self.layout == [1, 0]

    @property
    def dtype_str(self) -> str:
        return str(self._host.dtype)

    @property
    def dtype(self) -> np.dtype:
        return self._host.dtype

    @property
    def dims(self) -> int:
        return len(self._logical_shape)

    @property
    def shape(self) -> tuple[int, ...]:
        """The stored shape: transposed under layout [1, 0], as the reference's."""
        return tuple(self._host.shape)

    @property
    def size(self) -> int:
        return int(self._host.size)

    @property
    def data(self) -> Any:
        """The device pointer once on the device, else the host address."""
        if self.is_on_device():
            return self.runtime.memory_data_pointer(self.device_handle)
        return self._host.ctypes.data

    def numpy(self, out: np.ndarray | None = None) -> np.ndarray:
        """The logical array, copied back from the device first when it lives
        there; `out` (not with a transposed layout) receives it in place."""
        if self.is_on_device():
            self.runtime.memory_copy_from(self.device_handle, self._host.ctypes.data_as(ctypes.c_void_p),
                                          self._host.nbytes)
        if out is not None:
            if self.is_transposed():
                raise ValueError("numpy(out=) of a transposed NDArray")
            if not out.flags["C_CONTIGUOUS"] or out.dtype != self.dtype or out.size != self.size:
                raise ValueError("out must be a C-contiguous array of the same dtype and size")
            np.copyto(out.reshape(self._host.shape), self._host)
            return out
        return np.ascontiguousarray(self._host.T if self.is_transposed() else self._host).copy()

    def copy_from_numpy(self, array: np.ndarray) -> None:
        """Overwrites the contents with the logical array `array` (same shape
        and dtype), on the device too when the NDArray lives there: how an
        evaluator hands a payload's outputs back to NDArray parameters."""
        array = np.asarray(array)
        if tuple(array.shape) != self._logical_shape or array.dtype != self.dtype:
            raise ValueError(f"expected {self._logical_shape} {self.dtype}, got {array.shape} {array.dtype}")
        np.copyto(self._host, array.T if self.is_transposed() else array)
        if self.is_on_device():
            self.runtime.memory_copy_to(self.device_handle, self._host.ctypes.data_as(ctypes.c_void_p),
                                        self._host.nbytes)

    def __del__(self) -> None:
        handle = getattr(self, "device_handle", None)
        if handle is not None and self.runtime is not None:
            try:
                self.runtime.memory_free(handle)
            except Exception:
                pass
            self.device_handle = None

    def __repr__(self) -> str:
        where = "device" if self.is_on_device() else "host"
        return f"NDArray(shape={self._logical_shape}, dtype={self.dtype_str}, {where})"
