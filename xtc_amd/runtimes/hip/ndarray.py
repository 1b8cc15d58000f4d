# SPDX-License-Identifier: BSD-3-Clause
"""Device-resident arrays of the HIP backend.

Plays the role of the reference's NDArray with a device runtime
(src/xtc/runtimes/types/ndarray.py:27-237): owns an HBM copy of a host
tensor, hands its bare pointer to payloads, and copies back on demand.
"bfloat16" arrays are float32 on the host and uint16 bit patterns on the
device (an extension: the reference has no bf16).

`layout` follows the reference's tensor layouts (ndarray.py:70-102): the
array keeps its logical shape, and with layout [1, 0] (2-D only) the device
holds the transpose, row-major.  copy_from / numpy take and return the
logical array.
"""

from __future__ import annotations

import ctypes
from typing import Any

import numpy as np

from ...utils.bf16 import bf16_bits_to_f32, f32_to_bf16_bits, host_dtype, is_bf16, itemsize
from .device import HipDevice

__all__ = ["DeviceArray"]


class DeviceArray:
    """An HBM buffer with a shape and an XTC dtype name."""

    def __init__(
        self, shape: tuple[int, ...], dtype: str, device: HipDevice | None = None, layout: list[int] | None = None
    ) -> None:
        self.device = device or HipDevice()
        self.shape = tuple(int(d) for d in shape)
        self.dtype = str(dtype)
        self.layout = None if layout is None or list(layout) == list(range(len(self.shape))) else list(layout)
        if self.layout is not None and (len(self.shape) != 2 or self.layout != [1, 0]):
            raise ValueError(f"layout {layout} is not supported (only [1, 0] on 2-D arrays)")
        self.size = int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1
        self.nbytes = self.size * itemsize(self.dtype)
        self.handle: int | None = self.device.memory_allocate(self.nbytes)

    @classmethod
    def from_numpy(
        cls,
        array: np.ndarray,
        dtype: str | None = None,
        device: HipDevice | None = None,
        layout: list[int] | None = None,
    ) -> "DeviceArray":
        dt = dtype or str(array.dtype)
        out = cls(array.shape, dt, device, layout)
        out.copy_from(array)
        return out

    @property
    def data(self) -> int:
        assert self.handle is not None, "freed array"
        return self.handle

    @property
    def c_ptr(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(self.data)

    def is_transposed(self) -> bool:
        return self.layout == [1, 0]

    def copy_from(self, array: np.ndarray) -> None:
        a = np.asarray(array)
        if a.shape != self.shape and a.size != self.size:
            raise ValueError(f"shape {a.shape} does not match device array {self.shape}")
        if self.is_transposed():
            a = np.ascontiguousarray(a.reshape(self.shape).T)
        if is_bf16(self.dtype):
            host = f32_to_bf16_bits(a.astype(np.float32)).reshape(-1)
        else:
            host = np.ascontiguousarray(a, dtype=host_dtype(self.dtype)).reshape(-1)
        self.device.memory_copy_to(self.data, host.ctypes.data_as(ctypes.c_void_p), self.nbytes)

    def numpy(self, out: np.ndarray | None = None) -> np.ndarray:
        """Host copy (float32 values for bf16 arrays)."""
        stored = self.shape[::-1] if self.is_transposed() else self.shape
        if is_bf16(self.dtype):
            raw = np.empty(self.size, np.uint16)
            self.device.memory_copy_from(self.data, raw.ctypes.data_as(ctypes.c_void_p), self.nbytes)
            host = bf16_bits_to_f32(raw).reshape(stored)
        else:
            host = np.empty(stored, host_dtype(self.dtype))
            self.device.memory_copy_from(self.data, host.ctypes.data_as(ctypes.c_void_p), self.nbytes)
        if self.is_transposed():
            host = np.ascontiguousarray(host.T)
        if out is not None:
            out[...] = host
            return out
        return host

    def fill_zero(self) -> None:
        self.device.memory_fill_zero(self.data, self.nbytes)

    def free(self) -> None:
        if self.handle is not None:
            self.device.memory_free(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass

    def __repr__(self) -> str:
        lay = f", layout={self.layout}" if self.layout is not None else ""
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype}{lay}, ptr={self.handle:#x})"

    def __array__(self, dtype: Any = None, copy: Any = None) -> np.ndarray:
        a = self.numpy()
        return a if dtype is None else a.astype(dtype)
