# SPDX-License-Identifier: BSD-3-Clause
"""Device buffers in HBM owned from Python, over the libxtc_hip C-ABI."""

from __future__ import annotations

import ctypes

import numpy as np

from . import capi

__all__ = ["DeviceBuffer", "ensure_device"]

_initialised: set[int] = set()


def ensure_device(device: int = 0) -> None:
    """Initialises `device` once (library stream, device selection)."""
    if device not in _initialised:
        capi.check(capi.lib().xtc_hip_init(device), "xtc_hip_init")
        _initialised.add(device)


class DeviceBuffer:
    """A dense byte buffer in device memory (xtc_hip_malloc / xtc_hip_free)."""

    def __init__(self, nbytes: int, device: int = 0) -> None:
        ensure_device(device)
        self.nbytes = int(nbytes)
        self.device = device
        ptr = capi.lib().xtc_hip_malloc(max(1, self.nbytes))
        if not ptr:
            raise capi.HipError(f"xtc_hip_malloc({self.nbytes}): {capi.last_error()}")
        self.ptr: int | None = int(ptr)

    @classmethod
    def from_numpy(cls, array: np.ndarray, device: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(array)
        buf = cls(a.nbytes, device)
        buf.copy_from(a)
        return buf

    def copy_from(self, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes, "host array larger than device buffer"
        capi.check(
            capi.lib().xtc_hip_memcpy_h2d(self.ptr, a.ctypes.data_as(ctypes.c_void_p), a.nbytes),
            "memcpy_h2d",
        )

    def to_numpy(self, shape: tuple[int, ...], dtype: object) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes, "requested view larger than device buffer"
        capi.check(
            capi.lib().xtc_hip_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), self.ptr, out.nbytes),
            "memcpy_d2h",
        )
        return out

    def zero(self) -> None:
        capi.check(capi.lib().xtc_hip_memset_zero(self.ptr, self.nbytes), "memset_zero")

    @property
    def c_ptr(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(self.ptr)

    def free(self) -> None:
        if self.ptr is not None:
            capi.lib().xtc_hip_free(self.ptr)
            self.ptr = None

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass
