# SPDX-License-Identifier: BSD-3-Clause
"""bfloat16 storage helpers for numpy (numpy has no native bf16).

Graphs name the dtype "bfloat16".  On the host such a tensor is a float32
array whose values are bf16-representable; it becomes uint16 bit patterns
only when copied to the device.  The reference has no bf16 type (its numpy
dtype map stops at float64, src/xtc/runtimes/types/ndarray.py:28-39), so this
is an extension.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "BF16",
    "f32_to_bf16_bits",
    "bf16_bits_to_f32",
    "round_to_bf16",
    "is_bf16",
    "host_dtype",
    "itemsize",
]

BF16 = "bfloat16"


def is_bf16(dtype: object) -> bool:
    return str(dtype) == BF16


def host_dtype(dtype: object) -> np.dtype:
    """numpy dtype used on the host for a graph dtype."""
    return np.dtype(np.float32) if is_bf16(dtype) else np.dtype(str(dtype))


def itemsize(dtype: object) -> int:
    """Bytes per element on the device."""
    return 2 if is_bf16(dtype) else np.dtype(str(dtype)).itemsize


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16).

    NaNs stay NaNs (quiet bit set); infinities and overflow to infinity
    follow IEEE rounding.
    """
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    quiet = ((u >> 16) | 0x40).astype(np.uint16)
    return np.where(nan, quiet, rounded).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """Exact bf16 (uint16 bit patterns) -> float32."""
    u = np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16
    return u.view(np.float32)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
