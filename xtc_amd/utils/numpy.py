# SPDX-License-Identifier: BSD-3-Clause
"""Default evaluation inputs (src/xtc/utils/numpy.py:12-19)."""

from __future__ import annotations

from typing import Any, Sequence

import numpy as np

from .bf16 import host_dtype

__all__ = ["np_init"]


def np_init(shape: Sequence[int], dtype: str) -> np.ndarray[Any, Any]:
    """Integers 1..9 repeating in C order, as `dtype`.

    Such inputs keep every matmul/conv partial sum an exact integer in fp32
    while 81*K < 2**24, so results do not depend on summation order.
    "bfloat16" tensors are held on the host as float32 arrays of
    bf16-representable values (1..9 are exact).
    """
    n = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    vals = np.arange(n, dtype=np.int64) % 9 + 1
    return vals.reshape(tuple(shape)).astype(host_dtype(dtype))
