# SPDX-License-Identifier: BSD-3-Clause
"""Runtime value types (src/xtc/runtimes/types/)."""

from .ndarray import NDArray, NDArrayLocation

__all__ = ["NDArray", "NDArrayLocation"]
