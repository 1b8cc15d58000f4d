# SPDX-License-Identifier: BSD-3-Clause
"""`import xtc_amd.graphs.xtc.ty as T` (src/xtc/graphs/xtc/ty.py)."""

from .data import XTCTensor as Tensor  # noqa: F401
from .data import XTCTensorType as TensorType  # noqa: F401
