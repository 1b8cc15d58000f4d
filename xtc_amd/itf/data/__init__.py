# SPDX-License-Identifier: BSD-3-Clause
"""Data interfaces (src/xtc/itf/data/)."""

from .tensor import (
    ConstantDataType,
    ConstantShapeType,
    ConstantTensorType,
    DataType,
    ShapeType,
    Tensor,
    TensorType,
)

__all__ = ["ShapeType", "DataType", "ConstantShapeType", "ConstantDataType", "TensorType", "ConstantTensorType",
           "Tensor"]
