# SPDX-License-Identifier: BSD-3-Clause
"""Iteration-space description of a node (src/xtc/graphs/xtc/operation.py:17-99)."""

from __future__ import annotations

import json
from collections.abc import Mapping, Sequence
from math import prod
from typing import Any

from ...itf.graph import AccessesMaps, Operation
from .data import XTCTensorType

__all__ = ["XTCOperation"]


class XTCOperation(Operation):
    """Dims (ordered name -> extent), their kinds ("P"/"R") and access maps."""

    def __init__(
        self,
        name: str,
        attrs: Mapping[str, Any],
        inputs_types: Sequence[XTCTensorType],
        outputs_types: Sequence[XTCTensorType],
        dims: Mapping[str, int | str],
        kinds: Sequence[str],
        inps_maps: Sequence[Sequence[str]],
        outs_maps: Sequence[Sequence[str]],
    ) -> None:
        if len(dims) != len(kinds):
            raise ValueError(f"{name}: {len(dims)} dims but {len(kinds)} kinds")
        self._name = name
        self._attrs = dict(attrs)
        self._inputs_types = tuple(inputs_types)
        self._outputs_types = tuple(outputs_types)
        self._dims = dict(dims)
        self._kinds = tuple(kinds)
        self._maps: AccessesMaps = (
            tuple(self._dims),
            tuple(tuple(m) for m in inps_maps),
            tuple(tuple(m) for m in outs_maps),
        )

    @property
    def name(self) -> str:
        return self._name

    @property
    def attrs(self) -> Mapping[str, Any]:
        return self._attrs

    @property
    def inputs_types(self) -> Sequence[XTCTensorType]:
        return self._inputs_types

    @property
    def outputs_types(self) -> Sequence[XTCTensorType]:
        return self._outputs_types

    @property
    def dims(self) -> Mapping[str, int | str]:
        return self._dims

    def dims_kind(self, kind: str) -> Sequence[str]:
        return [d for d, k in zip(self._dims, self._kinds) if k == kind]

    @property
    def accesses_maps(self) -> AccessesMaps:
        return self._maps

    @property
    def ops_count(self) -> int:
        """One op per point of the iteration space (an FMA for matmul/conv)."""
        extents = list(self._dims.values())
        if not all(isinstance(d, int) for d in extents):
            raise ValueError(f"{self._name}: symbolic dims {extents}")
        return prod(int(d) for d in extents)

    @property
    def ops_dtype(self) -> str:
        """dtype of the operation's arithmetic.  The reference takes the
        first output's (src/xtc/graphs/xtc/operation.py:86-89), where inputs
        and outputs share it.  Under the out_dtype extension (bfloat16
        operands, float32 result) the arithmetic is the operands', so the
        first input's dtype is taken when there is one: the same value for
        every graph the reference builds."""
        if self._inputs_types:
            return self._inputs_types[0].constant_dtype
        return self._outputs_types[0].constant_dtype

    @property
    def signature(self) -> list[Any]:
        return json.loads(json.dumps([self._name, list(self._dims.values()), self.ops_dtype, self._attrs]))
