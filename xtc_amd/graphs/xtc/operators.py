# SPDX-License-Identifier: BSD-3-Clause
"""Operators of the graph DSL with their numpy semantics.

Restates src/xtc/graphs/xtc/operators.py:159-804: shape/dtype inference
(`forward_types`), the numpy interpreter (`forward`, the reference the
Evaluator validates against) and the iteration space (`get_operation`, what
Schedulers and strategies see).  Attribute normalisation (padding, stride)
and dim names (matmul i,j,k; conv2d b,h,w,f,r,s,c; pad d0..dn) follow the
reference so that schedules and printed graphs carry over.

Extensions (no reference counterpart, marked as such): the `out_dtype`
attribute of matmul/conv2d (bf16 inputs with fp32 results) and the
`bias_add` operator.
"""

from __future__ import annotations

import hashlib
from collections.abc import Mapping, Sequence
from math import prod
from types import SimpleNamespace
from typing import Any

import numpy as np

from ...itf.data import Tensor, TensorType
from ...itf.operator import Operator
from ...utils.bf16 import host_dtype
from .data import XTCTensor, XTCTensorType
from .operation import XTCOperation

__all__ = [
    "XTCOperator",
    "XTCOperTensor",
    "XTCOperMatmul",
    "XTCOperRelu",
    "XTCOperConv2D",
    "XTCOperPad2D",
    "XTCOperPad",
    "XTCOperUnpad",
    "XTCOperReshape",
    "XTCOperTranspose",
    "XTCOperBiasAdd",
]


def _listify(obj: Any) -> Any:
    if isinstance(obj, dict):
        return {k: _listify(v) for k, v in obj.items()}
    if isinstance(obj, tuple):
        return [_listify(v) for v in obj]
    return obj


class XTCOperator(Operator):
    """Base operator: a name, a device and an ordered attribute namespace."""

    def __init__(self, name: str, device: Any = None, **attrs: Any) -> None:
        self._name = name
        self._device = device
        self._attrs = SimpleNamespace(**attrs)

    @property
    def name(self) -> str:
        return self._name

    @property
    def attrs(self) -> SimpleNamespace:
        return self._attrs

    @property
    def device(self) -> Any:
        return self._device

    def forward_types(self, inputs_types: Sequence[TensorType]) -> Sequence[XTCTensorType]:
        return list(inputs_types)  # type: ignore[arg-type]

    def forward(self, inputs: Sequence[Tensor]) -> Sequence[XTCTensor]:
        return list(inputs)  # type: ignore[arg-type]

    def _operation(
        self,
        inps_types: Sequence[XTCTensorType],
        outs_types: Sequence[XTCTensorType],
        dims: Mapping[str, int | str],
        kinds: Sequence[str],
        inps_maps: Sequence[Sequence[str]],
        outs_maps: Sequence[Sequence[str]],
    ) -> XTCOperation:
        return XTCOperation(
            name=self._name,
            attrs=vars(self._attrs),
            inputs_types=[t.constant for t in inps_types],
            outputs_types=[t.constant for t in outs_types],
            dims=dims,
            kinds=kinds,
            inps_maps=inps_maps,
            outs_maps=outs_maps,
        )

    def get_operation(
        self, inps_types: Sequence[XTCTensorType], outs_types: Sequence[XTCTensorType]
    ) -> XTCOperation:
        raise NotImplementedError(f"operator {self._name} has no iteration space")

    def to_dict(self) -> dict[str, Any]:
        return {"name": self._name, "attrs": {k: _listify(v) for k, v in vars(self._attrs).items()}}

    @classmethod
    def version_string(cls) -> str:
        """Digest of the registered operator classes (graph file compatibility)."""
        names = sorted(f"{c.__module__}.{c.__qualname__}" for c in cls.__subclasses__())
        return hashlib.sha256("|".join(names).encode()).hexdigest()[:16]

    def _check(self, out: XTCTensor, inputs: Sequence[Tensor]) -> XTCTensor:
        expected = self.forward_types([i.type for i in inputs])[0]
        if out.type != expected:
            raise AssertionError(f"{self._name}: output type {out.type} != expected {expected}")
        return out


class XTCOperTensor(XTCOperator):
    def __init__(self, **attrs: Any) -> None:
        super().__init__("tensor", **attrs)

    def get_operation(self, inps_types, outs_types) -> XTCOperation:  # type: ignore[override]
        return self._operation(inps_types, outs_types, {"i": outs_types[0].constant.size}, ("P",), (), (("i",),))


def _matmul_extents(a: tuple[int, ...], b: tuple[int, ...]) -> tuple[int, int, int]:
    """(i, j, k) with A viewed as (a0, prod(a1:)) and B as (prod(b:-1), b-1)."""
    i, k = a[0], prod(a[1:])
    kb, j = prod(b[:-1]), b[-1]
    if k != kb:
        raise ValueError(f"incompatible dimension k for matmul inputs shapes: ({i}, {k}) ({kb}, {j})")
    return i, j, k


def _out_dtype(op: XTCOperator, in_dtype: Any) -> Any:
    return getattr(op.attrs, "out_dtype", None) or in_dtype


class XTCOperMatmul(XTCOperator):
    """C[i,j] = sum_k A[i,k] * B[k,j] (operators.py:159-221)."""

    def __init__(self, **attrs: Any) -> None:
        super().__init__("matmul", **attrs)

    def get_operation(self, inps_types, outs_types) -> XTCOperation:  # type: ignore[override]
        i, j, k = _matmul_extents(inps_types[0].constant_shape, inps_types[1].constant_shape)
        return self._operation(
            inps_types,
            outs_types,
            {"i": i, "j": j, "k": k},
            ("P", "P", "R"),
            (("i", "k"), ("k", "j")),
            (("i", "j"),),
        )

    def forward_types(self, inputs_types):  # type: ignore[override]
        if len(inputs_types) != 2:
            raise ValueError("matmul takes two inputs")
        a = inputs_types[0].constant_shape
        b = inputs_types[1].constant_shape
        if len(a) < 2 or len(b) < 2:
            raise ValueError(f"matmul inputs must be at least 2-D: {a} {b}")
        i, j, _ = _matmul_extents(a, b)
        return [XTCTensorType(shape=(i, j), dtype=_out_dtype(self, inputs_types[0].dtype), device=self.device)]

    def forward(self, inputs):  # type: ignore[override]
        a = inputs[0].numpy()
        b = inputs[1].numpy()
        a = a.reshape((a.shape[0], -1))
        b = b.reshape((-1, b.shape[-1]))
        out_dtype = self.forward_types([i.type for i in inputs])[0].dtype
        return [self._check(XTCTensor(np.dot(a, b), dtype=out_dtype), inputs)]


class XTCOperRelu(XTCOperator):
    """max(x, threshold), threshold defaulting to 0 (operators.py:224-249)."""

    def __init__(self, **attrs: Any) -> None:
        super().__init__("relu", **attrs)
        self._threshold = attrs.get("threshold", 0)

    @property
    def threshold(self) -> float:
        return float(self._threshold)

    def get_operation(self, inps_types, outs_types) -> XTCOperation:  # type: ignore[override]
        n = prod(inps_types[0].constant_shape)
        return self._operation(inps_types, outs_types, {"i": n}, ("P",), (("i",),), (("i",),))

    def forward(self, inputs):  # type: ignore[override]
        x = inputs[0]
        return [XTCTensor(np.maximum(x.numpy(), self._threshold), dtype=x.type.dtype)]


def _pair(value: Any, what: str) -> tuple[int, int]:
    if isinstance(value, int):
        return (value, value)
    if isinstance(value, (tuple, list)) and len(value) == 1:
        return (int(value[0]), int(value[0]))
    if isinstance(value, (tuple, list)) and len(value) == 2:
        return (int(value[0]), int(value[1]))
    raise ValueError(f"{what} must be an int or a tuple of 1 or 2 ints: {value}")


class XTCOperConv2D(XTCOperator):
    """O[b,h,w,f] = sum_{r,s,c} I[b,h*SH+r,w*SW+s,c] * W[r,s,c,f].

    NHWC x RSCF -> NHWC, no implicit padding (operators.py:252-347); leading
    dims before H are flattened into b.
    """

    def __init__(self, **attrs: Any) -> None:
        super().__init__("conv2d", **attrs)
        self._stride = _pair(attrs.get("stride", 1), "stride")

    @property
    def stride(self) -> tuple[int, int]:
        return self._stride

    def _geometry(self, inp: tuple[int, ...], w: tuple[int, ...]) -> tuple[int, ...]:
        if len(inp) < 3 or len(w) != 4:
            raise ValueError(f"conv2d expects (...,H,W,C) and (R,S,C,F): {inp} {w}")
        h, wd, c = inp[-3:]
        r, s, wc, f = w
        if c != wc:
            raise ValueError(f"conv2d channel mismatch: input {inp}, weight {w}")
        sh, sw = self._stride
        oh, ow = (h - r) // sh + 1, (wd - s) // sw + 1
        return prod(inp[:-3]), oh, ow, f, r, s, c

    def get_operation(self, inps_types, outs_types) -> XTCOperation:  # type: ignore[override]
        b, oh, ow, f, r, s, c = self._geometry(inps_types[0].constant_shape, inps_types[1].constant_shape)
        sh, sw = self._stride
        return self._operation(
            inps_types,
            outs_types,
            {"b": b, "h": oh, "w": ow, "f": f, "r": r, "s": s, "c": c},
            ("P", "P", "P", "P", "R", "R", "R"),
            (("b", f"h*{sh}+r", f"w*{sw}+s", "c"), ("r", "s", "c", "f")),
            (("b", "h", "w", "f"),),
        )

    def forward_types(self, inputs_types):  # type: ignore[override]
        if len(inputs_types) != 2:
            raise ValueError("conv2d takes two inputs")
        inp = inputs_types[0].constant_shape
        _, oh, ow, f, _, _, _ = self._geometry(inp, inputs_types[1].constant_shape)
        return [
            XTCTensorType(
                shape=(*inp[:-3], oh, ow, f), dtype=_out_dtype(self, inputs_types[0].dtype), device=self.device
            )
        ]

    def forward(self, inputs):  # type: ignore[override]
        x = inputs[0].numpy()
        w = inputs[1].numpy()
        h, wd, c = x.shape[-3:]
        r, s, _, f = w.shape
        sh, sw = self._stride
        oh, ow = (h - r) // sh + 1, (wd - s) // sw + 1
        xb = x.reshape((-1, h, wd, c))
        # im2col in the input dtype, then one dot product per output pixel row
        cols = np.empty((xb.shape[0], oh, ow, r, s, c), dtype=x.dtype)
        for dr in range(r):
            for ds in range(s):
                cols[:, :, :, dr, ds, :] = xb[:, dr : dr + sh * (oh - 1) + 1 : sh, ds : ds + sw * (ow - 1) + 1 : sw, :]
        out = np.dot(cols.reshape((-1, r * s * c)), w.reshape((r * s * c, f)))
        out_dtype = self.forward_types([i.type for i in inputs])[0].dtype
        res = XTCTensor(out.reshape((*x.shape[:-3], oh, ow, f)), dtype=out_dtype)
        return [self._check(res, inputs)]


def _pad_per_axis(padding: Any, ndim: int) -> list[tuple[int, int]]:
    """(before, after) per axis of a normalised padding attribute."""
    if isinstance(padding, dict):
        pads = [(0, 0)] * ndim
        for axis, (lo, hi) in padding.items():
            if not -ndim <= axis < ndim:
                raise ValueError(f"pad axis {axis} out of range for rank {ndim}")
            pads[axis] = (int(lo), int(hi))
        return pads
    lo, hi = padding
    return [(int(lo), int(hi))] * ndim


class _PadSemantics:
    """Shared numpy semantics of pad/pad2d (operators.py:350-433)."""

    sign = 1

    def _pads(self, ndim: int) -> list[tuple[int, int]]:
        return _pad_per_axis(self.attrs.padding, ndim)  # type: ignore[attr-defined]

    def forward_types(self, inputs_types):  # type: ignore[no-untyped-def]
        if len(inputs_types) != 1:
            raise ValueError(f"{self.name} takes one input")  # type: ignore[attr-defined]
        shape = inputs_types[0].constant_shape
        if len(shape) < 2:
            raise ValueError(f"{self.name} needs rank >= 2")  # type: ignore[attr-defined]
        pads = self._pads(len(shape))
        out = tuple(d + self.sign * (lo + hi) for d, (lo, hi) in zip(shape, pads))
        return [XTCTensorType(shape=out, dtype=inputs_types[0].dtype, device=self.device)]  # type: ignore[attr-defined]

    def get_operation(self, inps_types, outs_types) -> XTCOperation:  # type: ignore[no-untyped-def]
        shape = inps_types[0].constant_shape
        pads = self._pads(len(shape))
        names = [f"d{i}" for i in range(len(shape))]
        extents = [d + self.sign * (lo + hi) for d, (lo, hi) in zip(shape, pads)]
        op = "-" if self.sign > 0 else "+"
        if isinstance(self.attrs.padding, dict):  # type: ignore[attr-defined]
            touched = {a % len(shape) for a in self.attrs.padding}  # type: ignore[attr-defined]
            inp = [f"{n}{op}{pads[i][0]}" if i in touched else n for i, n in enumerate(names)]
        else:
            inp = [f"{n}{op}{pads[0][0]}" for n in names]
        return self._operation(  # type: ignore[attr-defined]
            inps_types, outs_types, dict(zip(names, extents)), ("P",) * len(shape), (tuple(inp),), (tuple(names),)
        )


class XTCOperPad(_PadSemantics, XTCOperator):
    """Constant padding on any axes (operators.py:436-509).

    padding: int p (every axis (p,p)), a pair (lo,hi) (every axis), a
    sequence of per-trailing-axis ints/pairs, or {axis: int|pair}.
    """

    def __init__(self, **attrs: Any) -> None:
        padding = attrs.get("padding", 0)
        value = attrs.get("constant_value", 0)
        if not isinstance(value, (int, float)):
            raise ValueError("constant_value need to be a number")  # the reference's message (operators.py:461)
        if isinstance(padding, int):
            padding = (padding, padding)
        elif isinstance(padding, (tuple, list)) and len(padding) == 2 and all(isinstance(p, int) for p in padding):
            padding = tuple(padding)
        elif isinstance(padding, (tuple, list)):
            n = len(padding)
            padding = {i - n: (p, p) if isinstance(p, int) else tuple(p) for i, p in enumerate(padding)}
        elif isinstance(padding, dict):
            padding = {k: (v, v) if isinstance(v, (int, float)) else tuple(v) for k, v in padding.items()}
        else:
            raise ValueError("padding is either a list of tuple/int or int or a dict")
        if isinstance(padding, dict):
            padding = {k: v for k, v in padding.items() if v != (0, 0)}
        super().__init__("pad", device=attrs.get("device"), padding=padding, constant_value=value)

    def forward(self, inputs):  # type: ignore[override]
        x = inputs[0]
        pads = self._pads(x.numpy().ndim)
        out = np.pad(x.numpy(), pads, mode="constant", constant_values=self.attrs.constant_value)
        return [self._check(XTCTensor(out, dtype=x.type.dtype), inputs)]


class XTCOperPad2D(_PadSemantics, XTCOperator):
    """Constant padding of two axes, by default H and W of NHWC (operators.py:512-591).

    padding: int, (p,), (lo,hi) for both axes, ((lo,hi),(lo,hi)),
    (top,bottom,left,right) or {axis: int|pair}; axes default (-3, -2).
    """

    def __init__(self, **attrs: Any) -> None:
        padding = attrs.get("padding", (0, 0, 0, 0))
        value = attrs.get("constant_value", 0)
        axes = tuple(attrs.get("axes", (-3, -2)))
        # the error texts are the reference's assertion messages (operators.py:514-553)
        if len(axes) != 2:
            raise ValueError(f"axes for pad2d of wrong size, expected 2: {axes}")
        if axes[0] == axes[1]:
            raise ValueError(f"axes need 2 different dimension to pad: {axes}")
        if not isinstance(value, (int, float)):
            raise ValueError("constant_value need to be a number")
        if not isinstance(padding, (int, tuple, list, dict)):
            raise ValueError(f"padding for pad2d of wrong type, expect int or tuple or dict: {padding}")
        a0, a1 = axes
        if isinstance(padding, int):
            norm = {a0: (padding, padding), a1: (padding, padding)}
        elif isinstance(padding, dict):
            if len(padding) != 2:
                raise ValueError(f"padding for pad2d of wrong size, expected 1, 2 or 4: {padding}")
            norm = {k: (v, v) if isinstance(v, int) else tuple(v) for k, v in padding.items()}
        elif isinstance(padding, (tuple, list)) and len(padding) == 1:
            norm = {a0: (padding[0], padding[0]), a1: (padding[0], padding[0])}
        elif isinstance(padding, (tuple, list)) and len(padding) == 2 and all(isinstance(p, int) for p in padding):
            norm = {a0: (padding[0], padding[1]), a1: (padding[0], padding[1])}
        elif isinstance(padding, (tuple, list)) and len(padding) == 2:
            norm = {a0: tuple(padding[0]), a1: tuple(padding[1])}
        elif isinstance(padding, (tuple, list)) and len(padding) == 4:
            norm = {a0: (padding[0], padding[1]), a1: (padding[2], padding[3])}
        else:
            raise ValueError(f"padding for pad2d of wrong size, expected 1, 2 or 4: {padding}")
        norm = {k: v for k, v in norm.items() if v != (0, 0)}
        super().__init__("pad2d", device=attrs.get("device"), padding=norm, constant_value=value)

    def forward(self, inputs):  # type: ignore[override]
        x = inputs[0]
        pads = self._pads(x.numpy().ndim)
        out = np.pad(x.numpy(), pads, mode="constant", constant_values=self.attrs.constant_value)
        return [self._check(XTCTensor(out, dtype=x.type.dtype), inputs)]


class XTCOperUnpad(_PadSemantics, XTCOperator):
    """Crops what a pad added (operators.py:594-702)."""

    sign = -1

    def __init__(self, **attrs: Any) -> None:
        padding = attrs.get("padding", 0)
        if isinstance(padding, int):
            padding = (padding, padding)
        elif isinstance(padding, (tuple, list)) and len(padding) == 2 and all(isinstance(p, int) for p in padding):
            padding = tuple(padding)
        elif isinstance(padding, (tuple, list)):
            n = len(padding)
            padding = {i - n: (p, p) if isinstance(p, int) else tuple(p) for i, p in enumerate(padding)}
        elif isinstance(padding, dict):
            padding = {k: (v, v) if isinstance(v, (int, float)) else tuple(v) for k, v in padding.items()}
        else:
            raise ValueError("padding is an int, a pair, a sequence or a dict")
        if isinstance(padding, dict):
            padding = {k: v for k, v in padding.items() if v != (0, 0)}
        super().__init__("unpad", padding=padding)

    def forward(self, inputs):  # type: ignore[override]
        x = inputs[0].numpy()
        pads = self._pads(x.ndim)
        view = x[tuple(slice(lo, d - hi) for d, (lo, hi) in zip(x.shape, pads))]
        return [self._check(XTCTensor(view, dtype=inputs[0].type.dtype), inputs)]


class XTCOperReshape(XTCOperator):
    """Reshape with at most one -1 (operators.py:693-745)."""

    def __init__(self, **attrs: Any) -> None:
        super().__init__("reshape", **attrs)
        self._shape = tuple(attrs.get("shape", (-1,)))
        if sum(1 for d in self._shape if d == -1) > 1:
            raise ValueError("reshape accepts at most one -1")

    def get_operation(self, inps_types, outs_types) -> XTCOperation:  # type: ignore[override]
        n = prod(inps_types[0].constant_shape)
        return self._operation(inps_types, outs_types, {"i": n}, ("P",), (("i",),), (("i",),))

    def forward_types(self, inputs_types):  # type: ignore[override]
        size = prod(inputs_types[0].constant_shape)
        known = prod(d for d in self._shape if d != -1)
        shape = tuple(size // known if d == -1 else d for d in self._shape)
        if prod(shape) != size:
            raise ValueError(f"cannot reshape {inputs_types[0].constant_shape} to {self._shape}")
        return [XTCTensorType(shape=shape, dtype=inputs_types[0].dtype, device=self.device)]

    def forward(self, inputs):  # type: ignore[override]
        out = XTCTensor(inputs[0].numpy().reshape(self._shape), dtype=inputs[0].type.dtype)
        return [self._check(out, inputs)]


class XTCOperTranspose(XTCOperator):
    """Axis permutation, reversed by default (operators.py:748-804)."""

    def __init__(self, **attrs: Any) -> None:
        super().__init__("transpose", axes=tuple(attrs.get("axes", ())))

    def forward_types(self, inputs_types):  # type: ignore[override]
        shape = inputs_types[0].constant_shape
        axes = self.attrs.axes or tuple(range(len(shape)))[::-1]
        if len(axes) != len(shape):
            raise ValueError(f"transpose axes {axes} do not match rank {len(shape)}")
        return [XTCTensorType(shape=tuple(shape[a] for a in axes), dtype=inputs_types[0].dtype, device=self.device)]

    def forward(self, inputs):  # type: ignore[override]
        x = inputs[0]
        out = XTCTensor(x.numpy().transpose(self.attrs.axes or None), dtype=x.type.dtype)
        return [self._check(out, inputs)]

    def get_operation(self, inps_types, outs_types) -> XTCOperation:  # type: ignore[override]
        n = prod(inps_types[0].constant_shape)
        return self._operation(inps_types, outs_types, {"i": n}, ("P",), (("i",),), (("i",),))


class XTCOperBiasAdd(XTCOperator):
    """Extension (no reference operator): out[..., f] = x[..., f] + bias[f].

    The bias broadcasts over every axis but the last; the HIP backend fuses it
    into the epilogue of the matmul/conv2d producing x.
    """

    def __init__(self, **attrs: Any) -> None:
        super().__init__("bias_add", **attrs)

    def forward_types(self, inputs_types):  # type: ignore[override]
        x, b = inputs_types[0].constant_shape, inputs_types[1].constant_shape
        if len(b) != 1 or b[0] != x[-1]:
            raise ValueError(f"bias_add: bias {b} does not match last axis of {x}")
        return [XTCTensorType(shape=x, dtype=inputs_types[0].dtype, device=self.device)]

    def get_operation(self, inps_types, outs_types) -> XTCOperation:  # type: ignore[override]
        x = inps_types[0].constant_shape
        rows = prod(x[:-1])
        return self._operation(
            inps_types, outs_types, {"i": rows, "j": x[-1]}, ("P", "P"), (("i", "j"), ("j",)), (("i", "j"),)
        )

    def forward(self, inputs):  # type: ignore[override]
        x, b = inputs[0], inputs[1]
        dt = host_dtype(x.type.dtype)
        out = XTCTensor((x.numpy() + b.numpy()).astype(dt), dtype=x.type.dtype)
        return [self._check(out, inputs)]
