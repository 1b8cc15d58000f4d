# SPDX-License-Identifier: BSD-3-Clause
"""Graph -> kernel-launch plan of the HIP backend.

Every operator node of an XTC graph becomes one launch of a hand-written
gfx950 kernel, except where the producer/consumer pattern lets a kernel
absorb its neighbour (the MI355X design choice: keep intermediates out of
HBM):
  * pad2d/pad on H and W feeding conv2d input 0 -> folded into the
    implicit-GEMM loader (out-of-window taps read `constant_value`);
  * bias_add on a matmul/conv2d result -> GEMM epilogue;
  * relu on a matmul/conv2d(/bias_add) result -> GEMM epilogue.
A fusion happens only when the intermediate is used once and is not a graph
output.  A matmul operand with layout [1, 0] (stored transposed) becomes the
launch's trans_a / trans_b flag; other operators require natural layouts.  reshape is a view; unpad
is a crop kernel (16-byte row copies when the innermost dim is kept).  The reference lowers each node to its own
linalg op (src/xtc/backends/mlir/MlirOps.py:166-887) and fuses only through
transform-dialect producer fusion (MlirCompilerPasses.py:378-412).

The plan uses only the graph interfaces (nodes, operation, inputs/outputs,
types), so it accepts any Graph that follows xtc.itf.graph.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from math import prod
from typing import Any

from ...utils.bf16 import is_bf16, itemsize

__all__ = ["Buffer", "Launch", "Plan", "lower_graph", "UnsupportedGraph"]

F32 = "float32"
BF16 = "bfloat16"
F64 = "float64"


class UnsupportedGraph(ValueError):
    """The graph uses an operator or dtype the HIP backend does not run."""


@dataclass
class Buffer:
    """A tensor of the plan: a payload argument or a workspace slice."""

    uid: str
    shape: tuple[int, ...]
    dtype: str
    kind: str  # "input" | "output" | "temp" | "alias"
    arg_index: int = -1  # payload argument position for inputs/outputs
    offset: int = 0  # byte offset in the workspace for temps
    alias_of: str | None = None

    @property
    def nbytes(self) -> int:
        return prod(self.shape) * itemsize(self.dtype)


@dataclass
class Launch:
    """One kernel launch.  `node` is the scheduled node the launch serves
    (the matmul/conv2d for fused GEMMs); `absorbed` lists fused nodes."""

    kind: str  # "matmul" | "conv2d" | "relu" | "pad" | "unpad" | "copy" | "cast"
    node: str
    inputs: list[str]
    output: str
    attrs: dict[str, Any] = field(default_factory=dict)
    absorbed: list[str] = field(default_factory=list)


@dataclass
class Plan:
    name: str
    buffers: dict[str, Buffer]
    launches: list[Launch]
    args: list[str]  # payload argument uids: graph inputs then outputs
    workspace_bytes: int
    scheduled: dict[str, Any]  # node name -> graph node, for scheduled launches

    def buffer(self, uid: str) -> Buffer:
        b = self.buffers[uid]
        while b.alias_of is not None:
            b = self.buffers[b.alias_of]
        return b


def _shape(t: Any) -> tuple[int, ...]:
    return tuple(int(d) for d in t.constant_shape) if hasattr(t, "constant_shape") else tuple(int(d) for d in t.shape)


def _dtype(t: Any) -> str:
    return str(t.dtype)


def _pad_hw(node: Any, rank: int) -> tuple[int, int, int, int] | None:
    """(top, bottom, left, right) if the pad only touches axes H, W of NHWC."""
    padding = node.operation.attrs.get("padding")
    if isinstance(padding, dict):
        per = {a % rank: tuple(v) for a, v in padding.items()}
    else:
        per = {a: tuple(padding) for a in range(rank)}
    per = {a: v for a, v in per.items() if tuple(v) != (0, 0)}
    if any(a not in (rank - 3, rank - 2) for a in per):
        return None
    top, bottom = per.get(rank - 3, (0, 0))
    left, right = per.get(rank - 2, (0, 0))
    return int(top), int(bottom), int(left), int(right)


def lower_graph(graph: Any) -> Plan:
    nodes = graph.nodes  # uid -> node, any itf Graph
    inputs = list(graph.inputs)
    outputs = list(graph.outputs)
    if graph.outputs_types is None:
        raise UnsupportedGraph("graph types are not known: call graph.forward_types() first")

    op_nodes = [n for uid, n in nodes.items() if uid not in inputs]
    users: dict[str, list[Any]] = {}
    for n in op_nodes:
        for u in n.inputs:
            users.setdefault(u, []).append(n)

    def out_type(uid: str) -> Any:
        if uid in inputs:
            return graph.inputs_types[inputs.index(uid)]
        return nodes[uid].outputs_types[0]

    def drop_temp(uid: str) -> None:
        b = buffers.get(uid)
        if b is not None and b.kind == "temp":
            del buffers[uid]

    def single_internal_use(uid: str) -> Any | None:
        us = users.get(uid, [])
        if len(us) == 1 and uid not in outputs:
            return us[0]
        return None

    buffers: dict[str, Buffer] = {}
    for idx, uid in enumerate(inputs):
        t = out_type(uid)
        buffers[uid] = Buffer(uid, _shape(t), _dtype(t), "input", arg_index=idx)
    for idx, uid in enumerate(outputs):
        if uid in buffers:
            raise UnsupportedGraph(f"graph input {uid} is also an output")
        t = out_type(uid)
        buffers[uid] = Buffer(uid, _shape(t), _dtype(t), "output", arg_index=len(inputs) + idx)

    absorbed: set[str] = set()
    launches: list[Launch] = []
    scheduled: dict[str, Any] = {}

    # Nodes in a topological order: graph.nodes may hold them in build order.
    order: list[Any] = []
    seen: set[str] = set(inputs)

    def visit(n: Any) -> None:
        stack = [(n, False)]
        while stack:
            cur, done = stack.pop()
            if done:
                order.append(cur)
                continue
            if cur.uid in seen:
                continue
            seen.add(cur.uid)
            stack.append((cur, True))
            for u in reversed(cur.inputs):
                if u not in seen and u in nodes:
                    stack.append((nodes[u], False))

    for n in op_nodes:
        visit(n)

    # pad producers folded into the conv2d loader, decided before any launch
    pad_fusion: dict[str, tuple[Any, tuple[int, int, int, int]]] = {}
    for n in order:
        if n.operation.name != "conv2d" or n.inputs[0] in inputs:
            continue
        pad_node = nodes[n.inputs[0]]
        if pad_node.operation.name not in ("pad2d", "pad") or single_internal_use(pad_node.uid) is not n:
            continue
        rank = len(_shape(out_type(pad_node.inputs[0])))
        hw = _pad_hw(pad_node, rank) if rank >= 3 else None
        if hw is not None:
            pad_fusion[n.uid] = (pad_node, hw)
            absorbed.add(pad_node.uid)

    def transposed_inputs(n: Any) -> tuple[bool, ...]:
        """Per input: stored transposed (layout [1, 0]).  Only the two 2-D
        operands of a matmul may be (MlirOps.py:171-178); other operators
        need natural layouts, as in the reference (MlirOps.py:45-52)."""
        flags = []
        for idx, u in enumerate(n.inputs):
            t = out_type(u)
            lay = getattr(t, "layout", None)
            shp = _shape(t)
            if lay is None or list(lay) == list(range(len(shp))):
                flags.append(False)
            elif n.operation.name == "matmul" and idx < 2 and len(shp) == 2 and list(lay) == [1, 0]:
                flags.append(True)
            else:
                raise UnsupportedGraph(
                    f"{n.operation.name} {n.name}: tensor layout {list(lay)} of input {idx} is not supported "
                    "(only [1, 0] on a 2-D matmul operand)"
                )
        return tuple(flags)

    for n in order:
        trans = transposed_inputs(n)  # also checks the nodes a kernel absorbs
        if n.uid in absorbed:
            continue
        op = n.operation
        name = op.name
        t_out = n.outputs_types[0]
        if n.uid not in buffers:
            buffers[n.uid] = Buffer(n.uid, _shape(t_out), _dtype(t_out), "temp")
        if name in ("matmul", "conv2d"):
            in_dt = {_dtype(out_type(u)) for u in n.inputs}
            if len(in_dt) != 1 or not in_dt <= {F32, BF16, F64}:
                raise UnsupportedGraph(
                    f"{name} {n.name}: inputs must both be float32, float64 or bfloat16, got {in_dt}")
            attrs: dict[str, Any] = {"dtype": in_dt.pop(), "relu": False, "threshold": 0.0, "bias": None}
            fused: list[str] = []
            src_inputs = list(n.inputs)
            if name == "matmul":
                i, j, k = (int(op.dims[d]) for d in ("i", "j", "k"))
                attrs.update(M=i, N=j, K=k, trans_a=trans[0], trans_b=trans[1])
            else:
                pads = (0, 0, 0, 0)
                pad_value = 0.0
                if n.uid in pad_fusion:
                    pad_node, pads = pad_fusion[n.uid]
                    pad_value = float(pad_node.operation.attrs.get("constant_value", 0))
                    src_inputs[0] = pad_node.inputs[0]
                    fused.append(pad_node.name)
                ishape = _shape(out_type(src_inputs[0]))
                r, s, c, f = _shape(out_type(n.inputs[1]))
                stride = op.attrs.get("stride", 1)
                sh, sw = (stride, stride) if isinstance(stride, int) else (tuple(stride) * 2)[:2]
                attrs.update(
                    NB=prod(ishape[:-3]),
                    H=ishape[-3],
                    W=ishape[-2],
                    C=c,
                    F=f,
                    R=r,
                    S=s,
                    stride=(int(sh), int(sw)),
                    pads=pads,
                    pad_value=pad_value,
                    M=int(op.dims["b"]) * int(op.dims["h"]) * int(op.dims["w"]),
                    N=f,
                    K=r * s * c,
                )
            # epilogue fusions: bias_add then relu
            out_uid = n.uid
            nxt = single_internal_use(out_uid)
            if nxt is not None and nxt.operation.name == "bias_add" and nxt.inputs[0] == out_uid:
                attrs["bias"] = nxt.inputs[1]
                src_inputs.append(nxt.inputs[1])
                fused.append(nxt.name)
                absorbed.add(nxt.uid)
                drop_temp(out_uid)
                out_uid = nxt.uid
                nxt = single_internal_use(out_uid)
            if nxt is not None and nxt.operation.name == "relu":
                attrs["relu"] = True
                attrs["threshold"] = float(nxt.operation.attrs.get("threshold", 0))
                fused.append(nxt.name)
                absorbed.add(nxt.uid)
                drop_temp(out_uid)
                out_uid = nxt.uid
            out_dt = _dtype(nodes[out_uid].outputs_types[0])
            if out_uid not in buffers:
                buffers[out_uid] = Buffer(out_uid, _shape(nodes[out_uid].outputs_types[0]), out_dt, "temp")
            target = out_uid
            if attrs["dtype"] == F64:
                # fp64 kernels accumulate and store fp64 (the reference's
                # output dtype is the input's, operators.py:176-188)
                if out_dt != F64:
                    raise UnsupportedGraph(f"{name} {n.name}: float64 inputs need a float64 output, not {out_dt}")
            elif is_bf16(out_dt):
                # kernels accumulate and store fp32; a cast kernel narrows it
                target = out_uid + ".f32"
                buffers[target] = Buffer(target, buffers[out_uid].shape, F32, "temp")
            elif out_dt != F32:
                raise UnsupportedGraph(f"{name} {n.name}: output dtype {out_dt} is not supported")
            launches.append(Launch(name, n.name, src_inputs, target, attrs, fused))
            scheduled[n.name] = n
            if target != out_uid:
                launches.append(Launch("cast", n.name, [target], out_uid, {"n": prod(buffers[out_uid].shape)}))
        elif name == "relu":
            dt = _dtype(t_out)
            if dt not in (F32, F64):
                raise UnsupportedGraph(f"relu {n.name}: only float32 and float64 run standalone")
            attrs = {"threshold": float(op.attrs.get("threshold", 0)), "n": prod(_shape(t_out)), "dtype": dt}
            launches.append(Launch("relu", n.name, [n.inputs[0]], n.uid, attrs))
            scheduled[n.name] = n
        elif name in ("pad", "pad2d"):
            dt = _dtype(t_out)
            if dt not in (F32, F64):
                raise UnsupportedGraph(f"{name} {n.name}: only float32 and float64 run standalone")
            ishape = _shape(out_type(n.inputs[0]))
            padding = op.attrs.get("padding")
            rank = len(ishape)
            if isinstance(padding, dict):
                per = [(0, 0)] * rank
                for a, v in padding.items():
                    per[a % rank] = (int(v[0]), int(v[1]))
            else:
                per = [(int(padding[0]), int(padding[1]))] * rank
            attrs = {"shape": ishape, "pads": per, "value": float(op.attrs.get("constant_value", 0)), "dtype": dt}
            launches.append(Launch("pad", n.name, [n.inputs[0]], n.uid, attrs))
            scheduled[n.name] = n
        elif name == "unpad":
            # a crop: out[o] = in[o + before] per dim (operators.py:683-702)
            dt = _dtype(t_out)
            if dt not in (F32, F64, BF16):
                raise UnsupportedGraph(f"unpad {n.name}: dtype {dt} is not supported")
            ishape = _shape(out_type(n.inputs[0]))
            padding = op.attrs.get("padding")
            rank = len(ishape)
            if isinstance(padding, dict):
                per = [(0, 0)] * rank
                for a, v in padding.items():
                    per[a % rank] = (int(v[0]), int(v[1]))
            else:
                per = [(int(padding[0]), int(padding[1]))] * rank
            attrs = {"shape": ishape, "pads": per, "elem": 2 if dt == BF16 else 8 if dt == F64 else 4}
            launches.append(Launch("unpad", n.name, [n.inputs[0]], n.uid, attrs))
            scheduled[n.name] = n
        elif name == "reshape":
            if n.uid in outputs:
                launches.append(Launch("copy", n.name, [n.inputs[0]], n.uid, {}))
            else:
                buffers[n.uid].kind = "alias"
                buffers[n.uid].alias_of = n.inputs[0]
        else:
            raise UnsupportedGraph(
                f"operator {name} ({n.name}) is not supported by the HIP backend "
                "(supported: matmul, conv2d, relu, pad, pad2d, unpad, bias_add after matmul/conv2d, reshape)"
            )

    # workspace layout: temps packed at 256-byte alignment
    offset = 0
    for b in buffers.values():
        if b.kind == "temp":
            b.offset = offset
            offset += (b.nbytes + 255) // 256 * 256
    return Plan(
        name=graph.name or "payload",
        buffers=buffers,
        launches=launches,
        args=inputs + outputs,
        workspace_bytes=offset,
        scheduled=scheduled,
    )
