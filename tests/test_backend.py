# SPDX-License-Identifier: BSD-3-Clause
"""HIP backend host logic on the CPU: lowering (fusions, workspace), the
scheduler surface, schedule -> kernel mapping, payload code generation and
the C-ABI library's exports.  Nothing here launches a kernel."""

from __future__ import annotations

import ctypes
import re
import subprocess
import threading
from pathlib import Path

import numpy as np
import pytest

import xtc_amd.graphs.xtc.op as O
from xtc_amd.backends.hip import Backend
from xtc_amd.backends.hip.compiler import generate_payload
from xtc_amd.backends.hip.lowering import UnsupportedGraph
from xtc_amd.backends.hip.mapping import legal_tiles, map_gemm
from xtc_amd.backends.hip.scheduler import ScheduleError
from xtc_amd.runtimes.hip import capi

ROOT = Path(__file__).resolve().parent.parent


def _matmul(m, n, k, dtype="float32", name="mm", **kw):
    a = O.tensor((m, k), dtype, name="A")
    b = O.tensor((k, n), dtype, name="B")
    with O.graph(name=name) as gb:
        O.matmul(a, b, name="C", **kw)
    return gb.graph


def _conv_relu():
    x = O.tensor((8, 56, 56, 64), "float32", name="I")
    w = O.tensor((3, 3, 64, 64), "float32", name="W")
    with O.graph(name="conv_relu") as gb:
        p = O.pad2d(x, padding=1, axes=(1, 2), name="pad")
        c = O.conv2d(p, w, name="conv")
        O.relu(c, name="relu")
    return gb.graph


def _mlp():
    x = O.tensor((2048, 1024), "float32", name="X")
    w1 = O.tensor((1024, 4096), "float32", name="W1")
    w2 = O.tensor((4096, 1024), "float32", name="W2")
    with O.graph(name="mlp") as gb:
        h = O.relu(O.matmul(x, w1, name="fc1"), name="act")
        O.matmul(h, w2, name="fc2")
    return gb.graph


# ---------------------------------------------------------------- lowering

def test_conv_pad_relu_fuse_into_one_launch():
    plan = Backend(_conv_relu()).plan
    (ln,) = plan.launches
    assert ln.kind == "conv2d" and ln.node == "conv"
    assert ln.absorbed == ["pad", "relu"]
    assert ln.attrs["pads"] == (1, 1, 1, 1) and ln.attrs["relu"]
    assert (ln.attrs["M"], ln.attrs["N"], ln.attrs["K"]) == (8 * 56 * 56, 64, 576)
    assert (ln.attrs["H"], ln.attrs["W"]) == (56, 56)  # the loader reads the unpadded input
    assert plan.workspace_bytes == 0


def test_mlp_relu_epilogue_and_workspace():
    plan = Backend(_mlp()).plan
    assert [(l.kind, l.node, l.absorbed) for l in plan.launches] == [("matmul", "fc1", ["act"]), ("matmul", "fc2", [])]
    temps = [b for b in plan.buffers.values() if b.kind == "temp"]
    assert len(temps) == 1 and temps[0].nbytes == 2048 * 4096 * 4 and temps[0].offset % 256 == 0
    assert plan.workspace_bytes == 2048 * 4096 * 4


def test_relu_not_fused_when_intermediate_is_an_output():
    a = O.tensor((64, 64), "float32")
    b = O.tensor((64, 64), "float32")
    with O.graph(name="fused") as gb:
        O.relu(O.matmul(a, b, name="mm"), name="r")
    # single consumer, not an output: fused
    assert [l.kind for l in Backend(gb.graph).plan.launches] == ["matmul"]
    with O.graph(name="two_outs") as gb:
        c = O.matmul(a, b, name="mm")
        r = O.relu(c, name="r")
        O.outputs(c, r)
    plan = Backend(gb.graph).plan
    assert len(gb.graph.outputs) == 2
    assert [l.kind for l in plan.launches] == ["matmul", "relu"]
    assert not plan.launches[0].attrs["relu"]


def test_unfused_pad_and_standalone_relu():
    x = O.tensor((2, 5, 5, 3), "float32")
    with O.graph(name="pad_relu") as gb:
        O.relu(O.pad2d(x, padding=(1, 2), axes=(1, 2), constant_value=-1.0), threshold=0.5)
    plan = Backend(gb.graph).plan
    assert [l.kind for l in plan.launches] == ["pad", "relu"]
    pad = plan.launches[0]
    assert pad.attrs["pads"] == [(0, 0), (1, 2), (1, 2), (0, 0)] and pad.attrs["value"] == -1.0
    assert plan.launches[1].attrs == {"threshold": 0.5, "n": 2 * 8 * 8 * 3, "dtype": "float32"}


def test_bias_add_fuses_before_relu():
    a = O.tensor((128, 64), "float32")
    w = O.tensor((64, 32), "float32")
    bias = O.tensor((32,), "float32")
    with O.graph(name="fc") as gb:
        O.relu(O.bias_add(O.matmul(a, w, name="mm"), bias))
    (ln,) = Backend(gb.graph).plan.launches
    assert ln.attrs["bias"] is not None and ln.attrs["relu"] and len(ln.absorbed) == 2


def test_bf16_output_gets_a_cast_launch():
    plan = Backend(_matmul(256, 256, 64, "bfloat16")).plan
    assert [l.kind for l in plan.launches] == ["matmul", "cast"]
    plan32 = Backend(_matmul(256, 256, 64, "bfloat16", out_dtype="float32")).plan
    assert [l.kind for l in plan32.launches] == ["matmul"]


def test_reshape_is_an_alias():
    img = O.tensor((32, 32, 3), "float32")
    w = O.tensor((3072, 16), "float32")
    with O.graph(name="fc") as gb:
        O.matmul(O.reshape(img, shape=(1, -1)), w)
    plan = Backend(gb.graph).plan
    assert [l.kind for l in plan.launches] == ["matmul"]
    aliases = [b for b in plan.buffers.values() if b.kind == "alias"]
    assert len(aliases) == 1 and plan.buffer(aliases[0].uid).kind == "input"


def test_unsupported_operator_and_dtype_raise():
    k = O.tensor((8, 5, 5, 3), "float32")
    with O.graph(name="tr") as gb:
        O.transpose(k, axes=(1, 2, 3, 0))
    with pytest.raises(UnsupportedGraph):
        Backend(gb.graph)
    with pytest.raises(UnsupportedGraph):
        Backend(_matmul(16, 16, 16, "int32"))


def test_float64_graphs_lower_to_fp64_launches(tmp_path):
    # float64 matmul / conv2d / relu / pad, as the reference's MLIR backend
    # lowers them (MlirOps.py:194-195,234,339,463,616): fp64 kernels, fp64
    # outputs, thresholds and pad values passed as C doubles
    x = O.tensor((8, 14, 14, 16), "float64", name="I")
    w = O.tensor((3, 3, 16, 32), "float64", name="W")
    with O.graph(name="conv64") as gb:
        c = O.conv2d(O.pad2d(x, padding=1, axes=(1, 2), name="pad", constant_value=0.3), w, name="conv")
        r = O.relu(c, name="relu", threshold=0.1)
        O.pad(r, padding=(0, 1), name="post")
    b = Backend(gb.graph)
    kinds = [(ln.kind, ln.attrs.get("dtype")) for ln in b.plan.launches]
    assert kinds == [("conv2d", "float64"), ("pad", "float64")]
    cfgs = b.get_compiler().kernel_configs(b.get_scheduler().schedule())
    assert cfgs["conv"].dtype == "float64" and cfgs["conv"].tile in legal_tiles("float64", True)
    src = generate_payload(b.plan, cfgs, "conv64", 0, True)
    assert "XTC_HIP_F64" in src and "xtc_hip_pad_f64" in src
    assert ", 0.1, 0.3};" in src  # relu_threshold_f64, pad_value_f64: exact doubles
    module = b.get_compiler(dump_file=str(tmp_path / "conv64")).compile(b.get_scheduler().schedule())
    assert Path(module.file_name).exists()
    # fp64 operands need an fp64 output, as the reference's output dtype is the input's
    a64 = O.tensor((16, 16), "float64", name="A")
    b64 = O.tensor((16, 16), "float64", name="B")
    with O.graph(name="mm64") as gb2:
        O.matmul(a64, b64, name="C")
    (ln,) = Backend(gb2.graph).plan.launches
    assert ln.attrs["dtype"] == "float64"
    assert legal_tiles("float64", False) and capi.default_tile("float64", False, 4096, 4096, 4096)[0] == (
        128, 128, 16, 2, 2)
    # a schedule vectorizing j by 3 does not fit the 2-element fp64 vectors
    sch = Backend(_matmul(256, 96, 64, "float64")).get_scheduler()
    sch.tile("j", {"j1": 32, "j2": 3})
    sch.vectorize(["j2"])
    with pytest.raises(ScheduleError, match="2-element"):
        map_gemm(Backend(_matmul(256, 96, 64, "float64")).plan.launches[0].attrs, False,
                 sch.schedule().node("C"), "strict")


def test_operand_layouts_lower_to_transpose_flags(tmp_path):
    # layout [1, 0] on matmul operands, as tests/filecheck/backends/test_matmul_mlir_layout.py
    a = O.tensor((4, 512), "float32", name="A", layout=[1, 0])
    b = O.tensor((512, 32), "float32", name="B", layout=[1, 0])
    with O.graph(name="matmul_layout") as gb:
        O.matmul(a, b, name="C")
    assert "4x512xfloat32, <(0,1)->(1,0)>" in str(gb.graph)
    backend = Backend(gb.graph)
    (ln,) = backend.plan.launches
    assert ln.attrs["trans_a"] and ln.attrs["trans_b"] and (ln.attrs["M"], ln.attrs["N"], ln.attrs["K"]) == (4, 32, 512)
    module = backend.get_compiler(dump_file=str(tmp_path / "ml")).compile(backend.get_scheduler().schedule())
    # the two flags close the descriptor initializer (fields trans_a, trans_b)
    assert re.search(r"xtc_hip_matmul_desc d = \{.*, 1, 1, 0, 0.0\};", module.source)
    natural = Backend(_matmul(4, 32, 512)).plan.launches[0].attrs
    assert not natural["trans_a"] and not natural["trans_b"]


def test_layouts_outside_matmul_operands_raise():
    # the reference's MLIR backend raises for them too (MlirOps.py:45-52,
    # tests/filecheck/backends/invalid/test_relu_mlir_layout.py)
    a = O.tensor((4, 32), "float32", name="A", layout=[1, 0])
    with O.graph(name="relu_layout") as gb:
        O.relu(a, name="relu")
    with pytest.raises(UnsupportedGraph, match="layout"):
        Backend(gb.graph)
    x = O.tensor((64, 16), "float32", name="X")
    w = O.tensor((16, 8), "float32", name="W")
    bias = O.tensor((8, 1), "float32", name="b", layout=[1, 0])
    with O.graph(name="bias_layout") as gb:
        O.bias_add(O.matmul(x, w, name="mm"), O.reshape(bias, (8,)), name="ba")
    with pytest.raises(UnsupportedGraph, match="layout"):
        Backend(gb.graph)


def test_device_array_layout_round_trip_on_host(monkeypatch):
    # DeviceArray with layout [1, 0] stores the transpose and hands back the
    # logical array; a fake device (host memory) checks the byte order.
    from xtc_amd.runtimes.hip.ndarray import DeviceArray

    class FakeDevice:
        def __init__(self):
            self.mem = {}

        def memory_allocate(self, n):
            buf = (ctypes.c_char * n)()
            self.mem[ctypes.addressof(buf)] = buf
            return ctypes.addressof(buf)

        def memory_copy_to(self, dst, src, n):
            ctypes.memmove(dst, src, n)

        def memory_copy_from(self, src, dst, n):
            ctypes.memmove(dst, src, n)

        def memory_free(self, h):
            self.mem.pop(h, None)

    import numpy as np

    dev = FakeDevice()
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    d = DeviceArray.from_numpy(x, "float32", dev, [1, 0])
    stored = np.frombuffer(dev.mem[d.data], dtype=np.float32).reshape(4, 3)
    np.testing.assert_array_equal(stored, x.T)
    np.testing.assert_array_equal(d.numpy(), x)
    assert DeviceArray.from_numpy(x, "float32", dev, [0, 1]).layout is None
    with pytest.raises(ValueError):
        DeviceArray((2, 3, 4), "float32", dev, [2, 1, 0])


# ---------------------------------------------------------------- scheduler

def test_default_node_writes_the_output():
    assert Backend(_conv_relu()).get_scheduler().node_name == "conv"
    assert Backend(_mlp()).get_scheduler().node_name == "fc2"
    assert Backend(_mlp()).get_scheduler(default_node="fc1").node_name == "fc1"
    with pytest.raises(ScheduleError):
        Backend(_mlp()).get_scheduler(default_node="nope")


def test_schedule_records_primitives():
    sch = Backend(_matmul(512, 512, 512)).get_scheduler()
    sch.tile("i", {"i1": 128, "i2": 32})
    sch.tile("j", {"j1": 128})
    sch.interchange(["i", "j", "k", "i1", "j1", "i2"])
    sch.parallelize(["i"])
    sch.vectorize(["i2"])
    sch.unroll({"i2": 4})
    (s,) = sch.schedule().schedule_impl
    assert s.tiles == {"i": {"i1": 128, "i2": 32}, "j": {"j1": 128}, "k": {}}
    assert s.permutation["."][:3] == ["./i", "./j", "./k"]
    assert s.parallelization == ["./i"] and s.vectorization == ["./i2"] and s.unrolling == {"./i2": 4}
    assert "i1" in str(sch.schedule())
    with pytest.raises(ScheduleError):
        sch.tile("q", {"q1": 2})


def _pad_conv_mini():
    # tests/filecheck/backends/tensor_dialect/test_pad_conv2d_mlir_tensor_fused.py
    a = O.tensor((1, 8, 8, 3), "float32", name="I")
    b = O.tensor((5, 5, 3, 16), "float32", name="W")
    with O.graph(name="pad_conv2d_nhwc_mini") as gb:
        p = O.pad2d(a, padding=2, axes=(1, 2), name="pad")
        O.conv2d(p, b, stride=(2, 2), name="conv")
    return gb.graph


def test_fuse_producer_at_pad_into_conv(tmp_path):
    backend = Backend(_pad_conv_mini())
    sch = backend.get_scheduler()
    sch.interchange(["b", "h", "w", "r", "s", "c", "f"])
    sch.fuse_producer_at("w", 0)
    sch.vectorize(["f"])
    sched = sch.schedule()
    assert sched.node("conv").fused == [("./w", 0)]
    module = backend.get_compiler(dump_file=str(tmp_path / "pc")).compile(sched)
    (ln,) = module.plan.launches
    assert ln.kind == "conv2d" and ln.absorbed == ["pad"]
    with pytest.raises(ScheduleError):
        sch.fuse_producer_at("q", 0)  # not a loop of conv


def test_fuse_producer_at_rejects_what_is_not_fused(tmp_path):
    # input 1 (the weights) is a graph input: nothing to fuse
    backend = Backend(_pad_conv_mini())
    sch = backend.get_scheduler()
    sch.fuse_producer_at("w", 1)
    with pytest.raises(ScheduleError, match="graph input"):
        backend.get_compiler(dump_file=str(tmp_path / "a")).compile(sch.schedule())
    # a relu producer of a matmul is its own launch
    x = O.tensor((64, 64), "float32", name="X")
    w = O.tensor((64, 64), "float32", name="W")
    with O.graph(name="relu_mm") as gb:
        O.matmul(O.relu(x, name="act"), w, name="mm")
    backend = Backend(gb.graph)
    sch = backend.get_scheduler(default_node="mm")
    sch.fuse_producer_at("i", 0)
    with pytest.raises(ScheduleError, match="cannot fuse relu act"):
        backend.get_compiler(dump_file=str(tmp_path / "b")).compile(sch.schedule())


def test_meshes_are_rejected():
    sch = Backend(_matmul(64, 64, 64)).get_scheduler()
    for call in (lambda: sch.define_processor_mesh({"x": 2}), lambda: sch.define_memory_mesh({"x": 2}),
                 lambda: sch.distribute("i", "x"), lambda: sch.distributed_buffer_at("i", 0, ["x"])):
        with pytest.raises(ScheduleError, match="one GPU"):
            call()


def test_loop_nest():
    sch = Backend(_matmul(256, 256, 64)).get_scheduler()
    sch.tile("i", {"i1": 64})
    sch.interchange(["i", "j", "k", "i1"])
    nest = sch.get_loop_nest()
    assert nest.root_node.pretty_print() == "loop i\n  loop j\n    loop k\n      tile(i, 64)\n        ..."
    nest.check()


# ---------------------------------------------------------------- mapping

def _sched(graph, tiles=None, order=None, parallel=None):
    b = Backend(graph)
    sch = b.get_scheduler()
    for d, t in (tiles or {}).items():
        sch.tile(d, t)
    if order:
        sch.interchange(order)
    if parallel:
        sch.parallelize(parallel)
    (ln,) = [l for l in b.plan.launches if l.kind in ("matmul", "conv2d")]
    return ln.attrs, sch.schedule().node(ln.node)


def test_mapping_exact_c3a():
    attrs, s = _sched(_matmul(8192, 8192, 8192, "bfloat16", out_dtype="float32"),
                      {"i": {"i1": 256, "i2": 64}, "j": {"j1": 256, "j2": 128}, "k": {"k1": 64}})
    cfg = map_gemm(attrs, False, s, "strict")
    assert cfg.tile == (256, 256, 64, 4, 2) and cfg.exact and cfg.split_k == 1 and cfg.source == "schedule"


def test_mapping_strict_rejects_and_nearest_maps():
    attrs, s = _sched(_matmul(4096, 4096, 4096), {"i": {"i1": 96}, "j": {"j1": 96}, "k": {"k1": 16}})
    with pytest.raises(ScheduleError, match="no float32 matmul kernel"):
        map_gemm(attrs, False, s, "strict")
    cfg = map_gemm(attrs, False, s, "nearest")
    assert not cfg.exact and cfg.source == "nearest" and cfg.tile in legal_tiles("float32", False)


def test_unmapped_schedule_fails_at_evaluation_by_default():
    # no compile kwargs (as the reference's explorer calls it): the module
    # compiles, its payload launches nothing and reports the mapping error,
    # and the evaluator returns code 2 instead of timing another kernel
    g = _matmul(4096, 4096, 4096)
    b = Backend(g)
    sch = b.get_scheduler()
    for d, t in {"i": {"i1": 96}, "j": {"j1": 96}, "k": {"k1": 16}}.items():
        sch.tile(d, t)
    module = b.get_compiler().compile(sch.schedule())
    assert "no float32 matmul kernel for block tile 96x96x16" in module.schedule_error
    assert module.configs == {} and "xtc_hip_matmul(" not in module.source
    res, code, msg = module.get_evaluator().evaluate()
    assert (res, code) == ([], 2) and "no float32 matmul kernel" in msg
    assert module.get_executor().execute() == 2
    so = ctypes.CDLL(module.file_name)
    getattr(so, module.payload_name)(None, None, None)
    status = getattr(so, f"{module.payload_name}_status")
    message = getattr(so, f"{module.payload_name}_message")
    status.restype = ctypes.c_int
    message.restype = ctypes.c_char_p
    assert status() == 2 and b"no float32 matmul kernel" in message()
    with pytest.raises(ScheduleError, match="no float32 matmul kernel"):
        b.get_compiler(schedule_policy="strict").compile(sch.schedule())
    nearest = b.get_compiler(schedule_policy="nearest").compile(sch.schedule())
    assert nearest.schedule_error is None and not nearest.configs["C"].exact


def _split_schedule(b):
    """i split at 256 into two segments with their own tiles; the second
    segment's j split again at 128 (nested), each piece with its own tile
    (src/xtc/itf/schd/scheduler.py:65-81: segments by ascending start)."""
    sch = b.get_scheduler()
    sch.split("i", {"i_lo": 0, "i_hi": 256})
    sch.tile("i", {"i1": 128, "i2": 64}, root="./i_lo")
    sch.tile("j", {"j1": 128, "j2": 64}, root="./i_lo")
    sch.tile("k", {"k1": 32}, root="./i_lo")
    sch.split("j", {"j_a": 0, "j_b": 128}, root="./i_hi")
    sch.tile("i", {"i1": 64}, root="./i_hi/j_a")
    sch.tile("j", {"j1": 64}, root="./i_hi/j_a")
    sch.tile("k", {"k1": 32}, root="./i_hi/j_a")
    return sch


def test_split_maps_to_one_launch_per_segment():
    from xtc_amd.backends.hip.mapping import SplitConfig, map_node

    b = Backend(_matmul(384, 256, 512))
    sch = _split_schedule(b)
    (ln,) = b.plan.launches
    cfg = map_node(ln.attrs, False, sch.schedule().node(ln.node))
    assert isinstance(cfg, SplitConfig) and cfg.exact
    got = [(p.m0, p.M, p.n0, p.N, p.config.tile[:3], p.config.source) for p in cfg.pieces]
    assert got == [
        (0, 256, 0, 256, (128, 128, 32), "schedule"),
        (256, 128, 0, 128, (64, 64, 32), "schedule"),
        (256, 128, 128, 128, _default_tile_of(128, 128, 512), "default"),  # untiled segment
    ]
    # one launch per piece on the strided sub-views, whole-operand strides
    module = b.get_compiler().compile(sch.schedule())
    body = module.source.split(f"void {module.payload_name}(")[-1]
    assert body.count("xtc_hip_matmul(") == 3
    assert "(const char *)a0 + 524288ull" in body  # A rows from 256: 256 * 512 * 4 bytes
    assert "(const char *)a1 + 512ull" in body  # B columns from 128
    assert "(char *)a2 + 262656ull" in body  # C at (256, 128): (256 * 256 + 128) * 4
    assert re.search(r"= \{XTC_HIP_F32, 128, 128, 512, 512, 256, 256, ", body)


def _default_tile_of(m, n, k):
    tile, _ = capi.default_tile("float32", False, m, n, k)
    return tuple(tile[:3])


def test_split_transposed_operands_offset_the_other_way():
    from xtc_amd.backends.hip.mapping import SplitConfig

    a = O.tensor((256, 128), "float32", name="A", layout=[1, 0])
    bt = O.tensor((128, 256), "float32", name="B", layout=[1, 0])
    with O.graph(name="mmt") as gb:
        O.matmul(a, bt, name="C")
    b = Backend(gb.graph)
    sch = b.get_scheduler()
    sch.split("i", {"lo": 0, "hi": 64})
    sch.split("j", {"l": 0, "r": 32}, root="./hi")
    module = b.get_compiler().compile(sch.schedule())
    assert isinstance(module.configs["C"], SplitConfig)
    body = module.source.split(f"void {module.payload_name}(")[-1]
    # A^T [128][256]: rows 64.. of A are columns 64.. of A^T (64 * 4 bytes);
    # B^T [256][128]: columns 32.. of B are rows 32.. of B^T (32 * 128 * 4)
    assert "(const char *)a0 + 256ull" in body and "(const char *)a1 + 16384ull" in body
    assert re.search(r"= \{XTC_HIP_F32, 192, 32, 128, 256, 128, 256, ", body)


def test_nested_split_of_the_same_axis_keeps_both_levels():
    # i split at the root, then again inside the second segment (cut points
    # relative to the segment): three row pieces, none lost
    from xtc_amd.backends.hip.mapping import map_node

    b = Backend(_matmul(512, 128, 256))
    sch = b.get_scheduler()
    sch.split("i", {"lo": 0, "hi": 128})
    sch.split("i", {"a": 0, "b": 256}, root="./hi")
    (ln,) = b.plan.launches
    cfg = map_node(ln.attrs, False, sch.schedule().node(ln.node))
    assert [(p.m0, p.M, p.n0, p.N) for p in cfg.pieces] == [(0, 128, 0, 128), (128, 256, 0, 128), (384, 128, 0, 128)]


def test_reference_explorer_compile_kwargs(tmp_path):
    # src/xtc/search/explore.py:365-391 passes bare_ptr=False by default; the
    # payload still takes bare device pointers, as the MLIR compiler forces
    b = Backend(_matmul(64, 64, 64))
    module = b.get_compiler(shared_lib=True, dump_file=str(tmp_path / "payload_0"), bare_ptr=False,
                            debug=False).compile(b.get_scheduler().schedule())
    assert module.file_name.endswith(".so") and Path(module.file_name).exists()
    assert module._bare_ptr


def test_split_inside_a_tile_is_rejected():
    """A split after tiles of the same axis cuts every tile: no sub-matrix
    per segment, so no HIP mapping."""
    from xtc_amd.backends.hip.mapping import map_node

    b = Backend(_matmul(256, 256, 256))
    sch = b.get_scheduler()
    sch.tile("i", {"i1": 64})
    sch.split("i", {"i_lo": 0, "i_hi": 32})
    (ln,) = b.plan.launches
    with pytest.raises(ScheduleError, match="inside its tiles"):
        map_node(ln.attrs, False, sch.schedule().node(ln.node))


def test_split_on_k_or_conv_is_rejected():
    from xtc_amd.backends.hip.mapping import map_node

    b = Backend(_matmul(256, 256, 512))
    sch = b.get_scheduler()
    sch.split("k", {"k_lo": 0, "k_hi": 256})
    (ln,) = b.plan.launches
    with pytest.raises(ScheduleError, match="reduction axis"):
        map_node(ln.attrs, False, sch.schedule().node(ln.node))
    sch = b.get_scheduler()
    sch.split("i", {"a": 64, "b": 128})
    with pytest.raises(ScheduleError, match="starts at 64"):
        map_node(ln.attrs, False, sch.schedule().node(ln.node))
    g = _conv_relu()
    bc = Backend(g)
    sch = bc.get_scheduler()
    (cl,) = [l for l in bc.plan.launches if l.kind == "conv2d"]
    sch.split(sch.schedule().node(cl.node).dims[0], {"x": 0, "y": 4})
    with pytest.raises(ScheduleError, match="conv2d"):
        map_node(cl.attrs, True, sch.schedule().node(cl.node))


def test_mapping_split_k():
    attrs, s = _sched(_matmul(256, 256, 8192), {"i": {"i1": 128}, "j": {"j1": 128}, "k": {"k1": 1024, "k2": 32}},
                      parallel=["k"])
    cfg = map_gemm(attrs, False, s, "nearest")
    assert cfg.split_k == 8 and cfg.bk == 32
    attrs, s = _sched(_matmul(256, 256, 1000), {"k": {"k1": 300}}, parallel=["k"])
    with pytest.raises(ScheduleError, match="multiple"):
        map_gemm(attrs, False, s, "nearest")


def test_mapping_unroll_of_the_slab_loop_selects_the_pipeline_depth():
    from xtc_amd.backends.hip.mapping import pipeline_depths

    g = _matmul(4096, 4096, 4096)
    tiles = {"i": {"i1": 256, "i2": 64}, "j": {"j1": 128, "j2": 64}, "k": {"k1": 32}}

    def cfg(t, unroll, parallel=None, graph=g):
        b = Backend(graph)
        sch = b.get_scheduler()
        for d, v in t.items():
            sch.tile(d, v)
        if parallel:
            sch.parallelize(parallel)
        sch.unroll(unroll)
        (ln,) = [l for l in b.plan.launches if l.kind == "matmul"]
        return map_gemm(ln.attrs, False, sch.schedule().node(ln.node), "strict"), ln.attrs

    # LDS-DMA fp32 256x128x32: 3 stages (default) or 2
    c, attrs = cfg(tiles, {"k": 2})
    assert c.tile == (256, 128, 32, 4, 2) and c.stages == 2
    assert pipeline_depths(attrs, False, c.tile, 1) == [3, 2]
    assert cfg(tiles, {"k": 3})[0].stages == 0  # the default depth is left to the kernel
    with pytest.raises(ScheduleError, match=r"4-slab pipeline.*\[3, 2\]"):
        cfg(tiles, {"k": 4})
    # unroll of the MFMA loop inside a slab, or of M/N loops, is recorded only
    assert cfg(tiles, {"k1": 32, "i1": 256})[0].stages == 0
    # BK 16: 3-6 stages of 24 KB
    t16 = {**tiles, "k": {"k1": 16}}
    assert [cfg(t16, {"k": d})[0].stages for d in (3, 5, 6)] == [3, 5, 6]
    # split-K: the slab loop is k1 (k is the parallel loop over splits)
    tsk = {"i": {"i1": 128, "i2": 64}, "j": {"j1": 128, "j2": 32}, "k": {"k1": 2048, "k2": 32}}
    c, _ = cfg(tsk, {"k1": 4}, parallel=["i", "j", "k"])
    assert (c.split_k, c.stages) == (2, 4)
    # the generic template double-buffers: depth 2 only
    tg = {"i": {"i1": 64, "i2": 32}, "j": {"j1": 64, "j2": 32}, "k": {"k1": 32}}
    assert cfg(tg, {"k": 2})[0].stages == 0
    with pytest.raises(ScheduleError, match="pipeline"):
        cfg(tg, {"k": 3})
    # bf16 ping-pong 256x256x32: 4 (default), 3, 5
    g3 = _matmul(8192, 8192, 8192, "bfloat16", out_dtype="float32")
    tp = {"i": {"i1": 256, "i2": 128}, "j": {"j1": 256, "j2": 64}, "k": {"k1": 32}}
    assert [cfg(tp, {"k": d}, graph=g3)[0].stages for d in (3, 4, 5)] == [3, 0, 5]


def test_mapping_vectorize_checks_the_vector_width():
    g = _matmul(4096, 4096, 4096)
    b = Backend(g)
    sch = b.get_scheduler()
    sch.tile("i", {"i1": 256, "i2": 64})
    sch.tile("j", {"j1": 128, "j2": 64, "j3": 2})
    sch.tile("k", {"k1": 32})
    sch.vectorize(["j2"])
    (ln,) = b.plan.launches
    assert map_gemm(ln.attrs, False, sch.schedule().node(ln.node), "strict").exact
    sch.vectorize(["j3"])
    with pytest.raises(ScheduleError, match=r"vectorize\(j3\): extent 2 .* 4-element"):
        map_gemm(ln.attrs, False, sch.schedule().node(ln.node), "strict")


def test_pipeline_depth_queries():
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_BF16, M=16, N=8192, K=8192, tile=capi.Tile(16, 128, 64, 1, 4), split_k=8)
    assert capi.matmul_pipeline_depths(d) == [4, 3, 2]  # skinny bf16
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_F32, M=100, N=60, K=30)
    assert capi.matmul_pipeline_depths(d) == [1]  # K and N not multiples of the 4-element vector: scalar kernel
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_F32, M=512, N=512, K=512, tile=capi.Tile(32, 32, 16, 1, 1), split_k=4)
    assert capi.matmul_pipeline_depths(d) == [4, 2, 8]  # split-wave register ring
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_BF16, M=512, N=512, K=512, tile=capi.Tile(256, 256, 32, 2, 4), trans_b=1)
    assert capi.matmul_pipeline_depths(d) == [4, 3, 5]  # B^T read natively by the ping-pong kernel
    c = capi.Conv2dDesc(dtype=capi.XTC_HIP_F32, N=8, H=56, W=56, C=64, F=64, R=3, S=3, stride_h=1, stride_w=1,
                        pad_top=1, pad_bottom=1, pad_left=1, pad_right=1)
    assert capi.conv2d_pipeline_depths(c) == [3]  # direct conv 7x14: a register ring of 3 weight taps
    d = capi.MatmulDesc(dtype=7, M=1, N=1, K=1)
    with pytest.raises(capi.HipError, match="bad dtype"):
        capi.matmul_pipeline_depths(d)


def _conv_c(C, tile=None, split_k=0, pad_value=0.0):
    c = capi.Conv2dDesc(dtype=capi.XTC_HIP_F32, N=8, H=56, W=56, C=C, F=64, R=3, S=3, stride_h=1, stride_w=1,
                        pad_top=1, pad_bottom=1, pad_left=1, pad_right=1, pad_value=pad_value, split_k=split_k)
    if tile:
        c.tile = capi.Tile(*tile)
    return c


def test_conv_pipeline_depths_describe_the_channel_staged_kernel():
    # C = 3 is copied with a zero channel up to C = 4 and runs the MFMA conv:
    # the depth query answers for that kernel, exactly as for C = 4
    for tile, sk in ((None, 0), ((64, 64, 16, 2, 2), 4), ((64, 64, 16, 2, 2), 1)):
        assert capi.conv2d_pipeline_depths(_conv_c(3, tile, sk)) == capi.conv2d_pipeline_depths(_conv_c(4, tile, sk))
    assert capi.conv2d_pipeline_depths(_conv_c(3, (64, 64, 16, 2, 2), 4)) == [4]  # register ring under split-K
    # the direct-only tile needs 64-channel multiples: not runnable at C = 3 or 4
    for tile in ((112, 64, 16, 1, 4), (98, 64, 16, 1, 4)):
        for C in (3, 4):
            with pytest.raises(capi.HipError, match="exists only in the direct conv kernel"):
                capi.conv2d_pipeline_depths(_conv_c(C, tile))
        assert capi.conv2d_pipeline_depths(_conv_c(64, tile)) == [3]
    # a non-finite pad value cannot be staged (inf * 0 is NaN): the scalar kernel
    assert capi.conv2d_pipeline_depths(_conv_c(3, pad_value=float("inf"))) == [1]


def _integration_structs():
    """The ctypes structs of the binding that the integration guide at the
    repository root tells maintainers to write (its ctypes snippet)."""
    text = (ROOT / "INTEGRATION.md").read_text()
    block = re.search(r"```python\n(import ctypes\n\nclass Tile.*?)\nlib = ctypes\.CDLL", text, re.S)
    assert block, "INTEGRATION.md: ctypes binding snippet not found"
    ns: dict = {}
    exec(compile(block.group(1), "INTEGRATION.md", "exec"), ns)
    return ns


def test_descriptor_sizes_match_the_library_and_the_documented_binding():
    lib = capi.lib()  # loading checks capi's own structs against the library
    assert ctypes.sizeof(capi.MatmulDesc) == lib.xtc_hip_matmul_desc_size()
    assert ctypes.sizeof(capi.Conv2dDesc) == lib.xtc_hip_conv2d_desc_size()
    ns = _integration_structs()
    assert ctypes.sizeof(ns["MatmulDesc"]) == lib.xtc_hip_matmul_desc_size()
    assert [f[0] for f in ns["MatmulDesc"]._fields_] == [f[0] for f in capi.MatmulDesc._fields_]
    assert [f[0] for f in ns["Tile"]._fields_] == [f[0] for f in capi.Tile._fields_]


def test_mapping_column_major_raster():
    g = _matmul(4096, 4096, 4096)
    attrs, s = _sched(g, {"i": {"i1": 128}, "j": {"j1": 128}, "k": {"k1": 16}}, order=["j", "i", "k", "i1", "j1", "k1"])
    assert map_gemm(attrs, False, s).group_m == 4096 // 128
    attrs, s = _sched(g, {"i": {"i1": 128}, "j": {"j1": 128}, "k": {"k1": 16}})
    assert map_gemm(attrs, False, s).group_m == 8


def test_mapping_default_and_conv_roles():
    attrs, s = _sched(_matmul(8192, 8192, 8192, "bfloat16", out_dtype="float32"))
    cfg = map_gemm(attrs, False, s)
    # bf16 8192^3 defaults to the ping-pong LDS-DMA kernel's tile
    assert cfg.source == "default" and cfg.tile == (256, 256, 32, 2, 4)
    # conv: b,h,w tile levels multiply into BM, f is N, r,s,c are K
    attrs, s = _sched(_conv_relu(), {"h": {"h1": 2}, "w": {"w1": 32}, "f": {"f1": 64}, "c": {"c1": 16}})
    cfg = map_gemm(attrs, True, s, "nearest")
    assert cfg.conv and cfg.tile in legal_tiles("float32", True)


# ---------------------------------------------------------------- payload codegen

def test_payload_source_and_exports(tmp_path):
    g = _mlp()
    b = Backend(g)
    module = b.get_compiler(dump_file=str(tmp_path / "mlp")).compile(b.get_scheduler().schedule())
    src = module.source
    assert "xtc_hip_matmul" in src and "xtc_hip_synchronize" in src
    syms = subprocess.run(["nm", "-D", "--defined-only", module.file_name], capture_output=True, text=True,
                          check=True).stdout
    for sym in ("mlp", "mlp_status", "mlp_message", "mlp_release"):
        assert re.search(rf"\bT {sym}$", syms, re.M), sym
    # all scheduled GEMMs carry a kernel choice
    assert set(module.configs) == {"fc1", "fc2"}


def test_concurrent_compiles_share_the_cache():
    g = _matmul(1024, 1024, 1024)
    paths, errors = [], []

    def work():
        try:
            b = Backend(g)
            paths.append(b.get_compiler().compile(b.get_scheduler().schedule()).file_name)
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    ts = [threading.Thread(target=work) for _ in range(6)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors and len(set(paths)) == 1


def test_generated_payload_checks_status_between_launches():
    b = Backend(_conv_relu())
    cfgs = b.get_compiler().kernel_configs(b.get_scheduler().schedule())
    src = generate_payload(b.plan, cfgs, "conv_relu", 0, True)
    assert src.count("xtc_hip_conv2d(") == 1
    assert "conv_relu_status" in src and "xtc_hip_synchronize" in src
    assert "xtc_hip_synchronize" not in generate_payload(b.plan, cfgs, "conv_relu", 0, False).split("conv_relu(")[-1]


# ---------------------------------------------------------------- C-ABI library

def _header_functions(header: str = "xtc_hip.h") -> set[str]:
    text = (ROOT / "include" / header).read_text()
    return set(re.findall(r"\b(xtc_hip_\w+)\s*\(", text))


def test_library_exports_every_declared_function():
    lib = capi.lib()
    declared = _header_functions()
    assert len(declared) >= 25
    missing = [f for f in declared if not hasattr(lib, f)]
    assert not missing
    assert declared == set(capi.SIGNATURES)


def test_pmu_library_exports_every_declared_function():
    from xtc_amd.runtimes.hip import pmu

    lib = pmu.lib()  # loads without a GPU; nothing is called
    declared = _header_functions("xtc_hip_pmu.h")
    assert len(declared) == 9
    assert not [f for f in declared if not hasattr(lib, f)]
    assert declared == set(pmu._SIGNATURES)
    # every header under include/ is covered by one of the two libraries
    assert {h.name for h in (ROOT / "include").glob("*.h")} == {"xtc_hip.h", "xtc_hip_pmu.h"}
    assert pmu.is_hardware_counter("gpu.SQ_WAVES") and pmu.is_hardware_counter("gpu.cycles")
    assert not pmu.is_hardware_counter("gpu.time") and not pmu.is_hardware_counter("cycles")


def test_instances_and_default_tile():
    inst = capi.gemm_instances()
    assert len(inst) > 100
    tiles = {(i["dtype"], bool(i["conv"]), tuple(i["tile"])) for i in inst}
    assert ("bfloat16", False, (256, 256, 64, 4, 2)) in tiles
    assert ("bfloat16", False, (256, 256, 64, 2, 4)) in tiles
    assert ("bfloat16", False, (256, 256, 32, 2, 4)) in tiles
    assert any(d == "float32" and c for d, c, _ in tiles)
    # large aligned fp32: the LDS-DMA fp32 kernel's tile when it fills the chip
    assert tuple(capi.default_tile("float32", False, 4096, 4096, 4096)[0]) == (256, 128, 32, 4, 2)
    assert tuple(capi.default_tile("float32", False, 2048, 2048, 2048)[0]) == (128, 128, 32, 2, 2)
    tile, split = capi.default_tile("bfloat16", False, 8192, 8192, 8192)
    assert tuple(tile) == (256, 256, 32, 2, 4) and split == 1
    # few 64x64 tiles over a deep K: split-K up to 1024 workgroups and 32
    # splits, >= 4 slabs per split; from 128 tiles only over K >= 512
    cases = {
        ("float32", True, 49, 512, 4608): ((64, 64, 16, 2, 2), 32),      # ResNet18_12: 8 tiles
        ("float32", True, 8 * 56 * 56, 64, 576): ((64, 64, 16, 2, 2), 1),  # C4: 392 tiles, direct conv
        ("float32", True, 68 * 68, 128, 256): ((64, 64, 16, 2, 2), 1),     # Yolo9000_09: 146 tiles, K 256
        ("float32", True, 112 * 112, 64, 576): ((64, 64, 16, 2, 2), 4),    # MobilNet_02: 196 tiles
        ("float32", False, 512, 512, 512): ((64, 64, 32, 2, 2), 4),        # 64 tiles, 4 slabs per split
        ("float32", False, 128, 4096, 8192): ((128, 128, 32, 2, 4), 8),    # Llama3_QK: LDS-DMA fp32, 256 WGs
        ("float32", False, 256, 8192, 4608): ((128, 128, 32, 2, 4), 2),    # Gemma27B_QKV: 128 tiles
        ("float32", False, 256, 3584, 8192): ((128, 128, 32, 2, 4), 4),    # Gemma9B_QK: 224 WGs
        ("float32", False, 256, 3072, 8192): ((64, 64, 32, 2, 2), 8),      # Gemma7B_QK: 192 would idle CUs
        ("float32", False, 128, 4096, 8000): ((64, 64, 32, 2, 2), 8),      # unaligned K: 64x64 split-K
        ("float32", False, 1000, 1104, 1200): ((64, 64, 32, 2, 2), 8),     # Polybench_large: unequal split
        ("float32", False, 256, 4608, 8192): ((64, 64, 32, 2, 2), 8),      # Gemma27B_QK: 2304 workgroups
        ("float32", False, 768, 768, 4096): ((64, 64, 32, 2, 2), 16),      # 144 tiles x 16
        ("float32", False, 256, 1024, 4096): ((64, 64, 32, 2, 2), 16),     # LDS-DMA splits would be 256 deep
        ("float32", False, 1024, 1024, 8192): ((128, 128, 32, 2, 4), 4),   # 64 tiles x 4, 2048 deep
        ("float32", False, 2000, 2304, 2600): ((64, 64, 32, 2, 2), 2),     # 1152 tiles, K >= 2048: split 2
        ("float32", False, 1536, 1536, 512): ((64, 64, 32, 2, 2), 1),      # 576 tiles over a short K
        ("float32", False, 2000, 2400, 2600): ((64, 64, 32, 2, 2), 1),     # 1200 tiles: split 2 passes 2304
        # bf16: ping-pong from 128 aligned 256x256 tiles, else 128x128x64 (split-K to 512
        # workgroups when that reaches 256), else the 64x64 rules
        ("bfloat16", False, 3072, 24576, 3072): ((256, 256, 32, 2, 4), 1),
        ("bfloat16", False, 2048, 4096, 256): ((256, 256, 32, 2, 4), 1),
        ("bfloat16", False, 256, 8192, 4608): ((128, 128, 64, 2, 2), 4),
        ("bfloat16", False, 2000, 2304, 2600): ((128, 128, 64, 2, 2), 1),
        ("bfloat16", False, 1000, 1104, 1200): ((64, 64, 64, 2, 2), 1),
        # bf16 convs: 128x128x64 from 256 such tiles over >= 96 filters; a split of
        # 4 or more moves to 128x64x64 when that still makes >= 256 workgroups
        ("bfloat16", True, 289, 28272, 1024): ((128, 128, 64, 2, 2), 1),     # Yolo9000_23
        ("bfloat16", True, 224 * 224, 96, 147): ((128, 128, 64, 2, 2), 1),   # SqueezeNet_00
        ("bfloat16", True, 136 * 136, 128, 576): ((64, 64, 64, 2, 2), 1),    # Yolo9000_04: 145 such tiles
        ("bfloat16", True, 272 * 272, 64, 288): ((64, 64, 64, 2, 2), 1),     # Yolo9000_02: 64 filters
        ("bfloat16", True, 34 * 34, 512, 2304): ((128, 64, 64, 2, 2), 4),    # Yolo9000_12
        ("bfloat16", True, 17 * 17, 1024, 4608): ((128, 64, 64, 2, 2), 8),   # Yolo9000_18
        ("bfloat16", True, 49, 512, 4608): ((64, 64, 64, 2, 2), 8),          # ResNet18_12: 49 pixels
        ("bfloat16", True, 28 * 28, 256, 2304): ((64, 64, 64, 2, 2), 8),     # MobilNet_05: 224 workgroups
        ("bfloat16", True, 17 * 17, 512, 1024): ((64, 64, 64, 2, 2), 4),     # Yolo9000_19: 96 workgroups
        # bf16 convs split K unequally up to 8 when the slabs do not divide
        ("bfloat16", True, 15 * 15, 384, 1728): ((64, 64, 64, 2, 2), 4),     # AlexNet_02: 27 slabs
        ("bfloat16", True, 15 * 15, 256, 3456): ((64, 64, 64, 2, 2), 8),     # AlexNet_03
        ("bfloat16", True, 56 * 56, 64, 576): ((64, 64, 64, 2, 2), 2),       # ResNet18_02: 9 slabs
        ("bfloat16", True, 14 * 14, 512, 4608): ((64, 64, 64, 2, 2), 8),     # MobilNet_07: 16 needs whole slabs
        ("bfloat16", True, 7 * 7, 1024, 9216): ((64, 64, 64, 2, 2), 16),     # MobilNet_09: whole slabs
        ("float32", True, 56 * 56, 64, 576): ((64, 64, 16, 2, 2), 8),        # ResNet18_02: 36 slabs, 8 unequal
        ("float32", True, 15 * 15, 384, 1728): ((64, 64, 16, 2, 2), 8),      # fp32 AlexNet_02: unequal split 8
        ("float32", True, 27 * 27, 192, 432): ((64, 64, 16, 2, 2), 4),       # SqueezeNet_13: K % 64 != 0
        ("float32", True, 27 * 27, 32, 256): ((64, 64, 16, 2, 2), 4),        # SqueezeNet_08: 32 filters
        ("float32", True, 112 * 112, 32, 288): ((64, 64, 32, 2, 2), 1),      # MobilNet_01: no split
        ("float32", True, 272 * 272, 64, 288): ((64, 64, 32, 2, 2), 1),     # Yolo9000_02: no split
    }
    for args, (tile, split) in cases.items():
        got = capi.default_tile(*args)
        assert (tuple(got[0]), got[1]) == (tile, split), (args, got)


def test_conv_default_tile_direct_block():
    # a 1x4-wave direct conv block replaces the 8x8 one for windows wider
    # than 1x1 whose blocks fit in one wave of 256 CUs: 7x14 where its blocks
    # do, else 8x14
    def tile(n, h, w, c, f, r, pad):
        d = capi.Conv2dDesc(dtype=capi.XTC_HIP_F32, N=n, H=h, W=w, C=c, F=f, R=r, S=r, stride_h=1, stride_w=1,
                            pad_top=pad, pad_bottom=pad, pad_left=pad, pad_right=pad)
        return capi.conv2d_default_tile(d)[0]

    assert tile(8, 56, 56, 64, 64, 3, 1) == (98, 64, 16, 1, 4)       # C4: 256 blocks (224 of 8x14)
    assert tile(1, 70, 70, 128, 256, 3, 0) == (98, 64, 16, 1, 4)     # Yolo9000_08: 200 blocks
    assert tile(1, 115, 226, 64, 64, 3, 0) == (112, 64, 16, 1, 4)    # 113x224: 272 of 7x14, 240 of 8x14
    assert tile(1, 138, 138, 64, 128, 3, 0) == (64, 64, 16, 2, 2)    # Yolo9000_04: 340 blocks
    assert tile(1, 68, 68, 256, 128, 1, 0) == (64, 64, 16, 2, 2)     # Yolo9000_09: 1x1
    assert tile(1, 56, 56, 64, 64, 1, 0) == (64, 64, 16, 2, 2)       # ResNet18_03: 1x1


def test_datasheet_flops_are_half_the_flop_rate():
    lib = capi.lib()
    assert lib.xtc_hip_datasheet_flops(b"float32") == pytest.approx(157.3e12 / 2)
    assert lib.xtc_hip_datasheet_flops(b"bfloat16") == pytest.approx(2516.6e12 / 2)
    assert lib.xtc_hip_datasheet_flops(b"int4") == 0.0
    # the measured peak needs a device: without one it reports an error
    assert lib.xtc_hip_evaluate_flops(b"float32") == 0.0 and "xtc_hip_init" in capi.last_error()
    # a dtype with no MFMA peak reports 0.0 through the device interface, as the
    # explorer's peak_time expects, without touching a device
    from xtc_amd.runtimes.hip.device import HipDevice

    assert HipDevice().evaluate_flops("int4") == 0.0


def test_compile_service_refuses_to_start_after_the_gpu(monkeypatch):
    from xtc_amd.backends.hip import compiler

    class _Lib:
        @staticmethod
        def xtc_hip_stream():
            return 0x1234  # a library stream exists: xtc_hip_init has run

    monkeypatch.setattr(compiler.CompileService, "_server_started", False)
    monkeypatch.setattr(compiler.capi, "lib", lambda: _Lib)
    monkeypatch.setattr(compiler.capi, "library_available", lambda: True)
    with pytest.raises(RuntimeError, match="start_server"):
        compiler.CompileService(1)


def test_device_count_without_gpu_is_safe():
    n = capi.lib().xtc_hip_device_count()
    assert n >= 0
    assert isinstance(capi.lib().xtc_hip_last_error(), (bytes, type(None)))
    _ = ctypes  # ctypes types come from capi


def test_for_node_schedules_several_nodes():
    b = Backend(_mlp())
    sch = b.get_scheduler()
    sch.for_node("fc1").tile("i", {"i1": 256, "i2": 64})
    sch.for_node("fc2").tile("j", {"j1": 128})
    s = sch.schedule()
    assert s.node("fc1").tiles["i"] == {"i1": 256, "i2": 64}
    assert s.node("fc2").tiles["j"] == {"j1": 128}
    # a scheduler built on the shared states sees the same schedule
    other = b.get_scheduler(nodes_schedulers=sch.nodes_schedulers, default_node="fc1")
    assert other.schedule().node("fc2").tiles["j"] == {"j1": 128}


# ---------------------------------------------------------------- bench workloads

def test_bench_schedules_map_exactly():
    from xtc_amd import configs

    want = {
        "C1": {"C": ((32, 32, 16, 1, 1), 4, 0)},
        "C2": {"C": ((128, 256, 32, 2, 4), 1, 2)},
        "C3a": {"C": ((256, 256, 32, 2, 4), 1, 0)},
        "C5": {"fc1": ((128, 256, 32, 2, 4), 1, 0), "fc2": ((128, 128, 32, 2, 4), 2, 0)},
    }
    for cfg, kernels in want.items():
        b = Backend(configs.graph(cfg))
        sch = configs.apply_schedule(b.get_scheduler(), cfg)
        got = b.get_compiler(schedule_policy="strict").kernel_configs(sch.schedule())
        assert {n: (c.tile, c.split_k, c.stages) for n, c in got.items()} == kernels, cfg


@pytest.mark.parametrize("cfg", ["C1", "C3b", "C4", "C5"])
def test_bench_inputs_are_the_oracle_inputs(cfg):
    from oracle import reference as ref
    from xtc_amd import configs

    got = configs.inputs(cfg, configs.graph(cfg))
    want = ref.config_inputs(cfg)
    assert len(got) == len(want)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
