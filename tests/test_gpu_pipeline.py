# SPDX-License-Identifier: BSD-3-Clause
"""End-to-end parity on the GPU: XTC graph -> HipBackend -> Scheduler ->
Compiler -> payload .so -> HipEvaluator, for every BASELINE configuration.

Two checks per configuration:
  * XTC's own validation (HipEvaluator(validate=True)): np_init integer
    inputs 1..9, compared with the graph's numpy interpreter by np.allclose,
    as the reference's `CODE: 0` tests do
    (tests/filecheck/backends/test_matmul_mlir.py:150);
  * seeded BASELINE inputs against the float64 oracle with the tolerance
    max|out-ref| / (sqrt(K) max|A| max|B|) <= 1e-4 (fp32) / 1e-2 (bf16 inputs).
For the 8192^3 GEMM the oracle checks a band of rows (a full float64 8192^3
product takes minutes on the host); the integer check covers every element.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import xtc_amd.graphs.xtc.op as O
from oracle import reference as ref
from xtc_amd.backends.hip import Backend

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 1e-2


def _matmul_graph(m, n, k, dtype, name="matmul"):
    a = O.tensor((m, k), dtype, name="A")
    b = O.tensor((k, n), dtype, name="B")
    with O.graph(name=name) as gb:
        O.matmul(a, b, name="C", **({"out_dtype": "float32"} if dtype == "bfloat16" else {}))
    return gb.graph


def _conv_graph(relu=True, pad=1):
    x = O.tensor((8, 56, 56, 64), "float32", name="I")
    w = O.tensor((3, 3, 64, 64), "float32", name="W")
    with O.graph(name="conv_relu") as gb:
        p = O.pad2d(x, padding=pad, axes=(1, 2), name="pad")
        c = O.conv2d(p, w, name="conv")
        if relu:
            O.relu(c, name="relu")
    return gb.graph


def _mlp_graph():
    x = O.tensor((2048, 1024), "float32", name="X")
    w1 = O.tensor((1024, 4096), "float32", name="W1")
    w2 = O.tensor((4096, 1024), "float32", name="W2")
    with O.graph(name="mlp") as gb:
        h = O.relu(O.matmul(x, w1, name="fc1"), name="act")
        O.matmul(h, w2, name="fc2")
    return gb.graph


def _compile(graph, tiles=None, node=None, **kw):
    backend = Backend(graph)
    sch = backend.get_scheduler(default_node=node) if node else backend.get_scheduler()
    for dim, t in (tiles or {}).items():
        sch.tile(dim, t)
    return backend.get_compiler(**kw).compile(sch.schedule())


def _run(module, inputs):
    outs = [np.empty(t.constant_shape, np.float32) for t in module.graph.outputs_types]
    res, code, msg = module.get_evaluator(parameters=(inputs, outs), repeat=1, number=1, min_repeat_ms=0).evaluate()
    assert code == 0, msg
    return outs


GRAPHS = {
    "C1": lambda: _matmul_graph(512, 512, 512, "float32"),
    "C2": lambda: _matmul_graph(4096, 4096, 4096, "float32"),
    "C3a": lambda: _matmul_graph(8192, 8192, 8192, "bfloat16", "matmul_bf16"),
    "C3b": lambda: _matmul_graph(16, 8192, 8192, "bfloat16", "matmul_skinny"),
    "C4": _conv_graph,
    "C5": _mlp_graph,
}


@pytest.mark.parametrize("cfg", list(GRAPHS))
def test_xtc_validate_integer_inputs(cfg):
    module = _compile(GRAPHS[cfg]())
    # C5's second GEMM sums integers past 2**24, so fp32 results depend on the
    # summation order: a K-sequential fp32 loop (the order of the reference's
    # llvmir loop nest, restated in oracle/cpu_backend.c) is 2.85e-5 off numpy
    # there and fails np.allclose's default rtol=1e-5 just like the GPU
    # (tests/test_oracle.py::test_c5_integer_rounding_is_order_dependent).
    tol = {"rtol": 1e-4} if cfg == "C5" else {}
    res, code, msg = module.get_evaluator(validate=True, repeat=1, number=1, min_repeat_ms=0, **tol).evaluate()
    assert code == 0, msg
    assert len(res) == 1 and res[0] > 0


def test_c1_seeded():
    a, b = ref.config_inputs("C1")
    (out,) = _run(_compile(GRAPHS["C1"]()), [a, b])
    assert ref.scaled_error(out, ref.matmul(a, b), 512, 1.0, 1.0) <= TOL_F32


def test_c2_seeded_tuned():
    a, b = ref.config_inputs("C2")
    tiles = {"i": {"i1": 256, "i2": 64}, "j": {"j1": 128, "j2": 64}, "k": {"k1": 16}}
    module = _compile(GRAPHS["C2"](), tiles, schedule_policy="strict")
    (out,) = _run(module, [a, b])
    rows = slice(0, 4096, 7)
    expect = ref.matmul(a[rows], b)
    assert ref.scaled_error(out[rows], expect, 4096, np.abs(a).max(), np.abs(b).max()) <= TOL_F32


def test_c3a_seeded_tuned_rows():
    a, b = ref.config_inputs("C3a")
    tiles = {"i": {"i1": 256, "i2": 64}, "j": {"j1": 256, "j2": 128}, "k": {"k1": 64}}
    module = _compile(GRAPHS["C3a"](), tiles, schedule_policy="strict")
    (out,) = _run(module, [a, b])
    for rows in (slice(0, 64), slice(4032, 4160), slice(8192 - 64, 8192)):
        expect = ref.matmul(a[rows], b)
        assert ref.scaled_error(out[rows], expect, 8192, np.abs(a).max(), np.abs(b).max()) <= TOL_BF16
    # column band through the whole M range
    cols = slice(8192 - 96, 8192)
    expect = a.astype(np.float64) @ b[:, cols].astype(np.float64)
    assert ref.scaled_error(out[:, cols], expect, 8192, np.abs(a).max(), np.abs(b).max()) <= TOL_BF16


# The schedules bench.py measures (xtc_amd.configs.SCHEDULES), each compiled
# with the strict policy and checked on the seeded BASELINE inputs.
BENCH_KERNELS = {
    "C1": {"C": ((32, 32, 16, 1, 1), 4, 0)},
    "C2": {"C": ((128, 256, 32, 2, 4), 1, 2)},
    "C3a": {"C": ((256, 256, 32, 2, 4), 1, 0)},
    "C5": {"fc1": ((128, 256, 32, 2, 4), 1, 0), "fc2": ((128, 128, 32, 2, 4), 2, 0)},
}


def _bench_module(cfg):
    from xtc_amd import configs

    backend = Backend(configs.graph(cfg))
    sch = configs.apply_schedule(backend.get_scheduler(), cfg)
    module = backend.get_compiler(schedule_policy="strict").compile(sch.schedule())
    got = {node: (c.tile, c.split_k, c.stages) for node, c in module.configs.items()}
    if os.environ.get("XTC_HIP_GENERIC_GEMM") == "1":
        # every tile on the generic template: its one depth is the default
        want = {n: (t, sk, 0) for n, (t, sk, _) in BENCH_KERNELS[cfg].items()}
    else:
        want = BENCH_KERNELS[cfg]
    assert got == want, got
    return module


def test_bench_schedule_c1_seeded():
    a, b = ref.config_inputs("C1")
    (out,) = _run(_bench_module("C1"), [a, b])
    assert ref.scaled_error(out, ref.matmul(a, b), 512, 1.0, 1.0) <= TOL_F32


def test_bench_schedule_c2_seeded():
    a, b = ref.config_inputs("C2")
    (out,) = _run(_bench_module("C2"), [a, b])
    amax = (np.abs(a).max(), np.abs(b).max())
    rows = slice(3, 4096, 9)
    assert ref.scaled_error(out[rows], ref.matmul(a[rows], b), 4096, *amax) <= TOL_F32
    cols = slice(4096 - 80, 4096)
    expect = a.astype(np.float64) @ b[:, cols].astype(np.float64)
    assert ref.scaled_error(out[:, cols], expect, 4096, *amax) <= TOL_F32


def test_bench_schedule_c3a_seeded_rows_and_columns():
    a, b = ref.config_inputs("C3a")
    (out,) = _run(_bench_module("C3a"), [a, b])
    amax = (np.abs(a).max(), np.abs(b).max())
    # row bands across the first, a middle and the last tile rows
    for rows in (slice(0, 64), slice(4000, 4160), slice(8192 - 96, 8192)):
        assert ref.scaled_error(out[rows], ref.matmul(a[rows], b), 8192, *amax) <= TOL_BF16
    # column bands through the whole M range: every tile row, two tile columns
    for cols in (slice(0, 48), slice(8192 - 96, 8192)):
        expect = a.astype(np.float64) @ b[:, cols].astype(np.float64)
        assert ref.scaled_error(out[:, cols], expect, 8192, *amax) <= TOL_BF16


def test_bench_schedule_c5_seeded():
    x, w1, w2 = ref.config_inputs("C5")
    (out,) = _run(_bench_module("C5"), [x, w1, w2])
    h = ref.relu(ref.matmul(x, w1))
    assert ref.scaled_error(out, ref.matmul(h, w2), 4096, np.abs(h).max(), np.abs(w2).max()) <= TOL_F32


def test_c3b_seeded():
    a, b = ref.config_inputs("C3b")
    (out,) = _run(_compile(GRAPHS["C3b"]()), [a, b])
    assert ref.scaled_error(out, ref.matmul(a, b), 8192, np.abs(a).max(), np.abs(b).max()) <= TOL_BF16


def test_c4_seeded_pad_conv_relu():
    x, w = ref.config_inputs("C4")
    module = _compile(GRAPHS["C4"]())
    assert [ln.kind for ln in module.plan.launches] == ["conv2d"], "pad and relu must be fused"
    (out,) = _run(module, [x, w])
    xp = ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)])
    expect = ref.relu(ref.conv2d(xp, w))
    assert ref.scaled_error(out, expect, 576, np.abs(xp).max(), np.abs(w).max()) <= TOL_F32


def test_c5_seeded_mlp():
    x, w1, w2 = ref.config_inputs("C5")
    module = _compile(GRAPHS["C5"]())
    assert [ln.kind for ln in module.plan.launches] == ["matmul", "matmul"], "relu must be fused"
    (out,) = _run(module, [x, w1, w2])
    h = ref.relu(ref.matmul(x, w1))
    expect = ref.matmul(h, w2)
    assert ref.scaled_error(out, expect, 4096, np.abs(h).max(), np.abs(w2).max()) <= TOL_F32


def test_unfused_pad_and_relu_kernels():
    # pad on the channel axis cannot fold into the conv loader; a relu with a
    # second user cannot fold into the GEMM epilogue
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, (2, 9, 9, 6)).astype(np.float32)
    w = rng.uniform(-1, 1, (3, 3, 8, 16)).astype(np.float32)
    xi = O.tensor(x.shape, "float32", name="I")
    wi = O.tensor(w.shape, "float32", name="W")
    with O.graph(name="unfused") as gb:
        p = O.pad(xi, padding={3: (1, 1)}, constant_value=0.5)
        c = O.conv2d(p, wi, stride=2)
        r = O.relu(c, threshold=0.25)
        O.outputs(r, c)
    module = _compile(gb.graph)
    kinds = [ln.kind for ln in module.plan.launches]
    assert kinds == ["pad", "conv2d", "relu"], kinds
    r_out, c_out = _run(module, [x, w])
    xp = ref.pad(x, [(0, 0), (0, 0), (0, 0), (1, 1)], 0.5)
    conv = ref.conv2d(xp, w, (2, 2))
    assert ref.scaled_error(c_out, conv, 72, 1.0, 1.0) <= TOL_F32
    np.testing.assert_array_equal(r_out, np.maximum(c_out, 0.25))


def test_ndarray_parameters_on_the_device():
    """NDArray (runtimes/types/ndarray.py:23-237) with the HIP device as its
    runtime holds its tensor in HBM; an evaluator takes NDArrays as
    parameters and writes the payload's outputs back into them."""
    from xtc_amd.runtimes.hip.device import HipDevice
    from xtc_amd.runtimes.types.ndarray import NDArray

    rng = np.random.default_rng(8)
    a = rng.uniform(-1, 1, (64, 96)).astype(np.float32)
    b = rng.uniform(-1, 1, (96, 32)).astype(np.float32)
    dev = HipDevice()
    na, nb = NDArray(a, runtime=dev), NDArray(b, runtime=dev)
    nc = NDArray(np.zeros((64, 32), np.float32), runtime=dev)
    assert na.is_on_device() and na.data.value != a.ctypes.data and np.array_equal(na.numpy(), a)
    module = _compile(_matmul_graph(64, 32, 96, "float32"))
    _, code, msg = module.get_evaluator(parameters=([na, nb], [nc]), repeat=1, number=1, min_repeat_ms=0).evaluate()
    assert code == 0, msg
    assert ref.scaled_error(nc.numpy(), ref.matmul(a, b), 96, 1.0, 1.0) <= TOL_F32
    t = NDArray(a, runtime=dev, layout=[1, 0])  # stored transposed in HBM, read back logical
    assert t.shape == (96, 64) and np.array_equal(t.numpy(), a)


def test_bias_add_epilogue():
    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, (96, 64)).astype(np.float32)
    b = rng.uniform(-1, 1, (64, 48)).astype(np.float32)
    bias = rng.uniform(-1, 1, (48,)).astype(np.float32)
    ai, bi, ci = O.tensor(a.shape, "float32"), O.tensor(b.shape, "float32"), O.tensor(bias.shape, "float32")
    with O.graph(name="linear") as gb:
        O.relu(O.bias_add(O.matmul(ai, bi), ci))
    module = _compile(gb.graph)
    assert [ln.kind for ln in module.plan.launches] == ["matmul"]
    (out,) = _run(module, [a, b, bias])
    expect = np.maximum(ref.matmul(a, b) + bias, 0)
    assert ref.scaled_error(out, expect, 64, 1.0, 1.0) <= TOL_F32


def test_bf16_output_cast():
    rng = np.random.default_rng(5)
    a = ref.round_bf16(rng.uniform(-1, 1, (64, 128)).astype(np.float32))
    b = ref.round_bf16(rng.uniform(-1, 1, (128, 32)).astype(np.float32))
    ai, bi = O.tensor(a.shape, "bfloat16"), O.tensor(b.shape, "bfloat16")
    with O.graph(name="mm_bf16_out") as gb:
        O.matmul(ai, bi)
    module = _compile(gb.graph)
    assert [ln.kind for ln in module.plan.launches] == ["matmul", "cast"]
    (out,) = _run(module, [a, b])
    expect = ref.round_bf16(ref.matmul(a, b).astype(np.float32))
    # fp32 accumulation then one rounding to bf16: at most one bf16 ulp apart
    assert np.all(np.abs(out - expect) <= np.abs(expect) * 2.0**-7 + 1e-6)


def test_split_k_schedule():
    rng = np.random.default_rng(6)
    a = rng.uniform(-1, 1, (64, 4096)).astype(np.float32)
    b = rng.uniform(-1, 1, (4096, 128)).astype(np.float32)
    graph = _matmul_graph(64, 128, 4096, "float32", "splitk")
    backend = Backend(graph)
    sch = backend.get_scheduler()
    sch.tile("i", {"i1": 64})
    sch.tile("j", {"j1": 64})
    sch.tile("k", {"k1": 512, "k2": 32})
    sch.parallelize(["k"])
    module = backend.get_compiler(schedule_policy="strict").compile(sch.schedule())
    assert module.configs["C"].split_k == 8
    (out,) = _run(module, [a, b])
    assert ref.scaled_error(out, ref.matmul(a, b), 4096, 1.0, 1.0) <= TOL_F32


def test_evaluator_timing_and_gpu_time_counter():
    module = _compile(GRAPHS["C1"]())
    res, code, msg = module.get_evaluator(repeat=3, number=1, min_repeat_ms=20).evaluate()
    assert code == 0, msg and len(res) == 3
    res, code, msg = module.get_evaluator(
        repeat=2, number=1, min_repeat_ms=20, pmu_counters=["gpu.time", "gpu.clocks", "bogus"]
    ).evaluate()
    assert code == 0, msg
    assert len(res) == 6
    assert res[0] > 0 and abs(res[1] - res[0] * 1e9) <= 1e-3 * res[1] and res[2] == -1


def test_validation_failure_is_reported():
    module = _compile(GRAPHS["C1"]())
    bad = lambda *args: [np.copyto(o, 0) for o in args[2:]]  # noqa: E731
    res, code, msg = module.get_evaluator(validate=True, reference_impl=bad, min_repeat_ms=0).evaluate()
    assert code == 1 and "validation" in msg


def _layout_graph(m, n, k, dtype, la, lb, name):
    a = O.tensor((m, k), dtype, name="A", layout=[1, 0] if la else None)
    b = O.tensor((k, n), dtype, name="B", layout=[1, 0] if lb else None)
    with O.graph(name=name) as gb:
        O.matmul(a, b, name="C", **({"out_dtype": "float32"} if dtype == "bfloat16" else {}))
    return gb.graph


@pytest.mark.parametrize("la,lb", [(True, False), (False, True), (True, True)])
def test_operand_layouts_validate(la, lb):
    # tests/filecheck/backends/test_matmul_mlir_layout.py: A (4x512) with
    # layout [1, 0], executed with validate=True -> CODE: 0
    module = _compile(_layout_graph(4, 32, 512, "float32", la, lb, "matmul_layout"))
    assert module.get_executor(validate=True).execute() == 0
    # the bf16 C3a kernel family with B^T read natively (and A^T staged)
    module = _compile(_layout_graph(512, 512, 512, "bfloat16", la, lb, "matmul_layout_bf16"),
                      tiles={"i": {"i1": 256, "i2": 128}, "j": {"j1": 256, "j2": 64}, "k": {"k1": 64}})
    res, code, msg = module.get_evaluator(validate=True, repeat=1, number=1, min_repeat_ms=0).evaluate()
    assert code == 0, msg


def test_operand_layouts_seeded_logical_parameters():
    # parameters are logical arrays; the evaluator stores [1, 0] inputs
    # transposed on the device, like the reference's NDArray
    rng = np.random.default_rng(7)
    a = ref.round_bf16(rng.uniform(-1, 1, (256, 1024)).astype(np.float32))
    b = ref.round_bf16(rng.uniform(-1, 1, (1024, 768)).astype(np.float32))
    module = _compile(_layout_graph(256, 768, 1024, "bfloat16", False, True, "nt_seeded"),
                      tiles={"i": {"i1": 256, "i2": 128}, "j": {"j1": 256, "j2": 64}, "k": {"k1": 64}})
    (out,) = _run(module, [a, b])
    assert ref.scaled_error(out, ref.matmul(a, b), 1024, 1.0, 1.0) <= TOL_BF16


# split() of i or j: one launch per segment on strided sub-views, each segment
# with its own tiles (src/xtc/itf/schd/scheduler.py:65-81)
SPLIT_CASES = [
    # (dtype, layouts, M, N, K, i cut, j cut in the second i segment, relu)
    ("float32", (False, False), 384, 256, 512, 256, 128, True),
    ("float32", (True, True), 300, 200, 96, 100, 36, False),  # ragged, offsets not 16-byte aligned
    ("bfloat16", (False, True), 512, 512, 256, 256, 256, False),  # B^T read natively per piece
    ("bfloat16", (True, False), 96, 1024, 8192, 16, 512, True),  # skinny first piece
]


def _split_graph(dtype, layouts, m, n, k, relu):
    a = O.tensor((m, k), dtype, name="A", layout=[1, 0] if layouts[0] else None)
    b = O.tensor((k, n), dtype, name="B", layout=[1, 0] if layouts[1] else None)
    with O.graph(name="matmul_split") as gb:
        c = O.matmul(a, b, name="C", **({"out_dtype": "float32"} if dtype == "bfloat16" else {}))
        if relu:
            O.relu(c, name="relu")
    return gb.graph


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[f"{c[0]}-{c[2]}x{c[3]}x{c[4]}-ta{int(c[1][0])}tb{int(c[1][1])}"
                                                   for c in SPLIT_CASES])
def test_split_schedule_parity(case):
    from xtc_amd.backends.hip.mapping import SplitConfig

    dtype, layouts, m, n, k, icut, jcut, relu = case
    print(f"[split] {case}", flush=True)
    backend = Backend(_split_graph(dtype, layouts, m, n, k, relu))
    sch = backend.get_scheduler()
    sch.split("i", {"i_lo": 0, "i_hi": icut})
    if icut <= 16:
        tiles = {}  # the library default: the skinny bf16 kernel
    elif dtype == "bfloat16" and m >= 256 and icut % 256 == 0:
        tiles = {"i": {"i1": 256, "i2": 128}, "j": {"j1": 256, "j2": 64}, "k": {"k1": 32}}
    else:
        tiles = {"i": {"i1": 64}, "j": {"j1": 64}, "k": {"k1": 32 if dtype == "float32" else 64}}
    for dim, t in tiles.items():
        sch.tile(dim, t, root="./i_lo")
    sch.split("j", {"j_a": 0, "j_b": jcut}, root="./i_hi")
    sch.tile("i", {"i1": 32}, root="./i_hi/j_b")
    sch.tile("j", {"j1": 32}, root="./i_hi/j_b")
    sch.tile("k", {"k1": 16 if dtype == "float32" else 32}, root="./i_hi/j_b")
    module = backend.get_compiler().compile(sch.schedule())
    cfg = module.configs["C"]
    assert isinstance(cfg, SplitConfig) and len(cfg.pieces) == 3, cfg
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    if dtype == "bfloat16":
        a, b = ref.round_bf16(a), ref.round_bf16(b)
    (out,) = _run(module, [a, b])
    want = ref.matmul(a, b)
    if relu:
        want = np.maximum(want, 0.0)
    assert ref.scaled_error(out, want, k, 1.0, 1.0) <= (TOL_F32 if dtype == "float32" else TOL_BF16)
    # integer inputs: every piece exact, the XTC validation path included
    res, code, msg = module.get_evaluator(validate=True, repeat=1, number=1, min_repeat_ms=0).evaluate()
    assert code == 0, msg


def test_measured_mfma_peak():
    # the register-only MFMA probe behind evaluate_flops (FMA/s): at most the
    # datasheet peak, and zeros run at least as fast as random operands
    from xtc_amd.runtimes.hip.device import HipDevice

    dev = HipDevice(0)
    for dtype in ("float32", "bfloat16"):
        sheet = dev.datasheet_flops(dtype)
        ref_ops = dev.evaluate_flops(dtype)
        zero = dev.evaluate_flops(dtype, "zero")
        rand = dev.evaluate_flops(dtype, "random")
        print(f"[peak] {dtype}: reference operands {ref_ops / sheet:.3f}, zeros {zero / sheet:.3f}, "
              f"random {rand / sheet:.3f} of the datasheet", flush=True)
        for v in (ref_ops, zero, rand):
            assert 0.4 * sheet < v <= 1.02 * sheet
        assert zero >= 0.97 * rand


@pytest.mark.parametrize("opname", ["matmul", "conv2d"])
def test_reference_graph_files_validate(opname):
    # the reference's tests/graphs/*.graph.yaml, run with XTC's validation
    from pathlib import Path

    with O.graph() as gb:
        gb.load(Path(__file__).resolve().parent / "golden" / "graphs" / f"{opname}.graph.yaml")
    module = _compile(gb.graph)
    res, code, msg = module.get_evaluator(validate=True, repeat=1, number=1, min_repeat_ms=0).evaluate()
    assert code == 0, msg
