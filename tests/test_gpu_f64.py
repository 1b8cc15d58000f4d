# SPDX-License-Identifier: BSD-3-Clause
"""float64 graphs on the GPU: the fp64 MFMA GEMM and implicit-GEMM conv, the
fp64 relu and pad, through the C-ABI and through the XTC pipeline, against
the float64 oracle.

The reference lowers float64 matmul, conv2d, relu and pad
(src/xtc/backends/mlir/MlirOps.py:194-195,234,339,463,616) and validates
with np.allclose against numpy's float64 forward.  Bars here: bit-exact on
integer known-answer inputs (every product and partial sum is an integer
below 2^53); on seeded uniform inputs
max|out - ref| / (sqrt(K) max|A| max|B|) <= 1e-12, against a float64 oracle
that sums in another order (the order-dependent rounding of an fp64 sum of K
terms of that size is about 1e-16 sqrt(K) in those units).
"""

from __future__ import annotations

import csv
import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import reference as ref
from xtc_amd.runtimes.hip import capi
from xtc_amd.runtimes.hip.buffer import DeviceBuffer, ensure_device

pytestmark = pytest.mark.gpu

TOL_F64 = 1e-12
ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module", autouse=True)
def device():
    ensure_device(0)
    yield


def _dev(a: np.ndarray) -> DeviceBuffer:
    return DeviceBuffer.from_numpy(np.ascontiguousarray(a, dtype=np.float64))


def run_matmul64(a, b, tile=None, split_k=0, relu=False, thr=0.0, bias=None, trans_a=False, trans_b=False):
    """C = A @ B in fp64 through xtc_hip_matmul; a/b are the logical operands,
    stored transposed on the device when trans_a / trans_b."""
    M, K = a.shape
    N = b.shape[1]
    A = _dev(a.T if trans_a else a)
    B = _dev(b.T if trans_b else b)
    C = DeviceBuffer(M * N * 8)
    bias_buf = _dev(bias) if bias is not None else None
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_F64, M=M, N=N, K=K, split_k=split_k, xcd_remap=1, relu=int(relu),
                        relu_threshold=thr, relu_threshold_f64=thr, trans_a=int(trans_a), trans_b=int(trans_b))
    if tile is not None:
        d.tile = capi.Tile(*tile)
    L = capi.lib()
    capi.check(L.xtc_hip_matmul(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, bias_buf.c_ptr if bias_buf else None),
               "matmul f64")
    capi.check(L.xtc_hip_synchronize(), "sync")
    return C.to_numpy((M, N), np.float64)


def run_conv64(x, w, stride=(1, 1), pads=(0, 0, 0, 0), pad_value=0.0, tile=None, split_k=0, relu=False, thr=0.0,
               bias=None):
    n, h, wd, c = x.shape
    r, s, _, f = w.shape
    I, W = _dev(x), _dev(w)
    hp, wp = h + pads[0] + pads[1], wd + pads[2] + pads[3]
    oh, ow = (hp - r) // stride[0] + 1, (wp - s) // stride[1] + 1
    O = DeviceBuffer(n * oh * ow * f * 8)
    d = capi.Conv2dDesc(dtype=capi.XTC_HIP_F64, N=n, H=h, W=wd, C=c, F=f, R=r, S=s, stride_h=stride[0],
                        stride_w=stride[1], pad_top=pads[0], pad_bottom=pads[1], pad_left=pads[2], pad_right=pads[3],
                        pad_value=pad_value, pad_value_f64=pad_value, split_k=split_k, xcd_remap=1, relu=int(relu),
                        relu_threshold=thr, relu_threshold_f64=thr)
    if tile is not None:
        d.tile = capi.Tile(*tile)
    bias_buf = _dev(bias) if bias is not None else None
    L = capi.lib()
    capi.check(L.xtc_hip_conv2d(ctypes.byref(d), I.c_ptr, W.c_ptr, O.c_ptr, bias_buf.c_ptr if bias_buf else None),
               "conv2d f64")
    capi.check(L.xtc_hip_synchronize(), "sync")
    return O.to_numpy((n, oh, ow, f), np.float64)


def _uniform(seed, shape, low=-1.0, high=1.0):
    return np.random.default_rng(seed).uniform(low, high, size=shape)


F64_TILES = [i["tile"] for i in capi.gemm_instances() if i["dtype"] == "float64" and not i["conv"]]
F64_CONV_TILES = [i["tile"] for i in capi.gemm_instances() if i["dtype"] == "float64" and i["conv"]]


# ------------------------------------------------------------------ matmul


@pytest.mark.parametrize("tile", F64_TILES)
def test_matmul_f64_integer_kat_exact_every_tile(tile):
    # ragged against every tile (M, N not multiples of the block), K over
    # several slabs: exact, so the MFMA lane layout and the permuted k order
    # are right on every element
    M, N, K = 200, 146, 96
    a = ref.np_init((M, K), "float64")
    b = ref.np_init((K, N), "float64")
    np.testing.assert_array_equal(run_matmul64(a, b, tile=tile), ref.matmul(a, b))


def test_matmul_f64_distinct_entries_exact():
    # entries that identify their row and column: a transposed or shifted
    # output element would not match
    M, N, K = 64, 48, 32
    a = np.add.outer(np.arange(M) * 1000.0, np.arange(K))
    b = np.add.outer(np.arange(K) * 0.5, np.arange(N) * 64.0)
    np.testing.assert_array_equal(run_matmul64(a, b, tile=(32, 32, 16, 1, 1)), a @ b)


@pytest.mark.parametrize("shape,split_k", [((512, 512, 512), 0), ((256, 192, 2048), 4), ((64, 80, 4096), 16),
                                           ((1000, 700, 300), 0)])
def test_matmul_f64_seeded(shape, split_k):
    M, N, K = shape
    a, b = _uniform(1, (M, K)), _uniform(2, (K, N))
    out = run_matmul64(a, b, split_k=split_k)
    assert ref.scaled_error(out, ref.matmul(a, b), K, 1.0, 1.0) <= TOL_F64


def test_matmul_f64_bias_relu_threshold_and_nan():
    M, N, K = 130, 66, 70
    a, b = _uniform(3, (M, K)), _uniform(4, (K, N))
    a[5, 7] = np.nan  # row 5 is NaN everywhere: relu keeps NaN (numpy maximum)
    bias = _uniform(5, (N,))
    out = run_matmul64(a, b, relu=True, thr=0.1, bias=bias)
    want = ref.relu(ref.matmul(a, b) + bias, 0.1)
    assert np.isnan(out[5]).all()
    mask = ~np.isnan(want)
    assert ref.scaled_error(out[mask], want[mask], K, 1.0, 1.0) <= TOL_F64
    assert (out[mask] >= 0.1).all()


@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (True, True)])
def test_matmul_f64_transposed_operands(ta, tb):
    M, N, K = 96, 160, 128
    a, b = ref.np_init((M, K), "float64"), ref.np_init((K, N), "float64")
    np.testing.assert_array_equal(run_matmul64(a, b, trans_a=ta, trans_b=tb), ref.matmul(a, b))


def test_matmul_f64_odd_shapes_take_the_scalar_kernel():
    # K odd: no 16-byte rows, the scalar fp64 kernel; still exact
    M, N, K = 33, 17, 31
    a, b = ref.np_init((M, K), "float64"), ref.np_init((K, N), "float64")
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_F64, M=M, N=N, K=K)
    assert capi.matmul_pipeline_depths(d) == [1]
    np.testing.assert_array_equal(run_matmul64(a, b), ref.matmul(a, b))


def test_matmul_f64_pipeline_depth_and_unknown_tile():
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_F64, M=512, N=512, K=512, tile=capi.Tile(64, 64, 16, 2, 2))
    assert capi.matmul_pipeline_depths(d) == [2]
    d.tile = capi.Tile(256, 256, 32, 2, 4)  # a bf16 tile: no fp64 instance
    with pytest.raises(capi.HipError, match="no fp64 matmul kernel instance"):
        capi.matmul_pipeline_depths(d)


# ------------------------------------------------------------------ conv2d


@pytest.mark.parametrize("c,f,stride,pads", [(64, 64, (1, 1), (1, 1, 1, 1)), (6, 32, (2, 2), (1, 2, 0, 1)),
                                             (16, 48, (1, 2), (0, 0, 0, 0))])
def test_conv_f64_integer_kat_exact(c, f, stride, pads):
    x = ref.np_init((2, 13, 11, c), "float64")
    w = ref.np_init((3, 3, c, f), "float64")
    out = run_conv64(x, w, stride=stride, pads=pads, pad_value=0.5)
    xp = ref.pad(x, [(0, 0), (pads[0], pads[1]), (pads[2], pads[3]), (0, 0)], 0.5)
    np.testing.assert_array_equal(out, ref.conv2d(xp, w, stride))


@pytest.mark.parametrize("tile", F64_CONV_TILES)
def test_conv_f64_integer_kat_exact_every_tile(tile):
    # 2 x 9 x 7 outputs (126 pixels: partial row tiles), 24 filters (partial
    # column tiles), K = 3*3*32 over several slabs with the taps inside them
    x = ref.np_init((2, 11, 9, 32), "float64")
    w = ref.np_init((3, 3, 32, 24), "float64")
    np.testing.assert_array_equal(run_conv64(x, w, tile=tile), ref.conv2d(x, w))


def test_conv_f64_c4_shape_seeded_pad_relu():
    # the C4 shape in float64: pad 1 folded into the loader, relu fused
    rng = np.random.default_rng(0)
    x = rng.uniform(0, 1, (8, 56, 56, 64))
    w = rng.normal(0, np.sqrt(2 / 576), (3, 3, 64, 64))
    out = run_conv64(x, w, pads=(1, 1, 1, 1), relu=True)
    want = ref.relu(ref.conv2d(ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)]), w))
    assert ref.scaled_error(out, want, 576, 1.0, float(np.abs(w).max())) <= TOL_F64


def test_conv_f64_odd_channels_staged_and_odd_filters_scalar():
    x = ref.np_init((1, 9, 9, 3), "float64")
    w = ref.np_init((3, 3, 3, 8), "float64")
    np.testing.assert_array_equal(run_conv64(x, w, pads=(1, 1, 1, 1)),
                                  ref.conv2d(ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)]), w))
    w5 = ref.np_init((3, 3, 3, 5), "float64")  # F odd: the scalar fp64 conv
    np.testing.assert_array_equal(run_conv64(x, w5), ref.conv2d(x, w5))


def test_conv_f64_split_k_and_bias():
    x = _uniform(7, (2, 14, 14, 32))
    w = _uniform(8, (3, 3, 32, 16))
    bias = _uniform(9, (16,))
    out = run_conv64(x, w, tile=(64, 64, 16, 2, 2), split_k=3, bias=bias)
    assert ref.scaled_error(out, ref.conv2d(x, w) + bias, 288, 1.0, 1.0) <= TOL_F64


# ------------------------------------------------------------------ relu, pad


def test_relu_and_pad_f64_entry_points():
    L = capi.lib()
    x = _uniform(10, (1001,))
    x[3] = np.nan
    X, Y = _dev(x), DeviceBuffer(x.size * 8)
    capi.check(L.xtc_hip_relu_f64(X.c_ptr, Y.c_ptr, x.size, 0.25, None), "relu f64")
    capi.check(L.xtc_hip_synchronize(), "sync")
    np.testing.assert_array_equal(Y.to_numpy(x.shape, np.float64), ref.relu(x, 0.25))
    t = _uniform(11, (3, 5, 7))
    pads = [(1, 0), (0, 2), (3, 1)]
    T = _dev(t)
    out_shape = tuple(d + p0 + p1 for d, (p0, p1) in zip(t.shape, pads))
    P = DeviceBuffer(int(np.prod(out_shape)) * 8)
    arr = lambda v: (ctypes.c_int64 * 3)(*v)  # noqa: E731
    capi.check(L.xtc_hip_pad_f64(T.c_ptr, P.c_ptr, 3, arr(t.shape), arr([p[0] for p in pads]),
                                 arr([p[1] for p in pads]), 0.1, None), "pad f64")
    capi.check(L.xtc_hip_synchronize(), "sync")
    np.testing.assert_array_equal(P.to_numpy(out_shape, np.float64), ref.pad(t, pads, 0.1))


def test_fp64_mfma_peak_probe():
    from xtc_amd.runtimes.hip.device import HipDevice

    dev = HipDevice(0)
    peak = dev.evaluate_flops("float64")  # FMA/s
    assert 0.3 * dev.datasheet_flops("float64") < peak <= 1.05 * dev.datasheet_flops("float64")


# ------------------------------------------------------------------ XTC pipeline


def _evaluate(graph, inputs, **kw):
    from xtc_amd.backends.hip import Backend
    from xtc_amd.runtimes.hip.device import HipDevice
    from xtc_amd.runtimes.hip.ndarray import DeviceArray

    backend = Backend(graph)
    module = backend.get_compiler(**kw).compile(backend.get_scheduler().schedule())
    dev = HipDevice(0)
    dev.load_module(module)
    fn = dev.get_module_function(module, module.payload_name)
    fn.restype = None
    status = dev.module_symbol(module, f"{module.payload_name}_status")
    status.restype = ctypes.c_int
    d_in = [DeviceArray.from_numpy(a, "float64", dev) for a in inputs]
    d_out = [DeviceArray(t.constant_shape, t.constant_dtype, dev) for t in graph.outputs_types]
    fn(*[ctypes.c_void_p(d.data) for d in (*d_in, *d_out)])
    assert status() == 0
    return [d.numpy() for d in d_out], module


def test_pipeline_f64_conv_graph_full_size():
    """C4's graph pad2d -> conv2d -> relu in float64 at its full size, through
    Backend -> Scheduler -> Compiler -> payload: one fused launch."""
    import xtc_amd.graphs.xtc.op as O

    rng = np.random.default_rng(0)
    x = rng.uniform(0, 1, (8, 56, 56, 64))
    w = rng.normal(0, np.sqrt(2 / 576), (3, 3, 64, 64))
    xi = O.tensor(x.shape, "float64", name="I")
    wi = O.tensor(w.shape, "float64", name="W")
    with O.graph(name="conv64") as gb:
        O.relu(O.conv2d(O.pad2d(xi, padding=1, axes=(1, 2), name="pad"), wi, name="conv"), name="relu")
    (out,), module = _evaluate(gb.graph, [x, w])
    assert len(module.plan.launches) == 1
    want = ref.relu(ref.conv2d(ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)]), w))
    assert ref.scaled_error(out, want, 576, 1.0, float(np.abs(w).max())) <= TOL_F64


def test_pipeline_f64_mlp_full_size_and_validate():
    """C5's MLP in float64 at its full size (relu fused into fc1), then the
    reference's own check: the evaluator's validate=True on np_init inputs."""
    import xtc_amd.graphs.xtc.op as O
    from xtc_amd.backends.hip import Backend

    rng = np.random.default_rng(0)
    xs = rng.uniform(-1, 1, (2048, 1024))
    w1 = rng.normal(0, 0.02, (1024, 4096))
    w2 = rng.normal(0, 0.02, (4096, 1024))
    X = O.tensor(xs.shape, "float64", name="X")
    W1 = O.tensor(w1.shape, "float64", name="W1")
    W2 = O.tensor(w2.shape, "float64", name="W2")
    with O.graph(name="mlp64") as gb:
        O.matmul(O.relu(O.matmul(X, W1, name="fc1"), name="act"), W2, name="fc2")
    (out,), _ = _evaluate(gb.graph, [xs, w1, w2])
    h = ref.relu(ref.matmul(xs, w1))
    assert ref.scaled_error(out, ref.matmul(h, w2), 4096, float(np.abs(h).max()), float(np.abs(w2).max())) <= TOL_F64
    backend = Backend(gb.graph)
    module = backend.get_compiler().compile(backend.get_scheduler().schedule())
    times, code, msg = module.get_evaluator(validate=True, repeat=1, min_repeat_ms=0).evaluate()
    assert code == 0, msg


def test_loop_explore_float64(tmp_path):
    """loop-explore --dtype float64: the reference's CLI offers float32 and
    float64 (src/xtc/cli/explore.py:154-160); every sampled fp64 schedule is
    compiled, validated and timed."""
    out = tmp_path / "e64.csv"
    cmd = [sys.executable, "-u", "-m", "xtc_amd.cli.explore", "--operator", "matmul", "--dims", "512", "512", "512",
           "--dtype", "float64", "--strategy", "tile_hip", "--search", "random", "--trials", "6", "--seed", "0",
           "--repeat", "2", "--min-repeat-ms", "10", "--validate", "--output", str(out)]
    print("[explore]", " ".join(cmd[3:]), flush=True)
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr[-3000:]
    rows = list(csv.DictReader(open(out)))
    assert len(rows) == 6 and all(float(r["time"]) > 0 and float(r["peak"]) > 0 for r in rows), proc.stderr[-2000:]
