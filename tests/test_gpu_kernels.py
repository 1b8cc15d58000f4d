# SPDX-License-Identifier: BSD-3-Clause
"""Parity of the HIP kernels (through the libxtc_hip C-ABI) against the oracle.

Bars: bit-exact on integer known-answer inputs; otherwise
max|out-ref| / (sqrt(K) max|A| max|B|) <= 1e-4 (fp32) or 1e-2 (bf16 inputs),
with the oracle fed the same (bf16-rounded) values in float64.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from oracle import reference as ref
from xtc_amd.runtimes.hip import capi
from xtc_amd.runtimes.hip.buffer import DeviceBuffer, ensure_device
from xtc_amd.utils.bf16 import f32_to_bf16_bits

pytestmark = pytest.mark.gpu

# XTC_HIP_GENERIC_GEMM=1 sends every tile to the generic template: the tests
# of the specialised kernels' own properties (their pipeline depths) do not
# apply then, every numerical check still does
GENERIC_ONLY = os.environ.get("XTC_HIP_GENERIC_GEMM") == "1"
needs_specialised = pytest.mark.skipif(GENERIC_ONLY, reason="XTC_HIP_GENERIC_GEMM=1 disables the specialised kernels")

TOL_F32 = 1e-4
TOL_BF16 = 1e-2


@pytest.fixture(scope="module", autouse=True)
def device():
    ensure_device(0)
    yield


def _dev(a: np.ndarray, dtype: str) -> DeviceBuffer:
    if dtype == "bfloat16":
        return DeviceBuffer.from_numpy(f32_to_bf16_bits(a))
    return DeviceBuffer.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def run_matmul(a, b, dtype="float32", tile=None, split_k=0, relu=False, thr=0.0, bias=None):
    M, K = a.shape
    N = b.shape[1]
    A, B = _dev(a, dtype), _dev(b, dtype)
    C = DeviceBuffer(M * N * 4)
    bias_buf = DeviceBuffer.from_numpy(bias.astype(np.float32)) if bias is not None else None
    d = capi.MatmulDesc()
    d.dtype = capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16
    d.M, d.N, d.K = M, N, K
    if tile is not None:
        d.tile = capi.Tile(*tile)
    d.split_k = split_k
    d.xcd_remap = 1
    d.relu = int(relu)
    d.relu_threshold = thr
    L = capi.lib()
    capi.check(
        L.xtc_hip_matmul(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, bias_buf.c_ptr if bias_buf else None),
        "matmul",
    )
    capi.check(L.xtc_hip_synchronize(), "sync")
    return C.to_numpy((M, N), np.float32)


def run_conv(x, w, dtype="float32", stride=(1, 1), pads=(0, 0, 0, 0), pad_value=0.0, tile=None, relu=False, split_k=0,
             bias=None):
    n, h, wd, c = x.shape
    r, s, _, f = w.shape
    I, W = _dev(x, dtype), _dev(w, dtype)
    hp, wp = h + pads[0] + pads[1], wd + pads[2] + pads[3]
    oh, ow = (hp - r) // stride[0] + 1, (wp - s) // stride[1] + 1
    O = DeviceBuffer(n * oh * ow * f * 4)
    d = capi.Conv2dDesc()
    d.dtype = capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16
    d.N, d.H, d.W, d.C, d.F, d.R, d.S = n, h, wd, c, f, r, s
    d.stride_h, d.stride_w = stride
    d.pad_top, d.pad_bottom, d.pad_left, d.pad_right = pads
    d.pad_value = pad_value
    if tile is not None:
        d.tile = capi.Tile(*tile)
    d.split_k = split_k
    d.xcd_remap = 1
    d.relu = int(relu)
    L = capi.lib()
    bias_buf = DeviceBuffer.from_numpy(bias.astype(np.float32)) if bias is not None else None
    capi.check(L.xtc_hip_conv2d(ctypes.byref(d), I.c_ptr, W.c_ptr, O.c_ptr, bias_buf.c_ptr if bias_buf else None),
               "conv2d")
    capi.check(L.xtc_hip_synchronize(), "sync")
    return O.to_numpy((n, oh, ow, f), np.float32)


def rng_uniform(seed, shape, low=-1.0, high=1.0):
    return np.random.default_rng(seed).uniform(low, high, size=shape).astype(np.float32)


# ------------------------------------------------------------------ matmul


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("shape", [(64, 64, 64), (512, 512, 512), (256, 128, 1024)])
def test_matmul_integer_kat_exact(dtype, shape):
    M, N, K = shape
    a = ref.np_init((M, K), "float32")
    b = ref.np_init((K, N), "float32")
    out = run_matmul(a, b, dtype)
    np.testing.assert_array_equal(out, ref.matmul(a, b).astype(np.float32))


def test_matmul_c1_seeded_fp32():
    a, b = ref.config_inputs("C1")
    out = run_matmul(a, b)
    err = ref.scaled_error(out, ref.matmul(a, b), 512, 1.0, 1.0)
    assert err <= TOL_F32, err


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize(
    "shape",
    [(21, 32, 16), (100, 72, 40), (1, 8, 8), (257, 136, 64), (33, 264, 520), (5, 4, 3), (7, 6, 5), (9, 17, 1),
     (4, 1, 7)],
)
def test_matmul_ragged(dtype, shape):
    M, N, K = shape
    a = rng_uniform(1, (M, K))
    b = rng_uniform(2, (K, N))
    if dtype == "bfloat16":
        a, b = ref.round_bf16(a), ref.round_bf16(b)
    out = run_matmul(a, b, dtype)
    err = ref.scaled_error(out, ref.matmul(a, b), K, np.abs(a).max(), np.abs(b).max())
    assert err <= (TOL_F32 if dtype == "float32" else TOL_BF16), err


def _instances(conv: bool):
    # the fp64 instances have their own every-tile tests (test_gpu_f64.py)
    return [i for i in capi.gemm_instances() if i["conv"] == conv and i["dtype"] in ("float32", "bfloat16")]


def test_every_matmul_instance():
    """Each compiled tile on a shape with partial tiles in M and N and K."""
    failures = []
    for inst in _instances(False):
        bm, bn, bk, wgm, wgn = inst["tile"]
        dtype = inst["dtype"]
        vec = 4 if dtype == "float32" else 8
        M, N, K = 2 * bm + 3, 2 * bn + vec, 3 * bk + vec
        a = ref.np_init((M, K), "float32")
        b = (ref.np_init((K, N), "float32")[::-1]).copy()
        out = run_matmul(a, b, dtype, tile=inst["tile"])
        expect = ref.matmul(a, b).astype(np.float32)
        if not np.array_equal(out, expect):
            failures.append((dtype, inst["tile"], float(np.abs(out - expect).max())))
    assert not failures, failures[:10]


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_matmul_split_k_bias_relu(dtype):
    M, N, K = 96, 160, 2048
    a = rng_uniform(3, (M, K))
    b = rng_uniform(4, (K, N))
    bias = rng_uniform(5, (N,))
    if dtype == "bfloat16":
        a, b = ref.round_bf16(a), ref.round_bf16(b)
    out = run_matmul(a, b, dtype, split_k=8, relu=True, bias=bias)
    expect = ref.relu(ref.matmul(a, b) + bias)
    err = ref.scaled_error(out, expect, K, np.abs(a).max(), np.abs(b).max())
    assert err <= (TOL_F32 if dtype == "float32" else TOL_BF16), err
    # relu applied after the full reduction
    assert (out >= 0).all()


def _int_operands(M, N, K, seed):
    a = ((np.arange(M)[:, None] * (3 + seed) + np.arange(K)[None, :] * 5) % 7 - 3).astype(np.float32)
    b = ((np.arange(K)[:, None] * 11 + np.arange(N)[None, :] * (2 + seed)) % 9 - 4).astype(np.float32)
    return a, b


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_split_k_in_kernel_reduction_back_to_back(dtype):
    # The last workgroup of each output tile sums the partials and resets the
    # tile's arrival counter.  Back-to-back calls with other data, other tile
    # counts and other split counts only come out exact if every call leaves
    # the counters at zero; the ragged shapes (N % 4 != 0, partial tiles) take
    # the scalar finishing path, the aligned ones the float4 path.
    cases = [(70, 130, 1536, 3, 0), (64, 128, 4096, 4, 1), (70, 130, 1536, 3, 2), (33, 257, 2048, 8, 3),
             (64, 128, 4096, 2, 4)]
    for M, N, K, split, seed in cases:
        a, b = _int_operands(M, N, K, seed)
        bias = (np.arange(N) % 5 - 2).astype(np.float32)
        out = run_matmul(a, b, dtype, split_k=split, relu=True, thr=1.0, bias=bias)
        expect = ref.relu(ref.matmul(a, b) + bias, 1.0).astype(np.float32)
        np.testing.assert_array_equal(out, expect, err_msg=f"{dtype} {(M, N, K)} split {split}")


def test_split_k_conv_in_kernel_reduction():
    x = ((np.arange(2 * 9 * 11 * 24).reshape(2, 9, 11, 24) * 7) % 5 - 2).astype(np.float32)
    w = ((np.arange(3 * 3 * 24 * 20).reshape(3, 3, 24, 20) * 3) % 7 - 3).astype(np.float32)
    expect = ref.conv2d(x, w).astype(np.float32)
    for _ in range(2):
        out = run_conv(x, w, split_k=3)
        np.testing.assert_array_equal(out, expect)


def test_split_k_on_concurrent_streams():
    # Split-K partials, arrival counters and transposed-operand staging are
    # kept per stream: split-K launches (generic, skinny bf16, with a
    # transposed B staged first) queued on three streams without a wait in
    # between must each come out exact.
    L = capi.lib()
    streams = [None, L.xtc_hip_stream_create(), L.xtc_hip_stream_create()]
    assert streams[1] and streams[2], capi.last_error()
    cases = [("float32", 256, 256, 8192, 8, 0), ("bfloat16", 16, 1024, 8192, 8, 0), ("float32", 128, 256, 4096, 4, 1)]
    try:
        jobs = []
        for rep in range(3):
            for si, s in enumerate(streams):
                dtype, M, N, K, split, tb = cases[(si + rep) % 3]
                a, b = _int_operands(M, N, K, 3 * rep + si)
                A = _dev(a, dtype)
                B = _dev(np.ascontiguousarray(b.T) if tb else b, dtype)
                C = DeviceBuffer(M * N * 4)
                d = capi.MatmulDesc()
                d.dtype = capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16
                d.M, d.N, d.K = M, N, K
                d.split_k = split
                d.xcd_remap = 1
                d.trans_b = tb
                d.stream = s
                capi.check(L.xtc_hip_matmul(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, None), "matmul")
                jobs.append((A, B, C, ref.matmul(a, b).astype(np.float32), f"rep {rep} stream {si} {dtype} {(M, N, K)}"))
        for s in streams:
            capi.check(L.xtc_hip_stream_synchronize(s), "stream sync")
        for _, _, C, expect, what in jobs:
            np.testing.assert_array_equal(C.to_numpy(expect.shape, np.float32), expect, err_msg=what)
    finally:
        for s in streams[1:]:
            capi.check(L.xtc_hip_stream_destroy(s), "stream destroy")


def test_matmul_relu_threshold_nan():
    a = np.ones((16, 8), np.float32)
    b = np.ones((8, 16), np.float32)
    a[0, 0] = np.nan
    out = run_matmul(a, b, relu=True, thr=9.0)
    assert np.isnan(out[0]).all()
    np.testing.assert_array_equal(out[1:], np.full((15, 16), 9.0, np.float32))


def test_matmul_c3b_skinny_bf16():
    a, b = ref.config_inputs("C3b")
    out = run_matmul(a, b, "bfloat16")
    err = ref.scaled_error(out, ref.matmul(a, b), 8192, np.abs(a).max(), np.abs(b).max())
    assert err <= TOL_BF16, err


# ------------------------------------------------------------------ conv2d


def test_conv_c4_pad_relu_fp32():
    x, w = ref.config_inputs("C4")
    out = run_conv(x, w, pads=(1, 1, 1, 1), relu=True)
    xp = ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)])
    expect = ref.relu(ref.conv2d(xp, w))
    err = ref.scaled_error(out, expect, 576, np.abs(xp).max(), np.abs(w).max())
    assert err <= TOL_F32, err


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_conv_stride_asym_pad_value(dtype):
    x = rng_uniform(6, (2, 9, 11, 16))
    w = rng_uniform(7, (3, 2, 16, 24))
    if dtype == "bfloat16":
        x, w = ref.round_bf16(x), ref.round_bf16(w)
    pads = (2, 1, 0, 3)
    out = run_conv(x, w, dtype, stride=(2, 3), pads=pads, pad_value=0.5)
    xp = ref.pad(x, [(0, 0), (2, 1), (0, 3), (0, 0)], 0.5)
    expect = ref.conv2d(xp, w, (2, 3))
    err = ref.scaled_error(out, expect, 3 * 2 * 16, 1.0, np.abs(w).max())
    assert err <= (TOL_F32 if dtype == "float32" else TOL_BF16), err


def test_every_conv_instance():
    # tiles that exist only in the direct conv kernel (C and F multiples of
    # 64) have no kernel for this shape; test_direct_conv_wide_* cover them
    failures = []
    for inst in _instances(True):
        dtype = inst["dtype"]
        probe = capi.Conv2dDesc(dtype=capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16, N=2, H=10, W=12,
                                C=16, F=32, R=3, S=3, stride_h=1, stride_w=1, pad_top=1, pad_bottom=1, pad_left=1,
                                pad_right=1, tile=capi.Tile(*inst["tile"]))
        try:
            capi.conv2d_pipeline_depths(probe)
        except capi.HipError:
            assert inst["tile"] in WIDE_DIRECT_TILES, inst
            continue
        x = ref.np_init((2, 10, 12, 16), "float32")
        w = (ref.np_init((3, 3, 16, 32), "float32")[::-1]).copy()
        out = run_conv(x, w, dtype, pads=(1, 1, 1, 1), tile=inst["tile"])
        xp = ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)])
        expect = ref.conv2d(xp, w).astype(np.float32)
        if not np.array_equal(out, expect):
            failures.append((dtype, inst["tile"], float(np.abs(out - expect).max())))
    assert not failures, failures[:10]


def test_conv_unaligned_channels_fallback():
    x = rng_uniform(8, (1, 7, 7, 3))
    w = rng_uniform(9, (3, 3, 3, 5))
    out = run_conv(x, w, pads=(1, 1, 1, 1))
    expect = ref.conv2d(ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)]), w)
    assert ref.scaled_error(out, expect, 27, 1.0, 1.0) <= TOL_F32


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_conv_unaligned_channels_staged(dtype):
    """C = 3 with F a multiple of the vector: the input and the weights are
    staged with zero channels up to 4 (fp32) or 8 (bf16) and the MFMA conv
    runs on the copies; a finite pad value times a zero weight adds 0."""
    x = rng_uniform(21, (2, 23, 19, 3))
    w = rng_uniform(22, (5, 3, 3, 16))
    if dtype == "bfloat16":
        x, w = ref.round_bf16(x), ref.round_bf16(w)
    pads = (2, 1, 1, 2)
    out = run_conv(x, w, dtype, stride=(2, 1), pads=pads, pad_value=0.5)
    xp = ref.pad(x, [(0, 0), (2, 1), (1, 2), (0, 0)], 0.5)
    expect = ref.conv2d(xp, w, (2, 1))
    err = ref.scaled_error(out, expect, 5 * 3 * 3, 1.0, np.abs(w).max())
    assert err <= (TOL_F32 if dtype == "float32" else TOL_BF16), err
    # integer inputs: exact, also with an explicit tile and split-K
    xi = ref.np_init((1, 17, 17, 3), "float32")
    wi = (ref.np_init((7, 7, 3, 32), "float32") - 5.0).copy()
    expect = ref.conv2d(ref.pad(xi, [(0, 0), (3, 3), (3, 3), (0, 0)]), wi, (2, 2)).astype(np.float32)
    tile = (64, 64, 16, 2, 2) if dtype == "float32" else (64, 64, 32, 2, 2)
    for tile, split in ((None, 0), (tile, 2)):
        out = run_conv(xi, wi, dtype, stride=(2, 2), pads=(3, 3, 3, 3), tile=tile, split_k=split)
        np.testing.assert_array_equal(out, expect)


# ------------------------------------------------------------- aux kernels


def test_relu_kernel():
    x = rng_uniform(10, (1000003,))
    x[5] = np.nan
    X = DeviceBuffer.from_numpy(x)
    Y = DeviceBuffer(x.nbytes)
    L = capi.lib()
    capi.check(L.xtc_hip_relu(X.c_ptr, Y.c_ptr, x.size, ctypes.c_float(0.25), None))
    capi.check(L.xtc_hip_synchronize())
    y = Y.to_numpy(x.shape, np.float32)
    np.testing.assert_array_equal(y, ref.relu(x, 0.25))


def test_pad_kernel():
    x = rng_uniform(11, (3, 5, 7, 4))
    X = DeviceBuffer.from_numpy(x)
    pads = [(0, 0), (1, 2), (3, 0), (0, 1)]
    shape = (ctypes.c_int64 * 4)(*x.shape)
    before = (ctypes.c_int64 * 4)(*[p[0] for p in pads])
    after = (ctypes.c_int64 * 4)(*[p[1] for p in pads])
    expect = ref.pad(x, pads, -2.0)
    Y = DeviceBuffer(expect.nbytes)
    L = capi.lib()
    capi.check(L.xtc_hip_pad(X.c_ptr, Y.c_ptr, 4, shape, before, after, ctypes.c_float(-2.0), None))
    capi.check(L.xtc_hip_synchronize())
    np.testing.assert_array_equal(Y.to_numpy(expect.shape, np.float32), expect)


@pytest.mark.parametrize("shape,pads", [
    ((2, 9, 11, 64), [(0, 0), (1, 1), (2, 0), (0, 0)]),   # 16-byte row copies (innermost dim unpadded)
    ((4, 8), [(3, 2), (0, 0)]),
    ((12,), [(0, 0)]),                                      # rank 1, no padding: a copy
    ((2, 9, 11, 6), [(0, 0), (1, 1), (1, 1), (0, 0)]),    # rows of 6 floats: element path
])
def test_pad_kernel_paths(shape, pads):
    x = rng_uniform(13, shape)
    nd = len(shape)
    X = DeviceBuffer.from_numpy(x)
    expect = ref.pad(x, pads, 0.5)
    Y = DeviceBuffer(expect.nbytes)
    L = capi.lib()
    capi.check(L.xtc_hip_pad(X.c_ptr, Y.c_ptr, nd, (ctypes.c_int64 * nd)(*shape),
                             (ctypes.c_int64 * nd)(*[p[0] for p in pads]), (ctypes.c_int64 * nd)(*[p[1] for p in pads]),
                             ctypes.c_float(0.5), None))
    capi.check(L.xtc_hip_synchronize())
    np.testing.assert_array_equal(Y.to_numpy(expect.shape, np.float32), expect)


_UNPAD_DT = {2: np.uint16, 4: np.float32, 8: np.float64}


@pytest.mark.parametrize("shape,pads,elem", [
    ((2, 9, 11, 64), [(0, 0), (1, 1), (2, 0), (0, 0)], 4),   # 16-byte row copies (innermost dim kept)
    ((4, 8), [(3, 0), (1, 2)], 4),                           # element path
    ((5, 6, 8), [(1, 1), (2, 1), (0, 0)], 2),                # bf16 words, rows of 16 bytes
    ((3, 7, 5), [(0, 1), (1, 1), (1, 2)], 2),                # bf16 words, element path
    ((6, 10), [(1, 2), (3, 3)], 8),                          # fp64, element path
    ((4, 5, 6), [(1, 1), (0, 2), (0, 0)], 8),                # fp64, rows of 48 bytes
    ((12,), [(0, 0)], 4),                                    # rank 1, nothing cropped: a copy
    ((4, 3), [(2, 2), (0, 0)], 4),                           # empty output: nothing launched
])
def test_unpad_kernel_paths(shape, pads, elem):
    """xtc_hip_unpad against the oracle's crop (XTCOperUnpad.forward), the
    elements moved as raw words of their size: bit-exact."""
    rng = np.random.default_rng(17)
    dt = _UNPAD_DT[elem]
    x = rng.integers(0, 2**15, shape).astype(dt) if elem == 2 else rng.uniform(-1, 1, shape).astype(dt)
    expect = ref.unpad(x, pads)
    X = DeviceBuffer.from_numpy(x)
    Y = DeviceBuffer(max(expect.nbytes, 16))
    nd = len(shape)
    L = capi.lib()
    capi.check(L.xtc_hip_unpad(X.c_ptr, Y.c_ptr, elem, nd, (ctypes.c_int64 * nd)(*shape),
                               (ctypes.c_int64 * nd)(*[p[0] for p in pads]),
                               (ctypes.c_int64 * nd)(*[p[1] for p in pads]), None))
    capi.check(L.xtc_hip_synchronize())
    if expect.size:
        np.testing.assert_array_equal(Y.to_numpy(expect.shape, dt), expect)


def test_unpad_rejects_bad_crops():
    x = DeviceBuffer(4 * 24)
    y = DeviceBuffer(4 * 24)
    L = capi.lib()
    shape = (ctypes.c_int64 * 2)(4, 6)
    zero = (ctypes.c_int64 * 2)(0, 0)
    with pytest.raises(capi.HipError, match="exceeds dim 1"):
        capi.check(L.xtc_hip_unpad(x.c_ptr, y.c_ptr, 4, 2, shape, (ctypes.c_int64 * 2)(0, 4), (ctypes.c_int64 * 2)(0, 3),
                                   None))
    with pytest.raises(capi.HipError, match="element size 3"):
        capi.check(L.xtc_hip_unpad(x.c_ptr, y.c_ptr, 3, 2, shape, zero, zero, None))
    with pytest.raises(capi.HipError, match="negative"):
        capi.check(L.xtc_hip_unpad(x.c_ptr, y.c_ptr, 4, 2, shape, (ctypes.c_int64 * 2)(-1, 0), zero, None))


@pytest.mark.parametrize("offset", [0, 2])
def test_cast_bf16_vector_and_unaligned(offset):
    # offset 0: 16-byte aligned, 8 elements per thread step plus a tail of 5;
    # offset 2 elements: unaligned pointers, one element at a time
    n = 8 * 1000 + 5
    x = rng_uniform(14, (n + offset,), -3, 3)
    x[offset:offset + 4] = [np.nan, np.inf, -0.0, 1e-40]
    X = DeviceBuffer.from_numpy(x)
    H = DeviceBuffer((n + offset) * 2)
    Y = DeviceBuffer((n + offset) * 4)
    L = capi.lib()
    capi.check(L.xtc_hip_cast_f32_to_bf16(ctypes.c_void_p(X.ptr + 4 * offset), ctypes.c_void_p(H.ptr + 2 * offset), n,
                                          None))
    capi.check(L.xtc_hip_cast_bf16_to_f32(ctypes.c_void_p(H.ptr + 2 * offset), ctypes.c_void_p(Y.ptr + 4 * offset), n,
                                          None))
    capi.check(L.xtc_hip_synchronize())
    bits = H.to_numpy((n + offset,), np.uint16)[offset:]
    want = f32_to_bf16_bits(x[offset:])
    nan = np.isnan(x[offset:])
    np.testing.assert_array_equal(bits[~nan], want[~nan])
    assert np.all((bits[nan] & 0x7F80) == 0x7F80) and np.all(bits[nan] & 0x7F)
    back = Y.to_numpy((n + offset,), np.float32)[offset:]
    np.testing.assert_array_equal(back[~nan], ref.round_bf16(x[offset:])[~nan])


def test_cast_bf16_roundtrip():
    x = rng_uniform(12, (4099,), -100, 100)
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    X = DeviceBuffer.from_numpy(x)
    H = DeviceBuffer(x.size * 2)
    Y = DeviceBuffer(x.nbytes)
    L = capi.lib()
    capi.check(L.xtc_hip_cast_f32_to_bf16(X.c_ptr, H.c_ptr, x.size, None))
    capi.check(L.xtc_hip_cast_bf16_to_f32(H.c_ptr, Y.c_ptr, x.size, None))
    capi.check(L.xtc_hip_synchronize())
    np.testing.assert_array_equal(H.to_numpy(x.shape, np.uint16), f32_to_bf16_bits(x))
    np.testing.assert_array_equal(Y.to_numpy(x.shape, np.float32), ref.round_bf16(x))


def test_memset_zero():
    B = DeviceBuffer.from_numpy(np.ones(1031, np.uint8))
    B.zero()
    assert not B.to_numpy((1031,), np.uint8).any()


# ------------------------------------------- LDS-DMA bf16 kernel (256x256x64)


def _run_strided(a, b, tile, lda, ldb, ldc, relu=False, bias=None, split_k=1):
    """bf16 matmul with padded leading dimensions (elements)."""
    M, K = a.shape
    N = b.shape[1]
    ap = np.zeros((M, lda), np.float32)
    ap[:, :K] = a
    bp = np.zeros((K, ldb), np.float32)
    bp[:, :N] = b
    A, B = _dev(ap, "bfloat16"), _dev(bp, "bfloat16")
    C = DeviceBuffer(M * ldc * 4)
    C.zero()
    bias_buf = DeviceBuffer.from_numpy(bias.astype(np.float32)) if bias is not None else None
    d = capi.MatmulDesc()
    d.dtype = capi.XTC_HIP_BF16
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = lda, ldb, ldc
    d.tile = capi.Tile(*tile)
    d.split_k = split_k
    d.xcd_remap = 1
    d.relu = int(relu)
    L = capi.lib()
    capi.check(L.xtc_hip_matmul(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, bias_buf.c_ptr if bias_buf else None))
    capi.check(L.xtc_hip_synchronize())
    return C.to_numpy((M, ldc), np.float32)[:, :N]


def run_matmul_layout(a, b, dtype, ta, tb, tile=None, split_k=0, pad_a=0, pad_b=0, relu=False, bias=None):
    """C = a @ b with A stored transposed (At[K][M + pad_a]) when ta and B
    stored transposed (Bt[N][K + pad_b]) when tb, else row-major with the
    same padding of the leading dimension."""
    M, K = a.shape
    N = b.shape[1]
    sa = a.T if ta else a
    sb = b.T if tb else b
    ap = np.zeros((sa.shape[0], sa.shape[1] + pad_a), np.float32)
    ap[:, : sa.shape[1]] = sa
    bp = np.zeros((sb.shape[0], sb.shape[1] + pad_b), np.float32)
    bp[:, : sb.shape[1]] = sb
    A, B = _dev(ap, dtype), _dev(bp, dtype)
    C = DeviceBuffer(M * N * 4)
    bias_buf = DeviceBuffer.from_numpy(bias.astype(np.float32)) if bias is not None else None
    d = capi.MatmulDesc()
    d.dtype = capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb = ap.shape[1], bp.shape[1]
    d.trans_a, d.trans_b = int(ta), int(tb)
    if tile is not None:
        d.tile = capi.Tile(*tile)
    d.split_k = split_k
    d.xcd_remap = 1
    d.relu = int(relu)
    L = capi.lib()
    capi.check(L.xtc_hip_matmul(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, bias_buf.c_ptr if bias_buf else None),
               "matmul")
    capi.check(L.xtc_hip_synchronize(), "sync")
    return C.to_numpy((M, N), np.float32)


LAYOUTS = [(True, False), (False, True), (True, True)]


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_matmul_operand_layouts_integer_exact(dtype, ta, tb):
    # transposed storage (tensor layout [1, 0]) on every kernel family: the
    # generic template (ragged and aligned shapes, split-K), the skinny bf16
    # kernel and the LDS-DMA kernel (B^T read natively, A^T via a transposed
    # copy); padded leading dimensions on the stored matrices
    # transposed copies: 16-byte vectors when the stored dims are multiples
    # of the vector (ragged against the 64/128-element tile: 96, 136, 264),
    # element by element otherwise (70, 130, ld 100 for bf16)
    cases = [((64, 96, 128), None, 0, 0, 0), ((70, 130, 200), None, 0, 8, 4), ((96, 160, 2048), None, 4, 0, 0),
             ((136, 96, 264), None, 0, 0, 0)]
    if dtype == "bfloat16":
        cases += [((256, 512, 256), (256, 256, 64, 2, 4), 0, 0, 0), ((512, 256, 320), (256, 256, 64, 4, 2), 0, 16, 8),
                  ((16, 1024, 8192), (16, 128, 64, 1, 4), 8, 0, 0)]
    for (M, N, K), tile, split, pad_a, pad_b in cases:
        a, b = _int_operands(M, N, K, 5)
        out = run_matmul_layout(a, b, dtype, ta, tb, tile=tile, split_k=split, pad_a=pad_a, pad_b=pad_b)
        np.testing.assert_array_equal(out, ref.matmul(a, b).astype(np.float32),
                                      err_msg=f"{dtype} ta={ta} tb={tb} {(M, N, K)} tile={tile}")


@pytest.mark.parametrize("waves", [(2, 4), (4, 2)])
def test_lds_dma_bf16_transposed_b_seeded_bias_relu(waves):
    # B^T feeds the LDS-DMA kernel directly; seeded inputs, padded strides
    rng = np.random.default_rng(41)
    M, N, K = 512, 768, 1024
    a = ref.round_bf16(rng.uniform(-1, 1, (M, K)).astype(np.float32))
    b = ref.round_bf16(rng.uniform(-1, 1, (K, N)).astype(np.float32))
    bias = rng.uniform(-1, 1, (N,)).astype(np.float32)
    out = run_matmul_layout(a, b, "bfloat16", False, True, tile=(256, 256, 64, *waves), pad_a=8, pad_b=64,
                            relu=True, bias=bias)
    expect = ref.relu(ref.matmul(a, b) + bias)
    assert ref.scaled_error(out, expect, K, 1.0, 1.0) <= TOL_BF16
    # and bit-identical to the row-major B path: same fragments, same order
    same = run_matmul_layout(a, b, "bfloat16", False, False, tile=(256, 256, 64, *waves), pad_a=8, pad_b=64,
                             relu=True, bias=bias)
    np.testing.assert_array_equal(out, same)


@pytest.mark.parametrize("waves", [(2, 4), (4, 2)])
def test_lds_dma_bf16_integer_exact(waves):
    M, N, K = 512, 768, 1024
    a = ref.np_init((M, K), "float32")
    b = (ref.np_init((K, N), "float32")[::-1]).copy()
    out = run_matmul(a, b, "bfloat16", tile=(256, 256, 64, *waves))
    np.testing.assert_array_equal(out, ref.matmul(a, b).astype(np.float32))


@pytest.mark.parametrize("waves", [(2, 4), (4, 2)])
def test_lds_dma_bf16_seeded_bias_relu_strided(waves):
    rng = np.random.default_rng(21)
    M, N, K = 256, 512, 320
    a = ref.round_bf16(rng.uniform(-1, 1, (M, K)).astype(np.float32))
    b = ref.round_bf16(rng.uniform(-1, 1, (K, N)).astype(np.float32))
    bias = rng.uniform(-1, 1, (N,)).astype(np.float32)
    out = _run_strided(a, b, (256, 256, 64, *waves), lda=K + 64, ldb=N + 256, ldc=N + 4, relu=True, bias=bias)
    expect = ref.relu(ref.matmul(a, b) + bias)
    assert ref.scaled_error(out, expect, K, 1.0, 1.0) <= TOL_BF16


def test_lds_dma_bf16_swizzle_covers_every_position():
    # A and B hold distinct small integers at every (row, k) / (k, col), so any
    # swizzle or transpose mistake changes the exact result
    M, N, K = 256, 256, 64
    a = ((np.arange(M)[:, None] * 3 + np.arange(K)[None, :] * 5) % 7 - 3).astype(np.float32)
    b = ((np.arange(K)[:, None] * 11 + np.arange(N)[None, :] * 2) % 9 - 4).astype(np.float32)
    for waves in ((2, 4), (4, 2)):
        out = run_matmul(a, b, "bfloat16", tile=(256, 256, 64, *waves))
        np.testing.assert_array_equal(out, ref.matmul(a, b).astype(np.float32))


# ------------------------------- ping-pong LDS-DMA bf16 kernel (256x256x32, 2x4)

PINGPONG = (256, 256, 32, 2, 4)


@pytest.mark.parametrize("K", [32, 64, 96, 128, 160, 1024, 1056])
def test_pingpong_bf16_integer_exact_every_pipeline_depth(K):
    # K / 32 slabs below, at and above the DMA lead (3) and the stage count
    # (4), and not a multiple of it; 2x3 tiles give six different K-stagger
    # offsets, which wrap when there are fewer slabs than the offset
    M, N = 512, 768
    a, b = _int_operands(M, N, K, 5)
    out = run_matmul(a, b, "bfloat16", tile=PINGPONG)
    np.testing.assert_array_equal(out, ref.matmul(a, b).astype(np.float32), err_msg=f"K={K}")


def test_pingpong_bf16_swizzle_covers_every_position():
    # distinct small integers at every (row, k) / (k, col) of one slab
    M, N, K = 256, 256, 32
    a = ((np.arange(M)[:, None] * 3 + np.arange(K)[None, :] * 5) % 7 - 3).astype(np.float32)
    b = ((np.arange(K)[:, None] * 11 + np.arange(N)[None, :] * 2) % 9 - 4).astype(np.float32)
    out = run_matmul(a, b, "bfloat16", tile=PINGPONG)
    np.testing.assert_array_equal(out, ref.matmul(a, b).astype(np.float32))
    out_t = run_matmul_layout(a, b, "bfloat16", False, True, tile=PINGPONG)
    np.testing.assert_array_equal(out_t, ref.matmul(a, b).astype(np.float32))


def test_pingpong_bf16_seeded_bias_relu_strided():
    rng = np.random.default_rng(23)
    M, N, K = 512, 512, 544
    a = ref.round_bf16(rng.uniform(-1, 1, (M, K)).astype(np.float32))
    b = ref.round_bf16(rng.uniform(-1, 1, (K, N)).astype(np.float32))
    bias = rng.uniform(-1, 1, (N,)).astype(np.float32)
    out = _run_strided(a, b, PINGPONG, lda=K + 64, ldb=N + 256, ldc=N + 4, relu=True, bias=bias)
    expect = ref.relu(ref.matmul(a, b) + bias)
    assert ref.scaled_error(out, expect, K, 1.0, 1.0) <= TOL_BF16


def test_pingpong_bf16_transposed_b_matches_row_major_and_bk64():
    # B^T read natively: same fragments in the same order as row-major B, so
    # bit-identical; and the same K walk as the 256x256x64 kernel
    rng = np.random.default_rng(43)
    M, N, K = 512, 768, 1024
    a = ref.round_bf16(rng.uniform(-1, 1, (M, K)).astype(np.float32))
    b = ref.round_bf16(rng.uniform(-1, 1, (K, N)).astype(np.float32))
    bias = rng.uniform(-1, 1, (N,)).astype(np.float32)
    out = run_matmul_layout(a, b, "bfloat16", False, True, tile=PINGPONG, pad_a=8, pad_b=64, relu=True, bias=bias)
    expect = ref.relu(ref.matmul(a, b) + bias)
    assert ref.scaled_error(out, expect, K, 1.0, 1.0) <= TOL_BF16
    same = run_matmul_layout(a, b, "bfloat16", False, False, tile=PINGPONG, pad_a=8, pad_b=64, relu=True, bias=bias)
    np.testing.assert_array_equal(out, same)


@needs_specialised
def test_pingpong_bf16_split_k_bias_relu_strided():
    # split-K runs on the ping-pong kernel itself (its pipeline depths 3-5,
    # not the generic template's) when K splits into equal whole slabs: the
    # last workgroup of each tile sums the partial planes with bias and relu
    M, N, K = 512, 768, 1536
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_BF16, M=M, N=N, K=K, tile=capi.Tile(*PINGPONG), split_k=3)
    assert sorted(capi.matmul_pipeline_depths(d)) == [3, 4, 5]
    a, b = _int_operands(M, N, K, 7)
    bias = np.arange(-(N // 2), N - N // 2, dtype=np.float32)
    for split in (2, 3, 6):
        out = _run_strided(a, b, PINGPONG, lda=K + 64, ldb=N + 256, ldc=N + 4, relu=True, bias=bias, split_k=split)
        np.testing.assert_array_equal(out, ref.relu(ref.matmul(a, b) + bias).astype(np.float32), err_msg=f"{split}")
    rng = np.random.default_rng(29)
    ar = ref.round_bf16(rng.uniform(-1, 1, (M, K)).astype(np.float32))
    br = ref.round_bf16(rng.uniform(-1, 1, (K, N)).astype(np.float32))
    out = _run_strided(ar, br, PINGPONG, lda=K, ldb=N, ldc=N, split_k=4)
    assert ref.scaled_error(out, ref.matmul(ar, br), K, 1.0, 1.0) <= TOL_BF16
    # two launches in a row reuse the arrival counters: the second must not
    # see the first's counts
    again = _run_strided(ar, br, PINGPONG, lda=K, ldb=N, ldc=N, split_k=4)
    np.testing.assert_array_equal(out, again)


# ------------- LDS-DMA fp32 kernel (BK 32: 128x256, 256x128, 128x128; BK 16: 128x256, 256x128)

F32_LDS = [(128, 256, 32, 2, 4), (256, 128, 32, 4, 2), (128, 128, 32, 2, 4), (128, 256, 16, 2, 4), (256, 128, 16, 4, 2)]


@pytest.mark.parametrize("tile", F32_LDS)
@pytest.mark.parametrize("K,split", [(16, 1), (32, 1), (64, 1), (80, 1), (96, 1), (1024, 1), (1056, 1), (512, 2),
                                     (1024, 4), (2048, 8)])
def test_f32_lds_integer_exact_every_pipeline_depth(tile, K, split):
    # K / BK / split slabs below, at and above the DMA lead (2 for BK 32, 3
    # or 4 for BK 16; K = 16 and 80 take the generic kernel at BK 32);
    # split-K finished in the kernel
    M, N = 512, 512
    a, b = _int_operands(M, N, K, 7)
    out = run_matmul(a, b, "float32", tile=tile, split_k=split)
    np.testing.assert_array_equal(out, ref.matmul(a, b).astype(np.float32), err_msg=f"{tile} K={K} split={split}")


@pytest.mark.parametrize("tile", F32_LDS)
def test_f32_lds_seeded_bias_relu_strided(tile):
    rng = np.random.default_rng(37)
    M, N, K = 512, 512, 640
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = rng.uniform(-1, 1, (N,)).astype(np.float32)
    for split in (1, 2):
        out = _run_strided_f32(a, b, tile, lda=K + 12, ldb=N + 8, ldc=N + 4, relu=True, bias=bias, split_k=split)
        expect = ref.relu(ref.matmul(a, b) + bias)
        assert ref.scaled_error(out, expect, K, 1.0, 1.0) <= TOL_F32, f"split {split}"


def _run_strided_f32(a, b, tile, lda, ldb, ldc, relu=False, bias=None, split_k=1):
    """fp32 matmul with padded leading dimensions (elements)."""
    M, K = a.shape
    N = b.shape[1]
    ap = np.zeros((M, lda), np.float32)
    ap[:, :K] = a
    bp = np.zeros((K, ldb), np.float32)
    bp[:, :N] = b
    A, B = _dev(ap, "float32"), _dev(bp, "float32")
    C = DeviceBuffer(M * ldc * 4)
    C.zero()
    bias_buf = DeviceBuffer.from_numpy(bias.astype(np.float32)) if bias is not None else None
    d = capi.MatmulDesc()
    d.dtype = capi.XTC_HIP_F32
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = lda, ldb, ldc
    d.tile = capi.Tile(*tile)
    d.split_k = split_k
    d.xcd_remap = 1
    d.relu = int(relu)
    L = capi.lib()
    capi.check(L.xtc_hip_matmul(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, bias_buf.c_ptr if bias_buf else None))
    capi.check(L.xtc_hip_synchronize())
    return C.to_numpy((M, ldc), np.float32)[:, :N]


# ------------------------------ split-wave fp32 kernel (32x32x16, 1x1, split-K in a workgroup)

SPLITWAVE = (32, 32, 16, 1, 1)


@pytest.mark.parametrize("shape,split", [((512, 512, 512), 4), ((64, 96, 192), 3), ((32, 32, 32), 2),
                                         ((96, 64, 1024), 4), ((128, 32, 96), 2), ((512, 512, 512), 8),
                                         ((64, 64, 1280), 5), ((32, 64, 96), 6), ((64, 32, 2688), 7)])
def test_splitwave_f32_integer_exact(shape, split):
    # K / split / 16 chunks per wave below, at and above the register ring
    # depth (4)
    M, N, K = shape
    a, b = _int_operands(M, N, K, 3)
    out = run_matmul(a, b, "float32", tile=SPLITWAVE, split_k=split)
    np.testing.assert_array_equal(out, ref.matmul(a, b).astype(np.float32), err_msg=f"{shape} split {split}")


def test_splitwave_f32_seeded_bias_relu_strided():
    rng = np.random.default_rng(29)
    M, N, K = 256, 192, 512
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = rng.uniform(-1, 1, (N,)).astype(np.float32)
    ap = np.zeros((M, K + 12), np.float32)
    ap[:, :K] = a
    bp = np.zeros((K, N + 5), np.float32)
    bp[:, :N] = b
    A, B = _dev(ap, "float32"), _dev(bp, "float32")
    ldc = N + 3
    C = DeviceBuffer(M * ldc * 4)
    C.zero()
    bias_buf = DeviceBuffer.from_numpy(bias)
    d = capi.MatmulDesc()
    d.dtype = capi.XTC_HIP_F32
    d.M, d.N, d.K = M, N, K
    d.lda, d.ldb, d.ldc = K + 12, N + 5, ldc
    d.tile = capi.Tile(*SPLITWAVE)
    d.split_k = 4
    d.xcd_remap = 1
    d.relu = 1
    L = capi.lib()
    capi.check(L.xtc_hip_matmul(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, bias_buf.c_ptr), "matmul")
    capi.check(L.xtc_hip_synchronize(), "sync")
    out = C.to_numpy((M, ldc), np.float32)[:, :N]
    expect = ref.relu(ref.matmul(a, b) + bias)
    assert ref.scaled_error(out, expect, K, 1.0, 1.0) <= TOL_F32


def test_splitwave_f32_bit_identical_to_grid_split_k():
    # 48 rows are not a whole number of 32-row tiles, so the same tile and
    # split run on the generic kernel (split-K over the grid); the 64-row
    # problem with the same first 48 rows runs on the split-wave kernel.
    # Each output element depends on its own row only: the shared rows must
    # match bit for bit on random inputs, bias and relu included.
    rng = np.random.default_rng(31)
    N, K = 96, 512
    a = rng.uniform(-1, 1, (64, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = rng.uniform(-1, 1, (N,)).astype(np.float32)
    for split in (2, 4, 8):
        grid = run_matmul(a[:48].copy(), b, "float32", tile=SPLITWAVE, split_k=split, relu=True, bias=bias)
        wave = run_matmul(a, b, "float32", tile=SPLITWAVE, split_k=split, relu=True, bias=bias)
        np.testing.assert_array_equal(wave[:48], grid, err_msg=f"split {split}")


# ------------------------------------------------- skinny bf16 (B-streaming kernel)

SKINNY = (16, 128, 64, 1, 4)


@pytest.mark.parametrize("M,N,K,split", [(16, 1024, 8192, 8), (16, 512, 8192, 16), (16, 384, 1024, 1), (5, 256, 2048, 4),
                                         (1, 128, 512, 1)])
def test_skinny_bf16_integer_exact(M, N, K, split):
    # distinct small integers at every (row, k) / (k, col): a wrong swizzle,
    # transpose, chunk offset or split order changes the exact result
    a = ((np.arange(M)[:, None] * 5 + np.arange(K)[None, :] * 3) % 7 - 3).astype(np.float32)
    b = ((np.arange(K)[:, None] * 7 + np.arange(N)[None, :] * 5) % 9 - 4).astype(np.float32)
    out = run_matmul(a, b, "bfloat16", tile=SKINNY, split_k=split)
    np.testing.assert_array_equal(out, ref.matmul(a, b).astype(np.float32))


@pytest.mark.parametrize("split", [1, 2])
def test_skinny_bf16_strided_bias_relu(split):
    rng = np.random.default_rng(31)
    M, N, K = 12, 256, 1024 * split
    a = ref.round_bf16(rng.uniform(-1, 1, (M, K)).astype(np.float32))
    b = ref.round_bf16(rng.uniform(-1, 1, (K, N)).astype(np.float32))
    bias = rng.uniform(-1, 1, (N,)).astype(np.float32)
    out = _run_strided(a, b, SKINNY, lda=K + 8, ldb=N + 128, ldc=N + 4, relu=True, bias=bias, split_k=split)
    expect = ref.relu(ref.matmul(a, b) + bias)
    assert ref.scaled_error(out, expect, K, 1.0, 1.0) <= TOL_BF16


def test_skinny_is_the_default_for_c3b():
    tile, split = capi.default_tile("bfloat16", False, 16, 8192, 8192)
    assert tuple(tile) == SKINNY and split == 8


# ------------------------------------------- direct conv (fp32, C and F multiples of 64)

DIRECT = (64, 64, 16, 2, 2)


def _int_tensor(shape, mul, mod):
    idx = np.indices(shape).reshape(len(shape), -1)
    v = (sum((i + 1) * mul[j] for j, i in enumerate(idx)) % mod) - mod // 2
    return v.reshape(shape).astype(np.float32)


@pytest.mark.parametrize(
    "n,h,w,c,f,r,s,pads,pad_value",
    [
        (2, 13, 11, 64, 128, 3, 3, (1, 1, 1, 1), 0.0),   # partial 8x8 blocks, two filter blocks
        (1, 9, 10, 128, 64, 3, 3, (2, 0, 1, 3), 1.0),    # two channel chunks, asymmetric pads, pad value
        (3, 8, 8, 64, 64, 1, 1, (0, 0, 0, 0), 0.0),      # 1x1
        (1, 6, 7, 64, 64, 4, 2, (1, 2, 0, 1), -2.0),     # 4x2 window
    ],
)
def test_direct_conv_integer_exact(n, h, w, c, f, r, s, pads, pad_value):
    x = _int_tensor((n, h, w, c), (3, 5, 7, 1), 7)
    wt = _int_tensor((r, s, c, f), (2, 3, 1, 5), 5)
    out = run_conv(x, wt, pads=pads, pad_value=pad_value, tile=DIRECT)
    xp = ref.pad(x, [(0, 0), pads[:2], pads[2:], (0, 0)], pad_value)
    np.testing.assert_array_equal(out, ref.conv2d(xp, wt).astype(np.float32))


def test_direct_conv_bias_relu_seeded():
    rng = np.random.default_rng(41)
    x = rng.uniform(0, 1, (2, 14, 14, 64)).astype(np.float32)
    wt = rng.normal(0, 0.06, (3, 3, 64, 64)).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, (64,)).astype(np.float32)
    out = run_conv(x, wt, pads=(1, 1, 1, 1), tile=DIRECT, relu=True, bias=bias)
    xp = ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)])
    expect = ref.relu(ref.conv2d(xp, wt) + bias)
    assert ref.scaled_error(out, expect, 576, 1.0, np.abs(wt).max()) <= TOL_F32


def test_direct_conv_is_the_default_for_c4_and_strided_falls_back():
    tile, split = capi.default_tile("float32", True, 8 * 56 * 56, 64, 576)
    assert tuple(tile) == DIRECT and split == 1
    # stride 2: the 8x8 block's halo exceeds the LDS buffer -> implicit-GEMM kernel, same tile
    x = _int_tensor((1, 20, 20, 64), (3, 5, 7, 1), 7)
    wt = _int_tensor((3, 3, 64, 64), (2, 3, 1, 5), 5)
    out = run_conv(x, wt, stride=(2, 2), pads=(1, 1, 1, 1), tile=DIRECT)
    xp = ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)])
    np.testing.assert_array_equal(out, ref.conv2d(xp, wt, (2, 2)).astype(np.float32))


# ------------------------------------------------------------------ pipeline depths

# (dtype, tile, split_k, (M, N, K), trans_b): every kernel with more than one
# compiled pipeline depth, at slab counts below, at and above the depths
DEPTH_CASES = [
    ("float32", (256, 128, 16, 4, 2), 1, (512, 256, 512), False),
    ("float32", (256, 128, 16, 4, 2), 1, (256, 128, 48), False),
    ("float32", (128, 256, 16, 2, 4), 1, (256, 512, 160), False),
    ("float32", (256, 128, 32, 4, 2), 1, (512, 256, 64), False),
    ("float32", (128, 256, 32, 2, 4), 1, (256, 512, 512), False),
    ("float32", (128, 128, 32, 2, 4), 2, (256, 256, 1024), False),
    ("float32", (128, 128, 32, 2, 4), 1, (128, 128, 32), False),
    ("bfloat16", (256, 256, 32, 2, 4), 1, (512, 512, 32), False),
    ("bfloat16", (256, 256, 32, 2, 4), 1, (512, 512, 160), False),
    ("bfloat16", (256, 256, 32, 2, 4), 1, (512, 512, 1056), False),
    ("bfloat16", (256, 256, 32, 2, 4), 1, (512, 256, 224), True),
    # ping-pong split-K: 16, 16 and 3 slabs per split (3 < the DMA lead)
    ("bfloat16", (256, 256, 32, 2, 4), 2, (512, 512, 1024), False),
    ("bfloat16", (256, 256, 32, 2, 4), 4, (256, 512, 2048), True),
    ("bfloat16", (256, 256, 32, 2, 4), 8, (256, 256, 768), False),
    ("bfloat16", (16, 128, 64, 1, 4), 8, (16, 1024, 8192), False),
    ("bfloat16", (16, 128, 64, 1, 4), 8, (12, 1024, 4096), False),
    # split-wave register ring: 8 chunks per wave, then 3 and 5 (not multiples of the depth)
    ("float32", (32, 32, 16, 1, 1), 4, (512, 512, 512), False),
    ("float32", (32, 32, 16, 1, 1), 4, (64, 96, 192), False),
    ("float32", (32, 32, 16, 1, 1), 3, (96, 64, 240), False),
]


def _run_depth(a, b, dtype, tile, split_k, stages, trans_b):
    M, K = a.shape
    N = b.shape[1]
    A = _dev(a, dtype)
    B = _dev(np.ascontiguousarray(b.T) if trans_b else b, dtype)
    C = DeviceBuffer(M * N * 4)
    d = capi.MatmulDesc()
    d.dtype = capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16
    d.M, d.N, d.K = M, N, K
    d.tile = capi.Tile(*tile)
    d.split_k = split_k
    d.xcd_remap = 1
    d.trans_b = int(trans_b)
    d.stages = stages
    L = capi.lib()
    capi.check(L.xtc_hip_matmul(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, None), "matmul")
    capi.check(L.xtc_hip_synchronize(), "sync")
    return C.to_numpy((M, N), np.float32)


@pytest.mark.parametrize("case", DEPTH_CASES, ids=[f"{c[0]}-{c[1]}-sk{c[2]}-{c[3]}{'-bt' if c[4] else ''}"
                                                   for c in DEPTH_CASES])
@needs_specialised
def test_every_pipeline_depth(case):
    dtype, tile, split_k, (M, N, K), trans_b = case
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16, M=M, N=N, K=K,
                        tile=capi.Tile(*tile), split_k=split_k, trans_b=int(trans_b))
    depths = capi.matmul_pipeline_depths(d)
    assert len(depths) > 1, depths
    ai, bi = ref.np_init((M, K), "float32"), ref.np_init((K, N), "float32")
    want_int = ref.matmul(ai, bi).astype(np.float32)
    ar, br = rng_uniform(11, (M, K)), rng_uniform(12, (K, N))
    if dtype == "bfloat16":
        ar, br = ref.round_bf16(ar), ref.round_bf16(br)
    default = _run_depth(ar, br, dtype, tile, split_k, 0, trans_b)
    err = ref.scaled_error(default, ref.matmul(ar, br), K, np.abs(ar).max(), np.abs(br).max())
    assert err <= (TOL_F32 if dtype == "float32" else TOL_BF16), err
    for depth in depths:
        print(f"[depth] {depth}", flush=True)
        np.testing.assert_array_equal(_run_depth(ai, bi, dtype, tile, split_k, depth, trans_b), want_int)
        np.testing.assert_array_equal(_run_depth(ar, br, dtype, tile, split_k, depth, trans_b), default)


# the generic template's ring instances (64x64 tiles): three register sets
# of loads in flight; one and two slabs, slab counts that are not multiples
# of 3, ragged M, N, K, one split and several
RING_CASES = [
    ("float32", (64, 64, 32, 2, 2), 4, (512, 512, 512)),
    ("float32", (64, 64, 32, 2, 2), 1, (200, 224, 240)),
    ("float32", (64, 64, 16, 2, 2), 2, (130, 72, 80)),
    ("float32", (64, 64, 16, 2, 2), 1, (64, 64, 16)),
    ("float32", (64, 64, 16, 2, 2), 1, (64, 64, 32)),
    ("bfloat16", (64, 64, 64, 2, 2), 4, (256, 256, 2048)),
    ("bfloat16", (64, 64, 32, 2, 2), 1, (96, 160, 224)),
]


@pytest.mark.parametrize("case", RING_CASES, ids=[f"{c[0]}-{c[1]}-sk{c[2]}-{c[3]}" for c in RING_CASES])
def test_generic_ring_depth(case):
    dtype, tile, split_k, (M, N, K) = case
    d = capi.MatmulDesc(dtype=capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16, M=M, N=N, K=K,
                        tile=capi.Tile(*tile), split_k=split_k)
    depths = capi.matmul_pipeline_depths(d)
    kps = -(-(-(-K // split_k)) // tile[2]) * tile[2]
    assert depths == ([4, 2] if -(-K // kps) > 1 else [2, 4]), depths
    ai, bi = ref.np_init((M, K), "float32"), ref.np_init((K, N), "float32")
    want_int = ref.matmul(ai, bi).astype(np.float32)
    ar, br = rng_uniform(13, (M, K)), rng_uniform(14, (K, N))
    if dtype == "bfloat16":
        ar, br = ref.round_bf16(ar), ref.round_bf16(br)
    base = _run_depth(ar, br, dtype, tile, split_k, 2, False)
    err = ref.scaled_error(base, ref.matmul(ar, br), K, np.abs(ar).max(), np.abs(br).max())
    assert err <= (TOL_F32 if dtype == "float32" else TOL_BF16), err
    for depth in (2, 4):
        print(f"[ring] depth {depth}", flush=True)
        np.testing.assert_array_equal(_run_depth(ai, bi, dtype, tile, split_k, depth, False), want_int)
        # the same slabs in the same order: bit-identical
        np.testing.assert_array_equal(_run_depth(ar, br, dtype, tile, split_k, depth, False), base)
    np.testing.assert_array_equal(_run_depth(ar, br, dtype, tile, split_k, 0, False), base)


@needs_specialised
def test_unsupported_pipeline_depth_is_an_error():
    a, b = rng_uniform(1, (512, 64)), rng_uniform(2, (64, 256))
    with pytest.raises(capi.HipError, match=r"pipeline depths \{3, 2\}, not 5"):
        _run_depth(a, b, "float32", (256, 128, 32, 4, 2), 1, 5, False)


# ------------------------------------------------------------------ direct conv tiles

def test_direct_conv_8x14_tile_matches_8x8():
    # the 8x14-pixel, 1x4-wave direct conv tile (112x64x16, 224 equal blocks
    # for C4): exact on integer inputs, bit-identical to the 8x8 tile on the
    # seeded C4 inputs (same per-output MFMA order over taps and channels)
    x = ref.np_init((8, 56, 56, 64), "float32") % 5
    w = ref.np_init((3, 3, 64, 64), "float32") % 3 - 1
    xp = ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)])
    want = ref.relu(ref.conv2d(xp, w)).astype(np.float32)
    got = run_conv(x, w, pads=(1, 1, 1, 1), tile=(112, 64, 16, 1, 4), relu=True)
    np.testing.assert_array_equal(got, want)
    xs, ws = ref.config_inputs("C4")
    a = run_conv(xs, ws, pads=(1, 1, 1, 1), tile=(112, 64, 16, 1, 4), relu=True)
    b = run_conv(xs, ws, pads=(1, 1, 1, 1), tile=(64, 64, 16, 2, 2), relu=True)
    np.testing.assert_array_equal(a, b)
    xsp = ref.pad(xs, [(0, 0), (1, 1), (1, 1), (0, 0)])
    assert ref.scaled_error(a, ref.relu(ref.conv2d(xsp, ws)), 576, np.abs(xsp).max(), np.abs(ws).max()) <= TOL_F32


def test_direct_conv_7x14_tile():
    # the 7x14-pixel, 1x4-wave tile (98x64x16, 256 blocks for C4): 6 whole
    # 16-pixel tiles per wave as on the 8x14 tile, and the block's last 2
    # pixels on 4x4x1 MFMAs.  Exact on integer inputs; on the seeded C4
    # inputs the whole-tile pixels are bit-identical to the 8x8 tile (same
    # MFMA order), the 2 remainder pixels of each block sum their channels
    # in four phases and are within fp32 rounding
    x = ref.np_init((8, 56, 56, 64), "float32") % 5
    w = ref.np_init((3, 3, 64, 64), "float32") % 3 - 1
    xp = ref.pad(x, [(0, 0), (1, 1), (1, 1), (0, 0)])
    want = ref.relu(ref.conv2d(xp, w)).astype(np.float32)
    got = run_conv(x, w, pads=(1, 1, 1, 1), tile=(98, 64, 16, 1, 4), relu=True)
    np.testing.assert_array_equal(got, want)
    xs, ws = ref.config_inputs("C4")
    a = run_conv(xs, ws, pads=(1, 1, 1, 1), tile=(98, 64, 16, 1, 4), relu=True)
    b = run_conv(xs, ws, pads=(1, 1, 1, 1), tile=(64, 64, 16, 2, 2), relu=True)
    oh, ow = np.meshgrid(np.arange(56), np.arange(56), indexing="ij")
    rem = (oh % 7) * 14 + ow % 14 >= 96  # pixels 96 and 97 of each 7x14 block
    assert rem.sum() == 2 * 8 * 4
    np.testing.assert_array_equal(a[:, ~rem], b[:, ~rem])
    xsp = ref.pad(xs, [(0, 0), (1, 1), (1, 1), (0, 0)])
    assert ref.scaled_error(a, ref.relu(ref.conv2d(xsp, ws)), 576, np.abs(xsp).max(), np.abs(ws).max()) <= TOL_F32


WIDE_DIRECT_TILES = [(112, 64, 16, 1, 4), (98, 64, 16, 1, 4)]


@pytest.mark.parametrize("tile", WIDE_DIRECT_TILES, ids=["8x14", "7x14"])
@pytest.mark.parametrize("shape", [(2, 23, 30, 128, 64, 3, 3, 0), (1, 9, 15, 64, 128, 1, 1, 1), (3, 16, 40, 64, 64, 3, 3, 2)])
def test_direct_conv_wide_ragged(shape, tile):
    # partial blocks in H and W, more than one channel chunk, 1x1 windows, pads of 0-2
    n, h, wd, c, f, r, s, pad = shape
    x = rng_uniform(21, (n, h, wd, c))
    w = rng_uniform(22, (r, s, c, f))
    got = run_conv(x, w, pads=(pad, pad, pad, pad), pad_value=0.25, tile=tile)
    xp = ref.pad(x, [(0, 0), (pad, pad), (pad, pad), (0, 0)], 0.25)
    assert ref.scaled_error(got, ref.conv2d(xp, w), r * s * c, np.abs(xp).max(), 1.0) <= TOL_F32
    # integer inputs: exact, every weight tap of the register ring and every
    # channel chunk (the halo reload between chunks) included
    xi = ref.np_init((n, h, wd, c), "float32") % 5
    wi = ref.np_init((r, s, c, f), "float32") % 3 - 1
    got = run_conv(xi, wi, pads=(pad, pad, pad, pad), pad_value=2.0, tile=tile)
    xpi = ref.pad(xi, [(0, 0), (pad, pad), (pad, pad), (0, 0)], 2.0)
    np.testing.assert_array_equal(got, ref.conv2d(xpi, wi).astype(np.float32))


@pytest.mark.parametrize("tile", WIDE_DIRECT_TILES, ids=["8x14", "7x14"])
@pytest.mark.parametrize("r,s", [(3, 3), (3, 2), (2, 3)])
def test_direct_conv_wide_bias_relu(r, s, tile):
    # 3x3 at stride 1 runs the compile-time-offset kernel, the other windows
    # the general one, on the same tile: bias and relu in the epilogue, two
    # filter blocks, blocks that overhang the image in H and W
    x = rng_uniform(51, (2, 19, 33, 64), 0.0, 1.0)
    w = rng_uniform(52, (r, s, 64, 128), -0.1, 0.1)
    bias = rng_uniform(53, (128,), -0.3, 0.3)
    pads = (r // 2, r // 2, s // 2, s // 2)
    got = run_conv(x, w, pads=pads, tile=tile, relu=True, bias=bias)
    xp = ref.pad(x, [(0, 0), pads[:2], pads[2:], (0, 0)])
    want = ref.relu(ref.conv2d(xp, w) + bias)
    assert ref.scaled_error(got, want, r * s * 64, 1.0, 0.1) <= TOL_F32
    xi = ref.np_init(x.shape, "float32") % 5
    wi = ref.np_init(w.shape, "float32") % 3 - 1
    bi = np.arange(128, dtype=np.float32) % 7 - 3
    got = run_conv(xi, wi, pads=pads, tile=tile, relu=True, bias=bi)
    xpi = ref.pad(xi, [(0, 0), pads[:2], pads[2:], (0, 0)])
    np.testing.assert_array_equal(got, ref.relu(ref.conv2d(xpi, wi) + bi).astype(np.float32))


@pytest.mark.parametrize("tile", WIDE_DIRECT_TILES, ids=["8x14", "7x14"])
def test_direct_only_conv_tile_rejects_other_shapes(tile):
    x, w = rng_uniform(1, (1, 20, 20, 64)), rng_uniform(2, (3, 3, 64, 64))
    with pytest.raises(capi.HipError, match="exists only in the direct conv kernel"):
        run_conv(x, w, stride=(2, 2), tile=tile)
