# SPDX-License-Identifier: BSD-3-Clause
"""xtc_hip_matmul_noalloc against xtc_hip_matmul, through the C-ABI.

The no-allocation entry point runs the same kernels as xtc_hip_matmul with its
scratch (split-K partial sums and counters, transposed-operand copies) in the
library's static per-device array, so its outputs must be bit-identical.  Each
case makes two calls in a row, the second on a smaller input, because the
array keeps the previous call's contents.  The outputs are also checked
against the float64 oracle at the usual tolerance.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import reference as ref
from xtc_amd.runtimes.hip import capi
from xtc_amd.runtimes.hip.buffer import DeviceBuffer, ensure_device
from xtc_amd.utils.bf16 import f32_to_bf16_bits

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


@pytest.fixture(scope="module", autouse=True)
def device():
    ensure_device(0)
    yield


def _desc(dtype, M, N, K, tile, split_k, trans_a=False, trans_b=False, relu=False):
    d = capi.MatmulDesc()
    d.dtype = capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16
    d.M, d.N, d.K = M, N, K
    if tile is not None:
        d.tile = capi.Tile(*tile)
    d.split_k = split_k
    d.xcd_remap = 1
    d.relu = int(relu)
    d.trans_a = int(trans_a)
    d.trans_b = int(trans_b)
    return d


def _upload(x, dtype):
    if dtype == "bfloat16":
        return DeviceBuffer.from_numpy(f32_to_bf16_bits(x))
    return DeviceBuffer.from_numpy(np.ascontiguousarray(x, dtype=np.float32))


def _both(dtype, M, N, K, tile, split_k, seed, trans_a=False, trans_b=False, relu=False, bias=False):
    """(noalloc output, xtc_hip_matmul output, oracle, scale) for one shape."""
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    bv = rng.uniform(-1, 1, N).astype(np.float32) if bias else None
    if dtype == "bfloat16":
        a, b = ref.round_bf16(a), ref.round_bf16(b)
    A = _upload(a.T.copy() if trans_a else a, dtype)
    B = _upload(b.T.copy() if trans_b else b, dtype)
    bias_buf = DeviceBuffer.from_numpy(bv) if bias else None
    d = _desc(dtype, M, N, K, tile, split_k, trans_a, trans_b, relu)
    L = capi.lib()
    outs = []
    for fn in (L.xtc_hip_matmul_noalloc, L.xtc_hip_matmul):
        C = DeviceBuffer(M * N * 4)
        C.zero()
        capi.check(fn(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, bias_buf.c_ptr if bias else None), fn.__name__)
        capi.check(L.xtc_hip_synchronize(), "sync")
        outs.append(C.to_numpy((M, N), np.float32))
    want = ref.matmul(a, b)
    if bias:
        want = want + bv.astype(np.float64)
    if relu:
        want = np.maximum(want, 0.0)
    return outs[0], outs[1], want, (K, np.abs(a).max(), np.abs(b).max())


# (dtype, tile, split_k, first (M, N, K), second (M, N, K), options): every
# kernel family that takes scratch, plus one that takes none.
CASES = [
    # generic template, grid split-K: partials [4][M][N] and per-tile counters
    ("float32", (64, 64, 32, 2, 2), 4, (384, 320, 2048), (128, 192, 1024), {}),
    # LDS-DMA fp32 kernel with split-K 2, relu and bias in the finishing workgroup
    ("float32", (128, 128, 32, 2, 4), 2, (1024, 512, 2048), (512, 256, 512), {"relu": True, "bias": True}),
    # skinny bf16 kernel: split-K 8 over 1024-deep, then 512-deep chunks
    ("bfloat16", (16, 128, 64, 1, 4), 8, (16, 8192, 8192), (8, 4096, 4096), {}),
    # generic bf16 template with split-K 3 (ragged K per split)
    ("bfloat16", (64, 64, 64, 2, 2), 3, (256, 256, 1600), (64, 128, 704), {}),
    # transposed A and B: both staged in the scratch, then split-K 2
    ("float32", (64, 64, 32, 2, 2), 2, (512, 256, 384), (96, 160, 256), {"trans_a": True, "trans_b": True}),
    # split-wave kernel: scratch-free (partials meet in LDS)
    ("float32", (32, 32, 16, 1, 1), 4, (512, 512, 512), (256, 128, 256), {}),
    # ping-pong bf16 kernel, no split: scratch-free
    ("bfloat16", (256, 256, 32, 2, 4), 1, (1024, 1024, 1024), (512, 256, 512), {}),
    # ping-pong bf16 kernel with split-K 4: partials and counters, relu and bias
    ("bfloat16", (256, 256, 32, 2, 4), 4, (512, 768, 2048), (256, 256, 1024), {"relu": True, "bias": True}),
    # ping-pong bf16 kernel reading B^T natively, split-K 2
    ("bfloat16", (256, 256, 32, 2, 4), 2, (512, 512, 1024), (256, 512, 512), {"trans_b": True}),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[1]}-sk{c[2]}" for c in CASES])
def test_noalloc_matches_matmul_on_two_calls(case):
    dtype, tile, split_k, first, second, opts = case
    for seed, (M, N, K) in enumerate((first, second)):
        got, want_same, want, (k, ma, mb) = _both(dtype, M, N, K, tile, split_k, seed, **opts)
        np.testing.assert_array_equal(got, want_same)
        err = ref.scaled_error(got, want, k, ma, mb)
        assert err <= (1e-4 if dtype == "float32" else 1e-2), (M, N, K, err)


def test_noalloc_rejects_scratch_above_the_maximum():
    # fp32 4096^2 split-K 2 needs 128 MiB of partial sums: refused, and the
    # allocating entry point still runs the same call afterwards
    M = N = 4096
    K = 512
    d = _desc("float32", M, N, K, (128, 128, 32, 2, 4), 2)
    assert 2 * M * N * 4 > SCRATCH_BYTES
    L = capi.lib()
    A = DeviceBuffer(M * K * 4)
    B = DeviceBuffer(K * N * 4)
    C = DeviceBuffer(M * N * 4)
    A.zero()
    B.zero()
    status = L.xtc_hip_matmul_noalloc(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, None)
    assert status != 0
    assert "scratch" in capi.last_error()
    capi.check(L.xtc_hip_matmul(ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, None), "matmul")
    capi.check(L.xtc_hip_synchronize(), "sync")
    assert not C.to_numpy((M, N), np.float32).any()
