# SPDX-License-Identifier: BSD-3-Clause
"""Seeded random shapes through the C ABI, exact on small-integer inputs.

Matmuls: M, N, K drawn from 1..640 (N and K multiples of the 16-byte
vector, as the MFMA paths need; ragged otherwise), any compiled tile of the
dtype, split-K 1-8, every pipeline depth the library reports for the case,
and operand layouts (A and/or B stored transposed).  Convs: N 1-3, H and W
5-40, C a multiple of the vector or 3 (channel staging), F a multiple of
the vector, 1x1 to 5x5 windows, strides 1-3, asymmetric pads with a pad
value, any compiled conv tile, split-K 1-4.  Inputs are integers (1..9 and
-4..4), so every fp32 sum is exact and the output must equal the float64
oracle bit for bit.  The cases are drawn once from fixed seeds (448 of
them, then a wider draw of 2620 from other seeds); each one is checked on
the host (the library's own descriptor checks) before its GPU step.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import reference as ref
from test_gpu_kernels import _dev, run_conv
from xtc_amd.runtimes.hip import capi
from xtc_amd.runtimes.hip.buffer import DeviceBuffer

pytestmark = pytest.mark.gpu


# conv tiles only the direct kernel implements (C and F multiples of 64)
DIRECT_ONLY = {(112, 64, 16, 1, 4), (98, 64, 16, 1, 4)}


def _tiles(dtype: str, conv: bool) -> list[tuple[int, ...]]:
    return sorted({tuple(i["tile"]) for i in capi.gemm_instances() if i["dtype"] == dtype and bool(i["conv"]) == conv})


def _matmul_cases(n: int, seed: int) -> list[tuple]:
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dtype = "float32" if i % 3 else "bfloat16"
        vec = 4 if dtype == "float32" else 8
        M = int(rng.integers(1, 641))
        N = int(rng.integers(1, 641 // vec)) * vec
        K = int(rng.integers(1, 641 // vec)) * vec
        tiles = _tiles(dtype, False)
        tile = tiles[int(rng.integers(len(tiles)))]
        split = int(rng.choice([1, 1, 2, 3, 4, 8]))
        ta, tb = bool(rng.integers(2)), bool(rng.integers(2))
        out.append((i, dtype, M, N, K, tile, split, ta, tb))
    return out


def _conv_cases(n: int, seed: int) -> list[tuple]:
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dtype = "float32" if i % 3 else "bfloat16"
        vec = 4 if dtype == "float32" else 8
        nb = int(rng.integers(1, 4))
        h, w = int(rng.integers(5, 41)), int(rng.integers(5, 41))
        c = 3 if i % 5 == 0 else int(rng.integers(1, 9)) * vec
        f = int(rng.integers(1, 9)) * vec
        r, s = int(rng.integers(1, 6)), int(rng.integers(1, 6))
        sh, sw = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        pads = tuple(int(p) for p in rng.integers(0, 3, size=4))
        if h + pads[0] + pads[1] < r or w + pads[2] + pads[3] < s:
            continue
        tiles = [t for t in _tiles(dtype, True) if t not in DIRECT_ONLY]
        tile = tiles[int(rng.integers(len(tiles)))]
        split = int(rng.choice([1, 1, 2, 4]))
        out.append((i, dtype, nb, h, w, c, f, r, s, sh, sw, pads, tile, split))
    return out


MATMUL = _matmul_cases(240, 2024)
CONV = _conv_cases(160, 2025)


def _matmul_desc(dtype, M, N, K, tile, split, ta, tb, stages=0):
    return capi.MatmulDesc(dtype=capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16, M=M, N=N, K=K,
                           tile=capi.Tile(*tile), split_k=split, xcd_remap=1, trans_a=int(ta), trans_b=int(tb),
                           stages=stages)


@pytest.mark.parametrize("case", MATMUL, ids=[f"mm{c[0]}-{c[1]}-{c[2]}x{c[3]}x{c[4]}" for c in MATMUL])
def test_random_matmul_exact(case):
    i, dtype, M, N, K, tile, split, ta, tb = case
    depths = capi.matmul_pipeline_depths(_matmul_desc(dtype, M, N, K, tile, split, ta, tb))
    assert depths, depths
    rng = np.random.default_rng(1000 + i)
    a = rng.integers(1, 10, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (K, N)).astype(np.float32)
    want = ref.matmul(a, b).astype(np.float32)
    A = _dev(np.ascontiguousarray(a.T) if ta else a, dtype)
    B = _dev(np.ascontiguousarray(b.T) if tb else b, dtype)
    L = capi.lib()
    for depth in depths:
        print(f"[random] mm{i} {dtype} {M}x{N}x{K} tile={tile} split={split} ta={ta} tb={tb} depth={depth}",
              flush=True)
        C = DeviceBuffer(M * N * 4)
        d = _matmul_desc(dtype, M, N, K, tile, split, ta, tb, depth)
        capi.check(L.xtc_hip_matmul(capi.ctypes.byref(d), A.c_ptr, B.c_ptr, C.c_ptr, None), "matmul")
        capi.check(L.xtc_hip_synchronize(), "sync")
        np.testing.assert_array_equal(C.to_numpy((M, N), np.float32), want)


@pytest.mark.parametrize("case", CONV, ids=[f"conv{c[0]}-{c[1]}" for c in CONV])
def test_random_conv_exact(case):
    i, dtype, nb, h, w, c, f, r, s, sh, sw, pads, tile, split = case
    cd = capi.Conv2dDesc(dtype=capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16, N=nb, H=h, W=w, C=c,
                         F=f, R=r, S=s, stride_h=sh, stride_w=sw, pad_top=pads[0], pad_bottom=pads[1],
                         pad_left=pads[2], pad_right=pads[3], tile=capi.Tile(*tile), split_k=split)
    assert capi.conv2d_pipeline_depths(cd)
    rng = np.random.default_rng(2000 + i)
    x = rng.integers(1, 10, (nb, h, w, c)).astype(np.float32)
    wt = rng.integers(-4, 5, (r, s, c, f)).astype(np.float32)
    xp = ref.pad(x, [(0, 0), (pads[0], pads[1]), (pads[2], pads[3]), (0, 0)], 2.0)
    want = ref.conv2d(xp, wt, (sh, sw)).astype(np.float32)
    print(f"[random] conv{i} {dtype} x={x.shape} w={wt.shape} stride=({sh},{sw}) pads={pads} tile={tile} "
          f"split={split}", flush=True)
    got = run_conv(x, wt, dtype, stride=(sh, sw), pads=pads, pad_value=2.0, tile=tile, split_k=split)
    np.testing.assert_array_equal(got, want)


def _direct_conv_cases(n: int, seed: int, wide: tuple[int, ...] = (112, 64, 16, 1, 4)) -> list[tuple]:
    """fp32 convs the direct kernel takes (C and F multiples of 64, the block's
    halo within its LDS buffer): two in three on the 1x4-wave tile `wide`
    (8x14 pixels, or 7x14 with its 2 pixels on 4x4x1 MFMAs), the rest on
    8x8; half of them 3x3 at stride 1, which run the compile-time-offset
    kernel."""
    rng = np.random.default_rng(seed)
    out = []
    halo_pix = {(112, 64, 16, 1, 4): (8, 14, 49152 // 272), (98, 64, 16, 1, 4): (7, 14, 49152 // 272),
                (64, 64, 16, 2, 2): (8, 8, 32768 // 272)}
    while len(out) < n:
        i = len(out)
        tile = wide if i % 3 else (64, 64, 16, 2, 2)
        th, tw, cap = halo_pix[tile]
        if i % 2 == 0:
            r = s = 3
            sh = sw = 1
        else:
            r, s = int(rng.integers(1, 4)), int(rng.integers(1, 4))
            sh, sw = int(rng.integers(1, 3)), int(rng.integers(1, 3))
        if ((th - 1) * sh + r) * ((tw - 1) * sw + s) > cap:
            continue
        nb = int(rng.integers(1, 4))
        h, w = int(rng.integers(5, 41)), int(rng.integers(5, 41))
        c = int(rng.choice([64, 128, 192]))
        f = int(rng.choice([64, 128]))
        pads = tuple(int(p) for p in rng.integers(0, 3, size=4))
        if h + pads[0] + pads[1] < r or w + pads[2] + pads[3] < s:
            continue
        out.append((i, nb, h, w, c, f, r, s, sh, sw, pads, tile, bool(rng.integers(2))))
    return out


DIRECT = _direct_conv_cases(24, 2026) + _direct_conv_cases(24, 2027, (98, 64, 16, 1, 4))


@pytest.mark.parametrize("case", DIRECT, ids=[f"dconv{k}-{c[6]}x{c[7]}s{c[8]}{c[9]}" for k, c in enumerate(DIRECT)])
def test_random_direct_conv_exact(case):
    i, nb, h, w, c, f, r, s, sh, sw, pads, tile, with_bias = case
    rng = np.random.default_rng(3000 + i)
    x = rng.integers(1, 10, (nb, h, w, c)).astype(np.float32)
    wt = rng.integers(-4, 5, (r, s, c, f)).astype(np.float32)
    bias = rng.integers(-3, 4, (f,)).astype(np.float32) if with_bias else None
    xp = ref.pad(x, [(0, 0), (pads[0], pads[1]), (pads[2], pads[3]), (0, 0)], 2.0)
    want = ref.relu(ref.conv2d(xp, wt, (sh, sw)) + (bias if with_bias else 0.0)).astype(np.float32)
    print(f"[random] dconv{i} x={x.shape} w={wt.shape} stride=({sh},{sw}) pads={pads} tile={tile} bias={with_bias}",
          flush=True)
    got = run_conv(x, wt, "float32", stride=(sh, sw), pads=pads, pad_value=2.0, tile=tile, relu=True, bias=bias)
    np.testing.assert_array_equal(got, want)


# A wider draw of the same generators from other seeds: 1500 matmuls, 800
# convs and 320 direct convs more, each exact as above (about 6 s on MI355X).
WIDE_MATMUL = _matmul_cases(1500, 7001)
WIDE_CONV = _conv_cases(800, 7002)
WIDE_DIRECT = _direct_conv_cases(160, 7003) + _direct_conv_cases(160, 7004, (98, 64, 16, 1, 4))


@pytest.mark.parametrize("case", WIDE_MATMUL, ids=[f"wmm{c[0]}-{c[1]}-{c[2]}x{c[3]}x{c[4]}" for c in WIDE_MATMUL])
def test_wide_random_matmul_exact(case):
    test_random_matmul_exact(case)


@pytest.mark.parametrize("case", WIDE_CONV, ids=[f"wconv{c[0]}-{c[1]}" for c in WIDE_CONV])
def test_wide_random_conv_exact(case):
    test_random_conv_exact(case)


@pytest.mark.parametrize("case", WIDE_DIRECT, ids=[f"wdconv{k}" for k in range(len(WIDE_DIRECT))])
def test_wide_random_direct_conv_exact(case):
    test_random_direct_conv_exact(case)
