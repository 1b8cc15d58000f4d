# SPDX-License-Identifier: BSD-3-Clause
"""Pinning of the CPU oracle (oracle/reference.py, oracle/cpu_backend.c).

Every oracle function is checked against something other than a retyping
of its own formula: the reference's printed outputs (tests/test_graphs.py),
integer known-answer tests, closed forms, brute force on tiny shapes, and a
library routine for bf16 rounding.  The C restatement of the llvmir CPU
backend is checked against the float64 oracle on every tile variant.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import cpu_baseline as CB
from oracle import reference as R


# ---------------------------------------------------------------- np_init

def test_np_init_cycles_one_to_nine():
    x = R.np_init((2, 7), "float32")
    assert x.dtype == np.float32
    assert x.ravel().tolist() == [1, 2, 3, 4, 5, 6, 7, 8, 9, 1, 2, 3, 4, 5]
    assert R.np_init((), "int32").tolist() == 1


# ---------------------------------------------------------------- matmul

def test_matmul_closed_forms():
    k = 37
    assert np.all(R.matmul(np.ones((5, k)), np.ones((k, 3))) == k)
    eye = np.eye(6)
    a = np.arange(36.0).reshape(6, 6)
    np.testing.assert_array_equal(R.matmul(a, eye), a)
    np.testing.assert_array_equal(R.matmul(eye, a), a)
    u, v = np.arange(1.0, 5.0), np.arange(1.0, 4.0)
    # rank one: (u 1^T)(1 v^T) = K u v^T
    np.testing.assert_array_equal(R.matmul(np.outer(u, np.ones(k)), np.outer(np.ones(k), v)), k * np.outer(u, v))


def test_matmul_integer_known_answer():
    # A = [[1,2],[3,4]], B = [[5,6],[7,8]]: the textbook product
    np.testing.assert_array_equal(R.matmul(np.array([[1, 2], [3, 4]]), np.array([[5, 6], [7, 8]])),
                                  [[19, 22], [43, 50]])
    # a transposed operand would give [[17, 23], [39, 53]]
    assert not np.array_equal(R.matmul(np.array([[1, 2], [3, 4]]), np.array([[5, 6], [7, 8]]).T), [[19, 22], [43, 50]])


def test_matmul_reshape_rule():
    # operators.py:210-221: A viewed as (shape[0], prod(rest)), B as (prod(rest[:-1]), last)
    a = np.arange(24.0).reshape(2, 3, 4)
    b = np.arange(36.0).reshape(12, 3)
    np.testing.assert_array_equal(R.matmul(a, b), a.reshape(2, 12) @ b)
    b3 = b.reshape(3, 4, 3)
    np.testing.assert_array_equal(R.matmul(a, b3), a.reshape(2, 12) @ b)


# ---------------------------------------------------------------- conv2d

@pytest.mark.parametrize("shape", [
    # (N, H, W, C, R, S, F, SH, SW)
    (1, 5, 5, 1, 3, 3, 1, 1, 1),
    (2, 7, 6, 3, 3, 2, 4, 2, 1),
    (1, 9, 9, 2, 5, 5, 3, 2, 2),
    (3, 4, 8, 5, 1, 1, 2, 1, 3),
])
def test_conv2d_im2col_equals_brute_force(shape):
    n, h, w, c, r, s, f, sh, sw = shape
    rng = np.random.default_rng(sum(shape))
    x = rng.integers(-4, 5, size=(n, h, w, c)).astype(np.float64)
    wt = rng.integers(-4, 5, size=(r, s, c, f)).astype(np.float64)
    fast = R.conv2d(x, wt, (sh, sw))
    oh, ow = (h - r) // sh + 1, (w - s) // sw + 1
    brute = np.zeros((n, oh, ow, f))
    for b in range(n):
        for y in range(oh):
            for z in range(ow):
                for q in range(f):
                    acc = 0.0
                    for i in range(r):
                        for j in range(s):
                            for ch in range(c):
                                acc += x[b, y * sh + i, z * sw + j, ch] * wt[i, j, ch, q]
                    brute[b, y, z, q] = acc
    np.testing.assert_array_equal(fast, brute)
    np.testing.assert_array_equal(R.conv2d_direct(x, wt, (sh, sw)), brute)


def test_conv2d_1x1_is_matmul():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 5, 6, 7))
    w = rng.standard_normal((1, 1, 7, 3))
    np.testing.assert_allclose(R.conv2d(x, w), (x.reshape(-1, 7) @ w.reshape(7, 3)).reshape(2, 5, 6, 3), rtol=1e-12)


def test_conv2d_all_ones_known_answer():
    out = R.conv2d(np.ones((1, 6, 6, 4)), np.ones((3, 3, 4, 2)), (1, 1))
    assert out.shape == (1, 4, 4, 2)
    assert np.all(out == 3 * 3 * 4)
    # a single nonzero input pixel reproduces the flipped-free kernel footprint
    x = np.zeros((1, 5, 5, 1))
    x[0, 2, 2, 0] = 1
    w = np.arange(9.0).reshape(3, 3, 1, 1)
    got = R.conv2d(x, w)[0, :, :, 0]
    # O[y,z] = W[2-y, 2-z]: correlation, not convolution
    np.testing.assert_array_equal(got, w[::-1, ::-1, 0, 0])


# ---------------------------------------------------------------- relu / pad

def test_relu_threshold_and_nan():
    x = np.array([-2.0, -0.0, 0.05, 0.2, np.nan, np.inf, -np.inf])
    got = R.relu(x, 0.1)
    np.testing.assert_array_equal(got[[0, 1, 2, 3, 5, 6]], [0.1, 0.1, 0.1, 0.2, np.inf, 0.1])
    assert np.isnan(got[4])


def test_pad2d_padding_forms():
    assert R.pad2d_padding(4, 2, axes=(1, 2)) == [(0, 0), (2, 2), (2, 2), (0, 0)]
    assert R.pad2d_padding(4, (3,), axes=(1, 2)) == [(0, 0), (3, 3), (3, 3), (0, 0)]
    assert R.pad2d_padding(4, (1, 2), axes=(1, 2)) == [(0, 0), (1, 2), (1, 2), (0, 0)]
    assert R.pad2d_padding(4, ((1, 2), (3, 4)), axes=(1, 2)) == [(0, 0), (1, 2), (3, 4), (0, 0)]
    assert R.pad2d_padding(4, (1, 2, 3, 4), axes=(1, 2)) == [(0, 0), (1, 2), (3, 4), (0, 0)]
    assert R.pad2d_padding(4, 1) == [(0, 0), (1, 1), (1, 1), (0, 0)]


def test_pad_layout():
    x = np.arange(6.0).reshape(1, 2, 3, 1)
    p = R.pad(x, [(0, 0), (1, 2), (3, 0), (0, 0)], value=-1.0)
    assert p.shape == (1, 5, 6, 1)
    np.testing.assert_array_equal(p[0, 1:3, 3:6, 0], x[0, :, :, 0])
    assert np.count_nonzero(p == -1.0) == p.size - x.size


def test_unpad_inverts_pad_and_matches_an_index_loop():
    rng = np.random.default_rng(5)
    x = rng.uniform(-1, 1, (3, 4, 5, 2))
    pads = [(0, 1), (2, 0), (1, 3), (0, 0)]
    # closed form: cropping what pad added gives the input back, whatever the pad value
    np.testing.assert_array_equal(R.unpad(R.pad(x, pads, 7.0), pads), x)
    # brute force on a tiny case: out[o] = in[o + before] per axis
    y = rng.uniform(-1, 1, (4, 6))
    got = R.unpad(y, [(1, 2), (3, 1)])
    assert got.shape == (1, 2)
    for i in range(1):
        for j in range(2):
            assert got[i, j] == y[i + 1, j + 3]
    # a transposed operand or swapped before/after is caught
    assert not np.array_equal(R.unpad(y, [(2, 1), (1, 3)]), got)
    with pytest.raises(ValueError):
        R.unpad(y, [(1, 1)])


# ---------------------------------------------------------------- bf16 rounding

def test_round_bf16_special_cases():
    one = np.float32(1.0)
    ulp = np.float32(2.0**-7)  # bf16 spacing at 1.0
    vals = np.array([1.0, 1 + 2.0**-8, 1 + 3 * 2.0**-8, 1 + 2.0**-8 + 2.0**-20, -1 - 2.0**-8, 0.0, -0.0], np.float32)
    got = R.round_bf16(vals)
    np.testing.assert_array_equal(got[:5], [one, one, one + 2 * ulp, one + ulp, -one])  # ties to even
    assert np.signbit(got[6]) and got[6] == 0
    assert np.isnan(R.round_bf16(np.array([np.nan], np.float32)))[0]
    assert np.isinf(R.round_bf16(np.array([np.inf], np.float32)))[0]


def test_round_bf16_matches_torch_cast():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000), rng.uniform(-1, 1, 100000) * 1e-30, rng.uniform(-1, 1, 1000) * 3e38])
    x = x.astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(R.round_bf16(x), ref)


def test_scaled_error():
    out = np.array([[1.0, 2.0], [3.0, 4.5]])
    ref = np.array([[1.0, 2.0], [3.0, 4.0]])
    assert R.scaled_error(out, ref, k=4, amax_a=1.0, amax_b=0.5) == pytest.approx(0.5 / (2 * 0.5))


# ---------------------------------------------------------------- C restatement of the CPU backend

@pytest.fixture(scope="module")
def cpu():
    return CB.load()


def test_cpu_backend_variants_match_oracle(cpu):
    rng = np.random.default_rng(0)
    for m, n, k in ((37, 53, 29), (64, 128, 96), (1, 10, 128)):
        a = rng.integers(-9, 10, size=(m, k)).astype(np.float32)
        b = rng.integers(-9, 10, size=(k, n)).astype(np.float32)
        exact = R.matmul(a, b)
        for v in range(len(CB.variants())):
            np.testing.assert_array_equal(CB.matmul(a, b, v), exact, err_msg=f"variant {v} {m}x{n}x{k}")


def test_cpu_backend_conv_matches_oracle(cpu):
    rng = np.random.default_rng(1)
    x = rng.integers(-4, 5, size=(2, 9, 8, 3)).astype(np.float32)
    w = rng.integers(-4, 5, size=(3, 3, 3, 5)).astype(np.float32)
    for stride in ((1, 1), (2, 1)):
        np.testing.assert_array_equal(CB.conv2d(x, w, stride), R.conv2d(x, w, stride))
        np.testing.assert_array_equal(CB.conv2d(x, w, stride, relu=True), R.relu(R.conv2d(x, w, stride)))


def test_cpu_backend_rejects_bad_variant(cpu):
    a = np.ones((4, 4), np.float32)
    with pytest.raises(ValueError):
        CB.matmul(a, a, variant=len(CB.variants()))


def test_c5_integer_rounding_is_order_dependent(cpu):
    """The C5 MLP on np_init inputs leaves fp32's exact-integer range: fc2
    sums reach ~5e8 > 2^24, so each fp32 summation order rounds differently.
    The K-sequential loop of the llvmir nest (the reference CPU backend's
    order) is 2.85e-5 off the exact value and fails np.allclose's default
    rtol=1e-5 against both it and numpy's blocked fp32 BLAS, which pairwise
    sums and stays at 3.2e-6.  Every order is within 1e-4."""
    x = R.np_init((2048, 1024), "float32")
    w1 = R.np_init((1024, 4096), "float32")
    w2 = R.np_init((4096, 1024), "float32")
    h = R.relu(CB.matmul(x, w1))
    np.testing.assert_array_equal(h, R.relu(R.matmul(x, w1)))  # fc1 is exact in fp32 (< 2^24)
    seq = CB.matmul(h, w2)
    blas = h @ w2
    exact = R.matmul(h, w2)
    assert exact.max() > 2**24
    assert not np.allclose(seq, exact)
    assert not np.allclose(seq, blas)
    assert np.allclose(seq, blas, rtol=1e-4)
    assert np.allclose(seq, exact, rtol=1e-4)
    assert np.allclose(blas, exact, rtol=1e-4)


def test_cpu_backend_single_schedule_builds_are_exact():
    # one compiled object per sampled tile_oo schedule (i1, k1, j1), ragged
    # against the shape: exact on integer inputs like the fixed variants
    import ctypes

    from oracle import cpu_baseline as cb

    a = R.np_init((37, 70), "float32")
    b = R.np_init((70, 45), "float32")
    want = R.matmul(a, b).astype(np.float32)
    for tiles in [(1, 1, 8), (2, 4, 16), (8, 64, 32), (5, 3, 7)]:
        lib = cb.schedule_lib(*tiles)
        lib.xtc_cpu_sched_configure(37, 45, 70)
        c = np.full((37, 45), np.nan, np.float32)
        lib.xtc_cpu_sched_payload.argtypes = [ctypes.c_void_p] * 3
        lib.xtc_cpu_sched_payload(a.ctypes.data, b.ctypes.data, c.ctypes.data)
        np.testing.assert_array_equal(c, want, err_msg=str(tiles))


def test_cpu_backend_pprprp_schedules_are_exact_and_follow_the_strategy():
    # tile_pprprp_vr samples of a 64 x 96 x 48 matmul, each built as its own
    # object with the sample's 7 tile extents: exact on integer inputs
    import ctypes

    from oracle import cpu_baseline as cb
    from xtc_amd.cli.explore import build_graph
    from xtc_amd.search.strategies import Strategies

    m, n, k = 64, 96, 48
    strategy = Strategies.create("tile_pprprp_vr", build_graph("matmul", [m, n, k], "float32"), threads=4)
    samples = list(strategy.sample(6, seed=0))
    a = R.np_init((m, k), "float32")
    b = R.np_init((k, n), "float32")
    want = R.matmul(a, b).astype(np.float32)
    for x in samples:
        tiles = cb.pprprp_tiles(strategy, x)
        i1, i2, i3, j1, j2, j3, k1 = tiles
        # nested extents of one axis divide each other, as factors_to_sizes gives them
        assert m % i1 == 0 and i1 % i2 == 0 and i2 % i3 == 0 and n % j1 == 0 and j1 % j2 == 0 and j2 % j3 == 0
        assert k % k1 == 0 and j3 >= 16  # the vector filter of tile_pprprp_vr
        lib = cb.schedule_lib(*tiles)
        lib.xtc_cpu_sched_configure(m, n, k)
        c = np.full((m, n), np.nan, np.float32)
        lib.xtc_cpu_sched_payload.argtypes = [ctypes.c_void_p] * 3
        lib.xtc_cpu_sched_payload(a.ctypes.data, b.ctypes.data, c.ctypes.data)
        np.testing.assert_array_equal(c, want, err_msg=str(tiles))
