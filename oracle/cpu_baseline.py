# SPDX-License-Identifier: BSD-3-Clause
"""TEST INFRASTRUCTURE: driver of the CPU baseline (oracle/cpu_backend.c).

Builds the C restatement of XTC's `llvmir` CPU backend for the host it runs
on (-march=native must match the machine, so the object is built per host),
auto-schedules it by timing every compiled tile variant, and times the best
one with the reference's evaluate_perf protocol: one warm-up call, then per
repeat a call count doubling until the batch lasts min_repeat_ms, result =
batch time / calls, min over repeats
(src/xtc/csrcs/runtimes/host/evaluate_perf.c:63-125).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import platform
import subprocess
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "cpu_backend.c"

__all__ = [
    "load",
    "schedule_lib",
    "time_schedule",
    "autoschedule_tile_oo",
    "autoschedule_strategy",
    "time_schedule_repeats",
    "pprprp_tiles",
    "threads",
    "matmul",
    "conv2d",
    "time_matmul",
    "autoschedule_matmul",
    "cpu_model",
    "ref_runtime",
    "ref_peak_flops",
]

REF_RUNTIME = HERE / "_ref" / "libxtc_ref_runtime.so"
_ref: ctypes.CDLL | None = None


def ref_runtime() -> ctypes.CDLL | None:
    """The reference's own host runtime built by `make -C oracle ref`
    (evaluate_perf, evaluate_flops), or None when it was not built."""
    global _ref
    if _ref is None and REF_RUNTIME.exists():
        h = ctypes.CDLL(str(REF_RUNTIME))
        h.evaluate_perf.argtypes = [
            ctypes.POINTER(ctypes.c_double),
            ctypes.c_int,
            ctypes.POINTER(ctypes.c_char_p),
            ctypes.c_int,
            ctypes.c_int,
            ctypes.c_int,
            ctypes.c_void_p,
            ctypes.POINTER(ctypes.c_void_p),
            ctypes.c_int,
        ]
        h.evaluate_perf.restype = None
        h.evaluate_flops.argtypes = [ctypes.c_char_p]
        h.evaluate_flops.restype = ctypes.c_double
        _ref = h
    return _ref


def ref_peak_flops(dtype: str = "float32") -> float | None:
    """Single-core FMA/s peak from the reference's evaluate_flops
    (src/xtc/csrcs/runtimes/host/evaluate_flops.c:461-494)."""
    h = ref_runtime()
    return None if h is None else float(h.evaluate_flops(dtype.encode()))

_lib: ctypes.CDLL | None = None


def _host_key() -> str:
    info = platform.node() + platform.machine() + cpu_model()
    return hashlib.sha256((info + SRC.read_text()).encode()).hexdigest()[:12]


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def load() -> ctypes.CDLL:
    """Builds (once per host) and loads libxtc_cpu.so."""
    global _lib
    if _lib is not None:
        return _lib
    out_dir = HERE / "_build" / _host_key()
    lib = out_dir / "libxtc_cpu.so"
    if not lib.exists():
        out_dir.mkdir(parents=True, exist_ok=True)
        cc = os.environ.get("CC", "gcc")
        tmp = lib.with_suffix(f".so.tmp{os.getpid()}")
        cmd = [cc, "-O3", "-march=native", "-ffp-contract=fast", "-fopenmp", "-fPIC", "-std=c11",
               "-shared", "-o", str(tmp), str(SRC)]
        subprocess.run(cmd, check=True, capture_output=True)
        os.replace(tmp, lib)
    handle = ctypes.CDLL(str(lib))
    fp = ctypes.POINTER(ctypes.c_float)
    handle.xtc_cpu_matmul.argtypes = [ctypes.c_int, fp, fp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    handle.xtc_cpu_matmul.restype = ctypes.c_int
    handle.xtc_cpu_conv2d.argtypes = [fp, fp, fp] + [ctypes.c_int] * 10
    handle.xtc_cpu_conv2d.restype = ctypes.c_int
    handle.xtc_cpu_matmul_variant_tiles.argtypes = [ctypes.c_int] + [ctypes.POINTER(ctypes.c_int)] * 3
    handle.xtc_cpu_set_threads.argtypes = [ctypes.c_int]
    handle.xtc_cpu_configure_matmul.argtypes = [ctypes.c_int] * 4
    _lib = handle
    return handle


def threads(n: int | None = None) -> int:
    lib = load()
    if n:
        lib.xtc_cpu_set_threads(int(n))
    return int(lib.xtc_cpu_threads())


def variants() -> list[tuple[int, int, int]]:
    lib = load()
    out = []
    for v in range(lib.xtc_cpu_matmul_variants()):
        ti, tk, tj = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        lib.xtc_cpu_matmul_variant_tiles(v, ctypes.byref(ti), ctypes.byref(tk), ctypes.byref(tj))
        out.append((ti.value, tk.value, tj.value))
    return out


def _fp(a: np.ndarray) -> "ctypes._Pointer[ctypes.c_float]":
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def matmul(a: np.ndarray, b: np.ndarray, variant: int = 0) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    if load().xtc_cpu_matmul(variant, _fp(a), _fp(b), _fp(c), m, n, k):
        raise ValueError("xtc_cpu_matmul rejected its arguments")
    return c


def conv2d(x_padded: np.ndarray, w: np.ndarray, stride: tuple[int, int] = (1, 1), relu: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(x_padded, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    nb, h, wd, c = x.shape
    r, s, _, f = w.shape
    oh, ow = (h - r) // stride[0] + 1, (wd - s) // stride[1] + 1
    o = np.empty((nb, oh, ow, f), np.float32)
    if load().xtc_cpu_conv2d(_fp(x), _fp(w), _fp(o), nb, h, wd, c, f, r, s, stride[0], stride[1], int(relu)):
        raise ValueError("xtc_cpu_conv2d rejected its arguments")
    return o


def time_call(fn, repeat: int = 3, min_repeat_ms: int = 100) -> float:  # type: ignore[no-untyped-def]
    """evaluate_perf protocol; returns min over repeats of seconds per call."""
    fn()
    best = float("inf")
    for _ in range(repeat):
        calls = 1
        while True:
            t0 = time.perf_counter()
            for _ in range(calls):
                fn()
            dt = time.perf_counter() - t0
            if dt * 1000.0 >= min_repeat_ms:
                break
            calls *= 2
        best = min(best, dt / calls)
    return best


def time_matmul(a: np.ndarray, b: np.ndarray, variant: int, repeat: int = 3, min_repeat_ms: int = 100) -> float:
    """Seconds per call of one variant, min over repeats.  Uses the
    reference's own evaluate_perf when oracle/_ref is built, else the same
    protocol restated in Python."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib = load()
    ref = ref_runtime()
    if ref is not None:
        if lib.xtc_cpu_configure_matmul(variant, m, n, k):
            raise ValueError("bad matmul configuration")
        results = (ctypes.c_double * repeat)()
        args = (ctypes.c_void_p * 3)(a.ctypes.data, b.ctypes.data, c.ctypes.data)
        fn = ctypes.cast(lib.xtc_cpu_matmul_payload, ctypes.c_void_p)
        ref.evaluate_perf(results, 0, None, repeat, 1, min_repeat_ms, fn, args, 3)
        return float(min(results))
    pa, pb, pc = _fp(a), _fp(b), _fp(c)
    return time_call(lambda: lib.xtc_cpu_matmul(variant, pa, pb, pc, m, n, k), repeat, min_repeat_ms)


_sched_libs: dict[tuple[int, ...], ctypes.CDLL] = {}


def _sched_defines(tiles: tuple[int, ...]) -> list[str]:
    """Compile-time tile constants of one schedule: 3 extents are a tile_oo
    schedule (i1, k1, j1); 7 are a tile_pprprp one (i1, i2, i3, j1, j2, j3, k1)."""
    if len(tiles) == 3:
        return [f"-DXTC_CPU_{n}={v}" for n, v in zip(("TI", "TK", "TJ"), tiles)]
    if len(tiles) == 7:
        return ["-DXTC_CPU_PPRPRP"] + [f"-DXTC_CPU_{n}={v}" for n, v in zip(("I1", "I2", "I3", "J1", "J2", "J3", "K1"),
                                                                             tiles)]
    raise ValueError(f"schedule tiles {tiles}: expected 3 (tile_oo) or 7 (tile_pprprp) extents")


def schedule_lib(*tiles: int) -> ctypes.CDLL:
    """The restatement built for one schedule, tiles as compile-time
    constants (see _sched_defines); cached per host."""
    key = tuple(int(t) for t in tiles)
    if key in _sched_libs:
        return _sched_libs[key]
    out_dir = HERE / "_build" / _host_key()
    tag = ("pprprp_" if len(key) == 7 else "") + "_".join(map(str, key))
    lib = out_dir / f"libxtc_cpu_sched_{tag}.so"
    if not lib.exists():
        out_dir.mkdir(parents=True, exist_ok=True)
        cc = os.environ.get("CC", "gcc")
        tmp = lib.with_suffix(f".so.tmp{os.getpid()}")
        cmd = [cc, "-O3", "-march=native", "-ffp-contract=fast", "-fopenmp", "-fPIC", "-std=c11", "-shared",
               *_sched_defines(key), "-o", str(tmp), str(SRC)]
        subprocess.run(cmd, check=True, capture_output=True)
        os.replace(tmp, lib)
    handle = ctypes.CDLL(str(lib))
    handle.xtc_cpu_sched_configure.argtypes = [ctypes.c_int] * 3
    handle.xtc_cpu_sched_configure.restype = None
    _sched_libs[key] = handle
    return handle


def time_schedule_repeats(tiles: tuple[int, ...], a: np.ndarray, b: np.ndarray, repeat: int = 2, number: int = 1,
                          min_repeat_ms: int = 50) -> list[float]:
    """Seconds per call of one compiled schedule for each repeat, with the
    reference's evaluate_perf when oracle/_ref is built (one warm-up call,
    then per repeat calls doubling from `number` until min_repeat_ms)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib = schedule_lib(*tiles)
    lib.xtc_cpu_sched_configure(m, n, k)
    ref = ref_runtime()
    fn = ctypes.cast(lib.xtc_cpu_sched_payload, ctypes.c_void_p)
    if ref is not None:
        results = (ctypes.c_double * repeat)()
        args = (ctypes.c_void_p * 3)(a.ctypes.data, b.ctypes.data, c.ctypes.data)
        ref.evaluate_perf(results, 0, None, repeat, number, min_repeat_ms, fn, args, 3)
        return [float(x) for x in results]
    payload = lib.xtc_cpu_sched_payload
    payload.argtypes = [ctypes.c_void_p] * 3
    return [time_call(lambda: payload(a.ctypes.data, b.ctypes.data, c.ctypes.data), 1, min_repeat_ms)
            for _ in range(repeat)]


def time_schedule(tiles: tuple[int, ...], a: np.ndarray, b: np.ndarray, repeat: int = 2, number: int = 1,
                  min_repeat_ms: int = 50) -> float:
    """Seconds per call of one compiled schedule, min over repeats."""
    return min(time_schedule_repeats(tiles, a, b, repeat, number, min_repeat_ms))


class _TileRecorder:
    """Scheduler stand-in that records the tile extents a strategy's
    generate() asks for (the only calls the PRT strategies make that the
    restatement needs; the loop order, parallel, vector and unroll choices
    of a scheme are fixed by the scheme and built into cpu_backend.c)."""

    def __init__(self) -> None:
        self.tiles: dict[str, dict[str, int]] = {}

    def tile(self, axis: str, tiles: dict[str, int], root: str = ".") -> None:
        self.tiles[axis] = dict(tiles)

    def __getattr__(self, name: str):  # interchange, parallelize, vectorize, unroll, ...
        return lambda *a, **k: None


def pprprp_tiles(strategy, sample) -> tuple[int, ...]:  # type: ignore[no-untyped-def]
    """(i1, i2, i3, j1, j2, j3, k1) extents of a tile_pprprp* sample."""
    rec = _TileRecorder()
    strategy.generate(rec, sample)
    t = rec.tiles
    return (t["i"]["i1"], t["i"]["i2"], t["i"]["i3"], t["j"]["j1"], t["j"]["j2"], t["j"]["j3"], t["k"]["k1"])


def autoschedule_tile_oo(n: int, trials: int = 64, seed: int = 0, bf16: bool = False,
                         jobs: int = 8) -> tuple[tuple[int, int, int], float, int]:
    """loop-explore of the restatement: `trials` seeded random samples of the
    reference's tile_oo strategy (src/xtc/search/strategies.py:739-758,
    restated in xtc_amd/search/strategies.py) for an n^3 fp32 matmul, each
    compiled as its own object and timed with the evaluate_perf protocol.
    Returns (best (i1, k1, j1), its seconds per call, samples timed)."""
    import concurrent.futures as cf

    from xtc_amd.cli.explore import build_graph
    from xtc_amd.search.strategies import Strategies

    graph = build_graph("matmul", [n, n, n], "float32")
    strategy = Strategies.create("tile_oo", graph, threads=threads())
    names = strategy.sample_names
    samples = [dict(zip(names, x)) for x in strategy.sample(trials, seed=seed)]
    # tile_oo's sample is (i1, j1, k1); the restatement takes (i1, k1, j1)
    tiles = [(x[names[0]], x[names[2]], x[names[1]]) for x in samples]
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(lambda t: schedule_lib(*t), tiles))
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    if bf16:
        from xtc_amd.utils.bf16 import round_to_bf16

        a, b = round_to_bf16(a), round_to_bf16(b)
    timed = [(time_schedule(t, a, b, repeat=1, min_repeat_ms=20), t) for t in tiles]
    t, best = min(timed)
    return best, t, len(timed)


def autoschedule_strategy(name: str, n: int, trials: int = 64, seed: int = 0, bf16: bool = False,
                          jobs: int = 8) -> list[tuple[float, tuple[int, ...]]]:
    """loop-explore of the restatement with one of the reference's PRT
    strategies ("tile_oo" or "tile_pprprp_vr", src/xtc/search/strategies.py:
    739-826, restated in xtc_amd/search/strategies.py): `trials` seeded
    random samples for an n^3 fp32 matmul, each compiled as its own object
    and timed once (min_repeat_ms 20).  Returns [(seconds per call, tiles)]
    sorted fastest first; tiles as schedule_lib takes them."""
    import concurrent.futures as cf

    from xtc_amd.cli.explore import build_graph
    from xtc_amd.search.strategies import Strategies

    graph = build_graph("matmul", [n, n, n], "float32")
    strategy = Strategies.create(name, graph, threads=threads())
    names = strategy.sample_names
    samples = list(strategy.sample(trials, seed=seed))
    if name == "tile_oo":
        # tile_oo's sample is (i1, j1, k1); the restatement takes (i1, k1, j1)
        tiles = [(x[0], x[2], x[1]) for x in samples]
    elif name.startswith("tile_pprprp"):
        tiles = [pprprp_tiles(strategy, x) for x in samples]
    else:
        raise ValueError(f"no CPU restatement of strategy {name} (sample names {names})")
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(lambda t: schedule_lib(*t), tiles))
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    if bf16:
        from xtc_amd.utils.bf16 import round_to_bf16

        a, b = round_to_bf16(a), round_to_bf16(b)
    return sorted((time_schedule(t, a, b, repeat=1, min_repeat_ms=20), t) for t in tiles)


def autoschedule_matmul(a: np.ndarray, b: np.ndarray, repeat: int = 2, min_repeat_ms: int = 50) -> tuple[int, float]:
    """Times every tile variant; returns (best variant, its seconds per call)."""
    results = [(time_matmul(a, b, v, repeat, min_repeat_ms), v) for v in range(len(variants()))]
    t, v = min(results)
    return v, t
