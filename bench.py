#!/usr/bin/env python3
# SPDX-License-Identifier: BSD-3-Clause
"""Headline benchmark: bf16-input / fp32-accumulate matmul M=N=K=8192 on one
MI355X, driven through the XTC pipeline (graph -> HipBackend -> Scheduler ->
Compiler -> payload), TFLOP/s and fraction of the dense bf16 MFMA peak.

A step is one call of the compiled payload over the resident inputs (one
GEMM launch).  Inputs are seeded uniform[-1,1) rounded to bf16 and are in HBM
before the timed region.  The K timed calls are queued back to back and
bracketed by HIP events on the payload's stream plus a wall clock with a
synchronisation on both sides.

Other configurations (--config C1|C2|C3b|C4|C5) print the same line for
their own workload; the driver runs the default.  --gpus N>1 is refused:
every box of this pool has one GPU.

The cpu_baseline leg times the C restatement of XTC's llvmir CPU backend
(oracle/, OpenMP on this host's cores): auto-scheduled over 64 seeded samples
each of the reference's tile_pprprp_vr and tile_oo strategies, then the best
schedule timed at the workload's GEMM shape with repeat 5 and min_repeat_ms
100, with the reference's own evaluate_perf harness when oracle/_ref is
built.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_TFLOPS = {"bfloat16": 2516.6, "float32": 157.3}  # dense MFMA, MI355X datasheet
PEAK_HBM_GBS = 8000.0


from xtc_amd import configs as workloads  # noqa: E402  (graphs, seeded inputs, tuned schedules)


def _traffic(cfg: str) -> float | None:
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    path = ROOT / "profiles" / f"traffic_{cfg}.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def _warm(step, synchronize, warmup: int, warmup_ms: float) -> dict:
    """`warmup` untimed steps, then more until `warmup_ms` of wall time has
    passed since the first: the GPU's clocks ramp up over the first tens of
    milliseconds of work (a cold C5 step runs 10 % slower), and the timed
    steps measure the steady state.  Returns what ran."""
    t0 = time.perf_counter()
    n = 0
    while n < warmup or (time.perf_counter() - t0) * 1e3 < warmup_ms:
        step()
        n += 1
        if n % 64 == 0 or n == warmup:
            synchronize()  # the wall clock above measures work done, not work queued
    synchronize()
    return {"steps": n, "ms": round((time.perf_counter() - t0) * 1e3, 1)}


def _vendor_matmul(host_in: list[np.ndarray], dtype: str, steps: int, warmup: int, warmup_ms: float) -> dict:
    """Times torch.matmul (hipBLASLt on this image) on the same inputs as a
    reference point for the vendor library, after the same warm-up as the
    bench's own steps; bf16 inputs give a bf16 output there (half the output
    bytes of the fp32 output measured here)."""
    import torch

    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float32
    a = torch.from_numpy(host_in[0]).to("cuda:0").to(tdt).contiguous()
    b = torch.from_numpy(host_in[1]).to("cuda:0").to(tdt).contiguous()
    _warm(lambda: torch.matmul(a, b), torch.cuda.synchronize, warmup, warmup_ms)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        torch.matmul(a, b)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    m, k = host_in[0].shape
    n = host_in[1].shape[1]
    return {"library": "torch.matmul (hipBLASLt)", "out_dtype": str(tdt).split(".")[1], "kernel_ms": round(ms, 4),
            "tflops": round(2 * m * n * k / ms / 1e9, 1)}


def _vendor_conv(host_in: list[np.ndarray], steps: int, warmup: int, warmup_ms: float) -> dict:
    """Times torch's conv2d (MIOpen on this image) on the C4 inputs, NHWC
    (channels_last) fp32 with a 1-pixel zero pad and relu, as a reference
    point for the vendor library after the same warm-up as the bench's own
    steps.  MIOpen picks its own algorithm (its numerics are not checked
    here)."""
    import torch

    x = torch.from_numpy(host_in[0]).to("cuda:0").permute(0, 3, 1, 2).contiguous(memory_format=torch.channels_last)
    w = torch.from_numpy(host_in[1]).to("cuda:0").permute(3, 2, 0, 1).contiguous(memory_format=torch.channels_last)

    def step() -> None:
        torch.relu_(torch.nn.functional.conv2d(x, w, padding=1))

    _warm(step, torch.cuda.synchronize, warmup, warmup_ms)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flop = workloads.flops("C4")
    return {"library": "torch.nn.functional.conv2d + relu_ (MIOpen), channels_last fp32", "kernel_ms": round(ms, 4),
            "tflops": round(flop / ms / 1e9, 1)}


def _cpu_baseline(cfg: str) -> dict:
    """Times the CPU restatement of XTC's llvmir backend (oracle/) on this
    host, auto-scheduled as loop-explore would: 64 seeded samples each of the
    reference's tile_pprprp_vr and tile_oo strategies (every sample compiled
    as its own object) plus the restatement's 8 fixed tile_oo variants, timed
    at 1024^3; the 8 fastest re-timed on the workload's N x K with 32 rows
    per thread; the winner then timed at the
    workload's own GEMM shape (C1, C2, C3a, C3b; a 512/2048 sample of it for
    the conv and MLP workloads) under the reference's evaluate_perf protocol
    with repeat 5 and min_repeat_ms 100 (evaluate_perf.c:63-125): min and
    median per call over the repeats."""
    from oracle import cpu_baseline as cb
    from xtc_amd.utils.bf16 import round_to_bf16

    bf16 = cfg.startswith("C3")
    rng = np.random.default_rng(0)

    def draw(shape: tuple[int, int]) -> np.ndarray:
        x = rng.uniform(-1, 1, shape).astype(np.float32)
        return round_to_bf16(x) if bf16 else x

    cores = cb.threads()
    jobs = min(16, cores)
    tune, trials = 1024, 64
    cands: list[tuple[float, tuple[int, ...], str]] = []
    for strat in ("tile_pprprp_vr", "tile_oo"):
        cands += [(t, s, strat) for t, s in cb.autoschedule_strategy(strat, tune, trials=trials, seed=0, bf16=bf16,
                                                                      jobs=jobs)]
    at, bt = draw((tune, tune)), draw((tune, tune))
    for v, (ti, tk, tj) in enumerate(cb.variants()):
        cands.append((cb.time_schedule((ti, tk, tj), at, bt, repeat=1, min_repeat_ms=20), (ti, tk, tj), "tile_oo fixed"))
    cands.sort()
    shape = {"C1": (512, 512, 512), "C2": (4096, 4096, 4096), "C3a": (8192, 8192, 8192),
             "C3b": (16, 8192, 8192)}.get(cfg, (2048, 2048, 2048) if cfg == "C5" else (512, 512, 512))
    m, n, k = shape

    def fits(s: tuple[int, ...]) -> bool:  # a pprprp schedule's i1/j1 extents must divide the shape
        return len(s) == 3 or (m % s[0] == 0 and n % s[3] == 0)

    # re-rank the 8 fastest on the workload's own N x K with fewer rows (32 per
    # thread): the panel traffic of a deep K is what a 1024^3 sample misses
    ms = min(m, 32 * cores)
    a2, b2 = draw((ms, k)), draw((k, n))
    finalists = sorted((cb.time_schedule(s, a2, b2, repeat=1, min_repeat_ms=50), s, how)
                       for _, s, how in [c for c in cands if fits(c[1]) and ms % c[1][0] == 0][:8])
    _, sched, strat = finalists[0]
    a, b = draw((m, k)), draw((k, n))
    repeat, min_repeat_ms = 5, 100
    times = cb.time_schedule_repeats(sched, a, b, repeat=repeat, number=1, min_repeat_ms=min_repeat_ms)
    t_min, t_med = min(times), statistics.median(times)
    names = ("i1", "i2", "i3", "j1", "j2", "j3", "k1") if len(sched) == 7 else ("i1", "k1", "j1")
    how = (f"{strat} schedule {dict(zip(names, sched))}: fastest at {ms}x{n}x{k} of the 8 best at {tune}^3 among "
           f"{trials} seeded tile_pprprp_vr samples, {trials} seeded tile_oo samples and 8 fixed tile_oo variants")
    harness = "reference evaluate_perf" if cb.ref_runtime() is not None else "evaluate_perf protocol (Python)"
    value = 2 * m * n * k / t_min / 1e12
    # the host's peak as the reference's explorer takes it: evaluate_flops's
    # single-core FMA/s (evaluate_flops.c:461-494) times the cores
    # (explore.py:619-625 divides the peak time by the threads)
    fma = cb.ref_peak_flops("float32")
    peak = {"peak_tflops": round(2 * fma * cores / 1e12, 3), "frac_of_peak": round(value / (2 * fma * cores / 1e12), 4),
            "peak_source": "reference evaluate_flops (float32) single-core FMA/s x cores"} if fma else {}
    return {
        "value": round(value, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "repeat": repeat,
        "min_repeat_ms": min_repeat_ms,
        "min_ms": round(t_min * 1e3, 3),
        "median_ms": round(t_med * 1e3, 3),
        "median_tflops": round(2 * m * n * k / t_med / 1e12, 4),
        **peak,
        "sample": (
            f"fp32 matmul {m}x{n}x{k} ({'the workload shape' if cfg in ('C1', 'C2', 'C3a', 'C3b') else 'a sample'}"
            f"{', bf16-rounded inputs' if bf16 else ''}), XTC llvmir restatement, {how}; value from the min of "
            f"{repeat} repeats (min_repeat_ms {min_repeat_ms}); OpenMP {cores} threads, {harness}, CPU: {cb.cpu_model()}"
        ),
    }


def _xtc_protocol(cfg: str, backend, sch, dev, cargs, flops: int, dtype: str) -> dict:  # type: ignore[no-untyped-def]
    """The bench's schedule under XTC's own timing protocol
    (evaluate_perf.c:92-120): per repeat, synchronous payload calls doubled
    until min_repeat_ms, time per call, min and median over repeats; device
    time from HIP events and host wall clock.  The protocol measures host
    time, so it takes the synchronising payload (the default compile)."""
    module = backend.get_compiler(schedule_policy="strict").compile(sch.schedule())
    dev.load_module(module)
    fn = dev.get_module_function(module, module.payload_name)
    fn.restype = None
    status = dev.module_symbol(module, f"{module.payload_name}_status")
    status.restype = ctypes.c_int
    proto: dict = {"repeat": 5, "number": 1, "min_repeat_ms": 100}
    for label, events in (("device", ["gpu.time"]), ("wall", [])):
        vals = dev.evaluate_perf(events, 5, 1, 100, fn, cargs, len(cargs))
        proto[f"{label}_min_ms"] = round(min(vals) * 1e3, 4)
        proto[f"{label}_median_ms"] = round(statistics.median(vals) * 1e3, 4)
    if status():
        raise SystemExit("payload reported an error under the evaluate_perf protocol")
    rate = (workloads.alg_bytes(cfg) / (proto["device_min_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBS if cfg == "C3b"
            else flops / (proto["device_min_ms"] * 1e-3) / 1e12 / PEAK_TFLOPS[dtype])
    proto["device_min_pct_of_peak"] = round(100 * rate, 2)
    return proto


def _print_peaks() -> int:
    """The measured MFMA peaks behind xtc_hip_evaluate_flops, as JSON lines."""
    from xtc_amd.runtimes.hip.device import HipDevice

    dev = HipDevice(0)
    for dtype in ("float32", "bfloat16"):
        for op in ("reference", "zero", "random"):
            tf = 2 * dev.evaluate_flops(dtype, op) / 1e12
            print(json.dumps({"mfma_peak": dtype, "operands": op, "tflops": round(tf, 1),
                              "frac_of_datasheet": round(tf / PEAK_TFLOPS[dtype], 4)}), flush=True)
    return 0


def _elementwise(steps: int) -> int:
    """HBM rate of the elementwise kernels, one JSON line each: relu, pad,
    unpad, the bf16 casts (library entry points) and the transpose that stages a
    transposed matmul operand (timed inside a trans_a matmul with N = 16, so
    its rate is read from the kernel trace: the line's time includes the
    generic GEMM that consumes the copy).  Bytes are algorithmic: every input
    element read once, every output element written once."""
    import numpy as np

    from xtc_amd.runtimes.hip import capi
    from xtc_amd.runtimes.hip.buffer import DeviceBuffer, ensure_device

    ensure_device(0)
    L = capi.lib()
    e0, e1 = L.xtc_hip_event_create(), L.xtc_hip_event_create()

    def timed(name: str, nbytes: int, launch) -> None:  # type: ignore[no-untyped-def]
        for _ in range(3):
            launch()
        capi.check(L.xtc_hip_event_record(e0, None), "event")
        for _ in range(steps):
            launch()
        capi.check(L.xtc_hip_event_record(e1, None), "event")
        ms = ctypes.c_float()
        capi.check(L.xtc_hip_event_elapsed_ms(e0, e1, ctypes.byref(ms)), "elapsed")
        us = ms.value * 1e3 / steps
        print(json.dumps({"kernel": name, "bytes": nbytes, "us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1),
                          "frac_of_hbm": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4)}), flush=True)

    n = 1 << 26  # 256 MiB of fp32
    x = DeviceBuffer(n * 4)
    y = DeviceBuffer(n * 4)
    h = DeviceBuffer(n * 2)
    x.zero()
    h.zero()
    xp, yp, hp = ctypes.c_void_p(x.ptr), ctypes.c_void_p(y.ptr), ctypes.c_void_p(h.ptr)
    timed("relu_kernel fp32 2^26", 8 * n, lambda: capi.check(L.xtc_hip_relu(xp, yp, n, 0.0, None), "relu"))
    timed("cast_f32_bf16_kernel 2^26", 6 * n, lambda: capi.check(L.xtc_hip_cast_f32_to_bf16(xp, hp, n, None), "cast"))
    timed("cast_bf16_f32_kernel 2^26", 6 * n, lambda: capi.check(L.xtc_hip_cast_bf16_to_f32(hp, yp, n, None), "cast"))
    for shape, pads in (((64, 112, 112, 64), ((0, 0), (1, 1), (1, 1), (0, 0))),
                        ((8, 56, 56, 64), ((0, 0), (0, 0), (0, 0), (1, 3)))):
        nd = len(shape)
        sh = (ctypes.c_int64 * nd)(*shape)
        be = (ctypes.c_int64 * nd)(*[p[0] for p in pads])
        af = (ctypes.c_int64 * nd)(*[p[1] for p in pads])
        out_elems = int(np.prod([d + p[0] + p[1] for d, p in zip(shape, pads)]))
        nbytes = 4 * (int(np.prod(shape)) + out_elems)
        timed(f"pad_kernel {'x'.join(map(str, shape))} pads {[list(p) for p in pads]}", nbytes,
              lambda sh=sh, be=be, af=af: capi.check(L.xtc_hip_pad(xp, yp, nd, sh, be, af, 0.0, None), "pad"))
    # unpad: the crop after a padded matmul or conv reads and writes each kept element once
    for shape, crops in (((64, 114, 114, 64), ((0, 0), (1, 1), (1, 1), (0, 0))),
                         ((8, 56, 56, 68), ((0, 0), (0, 0), (0, 0), (1, 3)))):
        nd = len(shape)
        sh = (ctypes.c_int64 * nd)(*shape)
        be = (ctypes.c_int64 * nd)(*[c[0] for c in crops])
        af = (ctypes.c_int64 * nd)(*[c[1] for c in crops])
        kept = int(np.prod([d - c[0] - c[1] for d, c in zip(shape, crops)]))
        timed(f"unpad_kernel {'x'.join(map(str, shape))} crops {[list(c) for c in crops]}", 8 * kept,
              lambda sh=sh, be=be, af=af: capi.check(L.xtc_hip_unpad(xp, yp, 4, nd, sh, be, af, None), "unpad"))
    # transposed A: the library stages A^T [K][M] into A [M][K] with transpose_kernel
    for dtype, esz in (("float32", 4), ("bfloat16", 2)):
        d = capi.MatmulDesc(dtype=capi.XTC_HIP_F32 if dtype == "float32" else capi.XTC_HIP_BF16, M=8192, N=16,
                            K=8192, trans_a=1, xcd_remap=1)
        timed(f"matmul trans_a {dtype} 8192x16x8192 (transposed copy + generic GEMM)", 2 * esz * 8192 * 8192,
              lambda d=d: capi.check(L.xtc_hip_matmul(ctypes.byref(d), xp, yp, hp, None), "matmul"))
    capi.check(L.xtc_hip_synchronize(), "synchronize")
    return 0


def _named_ops(steps: int, warmup_ms: float, dtype: str = "float32") -> int:
    """Every named operation of `loop-explore --op-name` (the reference's
    layer registry, src/xtc/artifacts) with the backend's default schedule,
    one JSON line each: kernel time per payload call over `steps`
    back-to-back calls at steady clocks (HIP events, seeded uniform inputs),
    TFLOP/s, and the fraction of the op's roofline max(FLOP / MFMA peak of
    `dtype`, algorithmic bytes / 8 TB/s), algorithmic bytes being every
    input read once and the output written once (bf16 inputs, fp32
    output).  A last line summarises."""
    import numpy as np

    from xtc_amd.artifacts import list_operations
    from xtc_amd.backends.hip import Backend
    from xtc_amd.cli.explore import _operation_dims, build_graph
    from xtc_amd.runtimes.hip import capi
    from xtc_amd.runtimes.hip.device import HipDevice
    from xtc_amd.runtimes.hip.ndarray import DeviceArray

    dev = HipDevice(0)
    dev.init_device()
    L = capi.lib()
    e0, e1 = L.xtc_hip_event_create(), L.xtc_hip_event_create()
    fracs = []
    for idx, (op, name) in enumerate(list_operations()):
        dims = _operation_dims(op, name)
        graph = build_graph(op, dims, dtype, name=name.lower())
        backend = Backend(graph)
        module = backend.get_compiler(synchronize=False, schedule_policy="strict").compile(
            backend.get_scheduler().schedule())
        dev.load_module(module)
        fn = dev.get_module_function(module, module.payload_name)
        fn.restype = None
        status = dev.module_symbol(module, f"{module.payload_name}_status")
        status.restype = ctypes.c_int
        rng = np.random.default_rng(idx)
        d_in = [DeviceArray.from_numpy(rng.uniform(-1, 1, t.constant_shape).astype(np.float32), t.constant_dtype, dev)
                for t in graph.inputs_types]
        d_out = [DeviceArray(t.constant_shape, t.constant_dtype, dev) for t in graph.outputs_types]
        cargs = [ctypes.c_void_p(d.data) for d in (*d_in, *d_out)]
        _warm(lambda: fn(*cargs), lambda: capi.check(L.xtc_hip_synchronize(), "synchronize"), 3, warmup_ms)
        capi.check(L.xtc_hip_event_record(e0, None), "event")
        for _ in range(steps):
            fn(*cargs)
        capi.check(L.xtc_hip_event_record(e1, None), "event")
        capi.check(L.xtc_hip_synchronize(), "synchronize")
        if status():
            raise SystemExit(f"{name}: payload reported an error")
        ms = ctypes.c_float()
        capi.check(L.xtc_hip_event_elapsed_ms(e0, e1, ctypes.byref(ms)), "elapsed")
        us = ms.value * 1e3 / steps
        flops = 2 * int(np.prod(dims[:7] if op == "conv2d" else dims))
        nbytes = sum(d.nbytes for d in (*d_in, *d_out))
        t_mfma, t_hbm = flops / (PEAK_TFLOPS[dtype] * 1e12), nbytes / (PEAK_HBM_GBS * 1e9)
        roof_us = max(t_mfma, t_hbm) * 1e6
        fracs.append(roof_us / us)
        print(json.dumps({"named_op": name, "operator": op, "dtype": dtype, "dims": dims, "us": round(us, 2),
                          "tflops": round(flops / us / 1e6, 2), "roofline_us": round(roof_us, 2),
                          "bound": "mfma" if t_mfma >= t_hbm else "hbm", "frac_of_roofline": round(roof_us / us, 4),
                          "kernel": "; ".join(f"{n}: {c.describe()}" for n, c in module.configs.items())}),
              flush=True)
        for d in (*d_in, *d_out):
            d.free()
        dev.unload_module(module)
    geo = float(np.exp(np.mean(np.log(fracs))))
    print(json.dumps({"named_ops": len(fracs), "geomean_frac_of_roofline": round(geo, 4),
                      "min_frac_of_roofline": round(min(fracs), 4), "max_frac_of_roofline": round(max(fracs), 4)}),
          flush=True)
    return 0


COPY_BYTES = 1 << 30


def _calibrate_copy(steps: int) -> int:
    """Streams COPY_BYTES through the library's elementwise kernel
    (relu_kernel, y = max(x, 0) over 2^28 fp32: exactly COPY_BYTES read and
    COPY_BYTES written per launch).  Under rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE its per-dispatch KiB give the factor that turns those counters
    into bytes for the GEMM dispatches."""
    from xtc_amd.runtimes.hip import capi
    from xtc_amd.runtimes.hip.device import HipDevice
    from xtc_amd.runtimes.hip.ndarray import DeviceArray

    dev = HipDevice(0)
    dev.init_device()
    n = COPY_BYTES // 4
    x = DeviceArray((n,), "float32", dev)
    y = DeviceArray((n,), "float32", dev)
    x.fill_zero()
    L = capi.lib()
    for _ in range(steps):
        capi.check(L.xtc_hip_relu(ctypes.c_void_p(x.data), ctypes.c_void_p(y.data), n, 0.0, None), "relu")
    capi.check(L.xtc_hip_synchronize(), "synchronize")
    print(json.dumps({"calibration": "relu_kernel copy", "bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES,
                      "launches": steps}), flush=True)
    x.free()
    y.free()
    return 0


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--warmup-ms", type=float, default=300.0,
                    help="after the --warmup steps, keep stepping (untimed) until this much wall time has passed, "
                         "so that the timed steps run at steady clocks (0: --warmup steps only)")
    ap.add_argument("--config", default="C3a", choices=["C1", "C2", "C3a", "C3b", "C4", "C5"])
    ap.add_argument("--no-protocol", action="store_true",
                    help="skip the evaluate_perf protocol pass (kernel traces then hold only the timed steps)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--no-ceiling", action="store_true", help="skip the measured MFMA ceiling")
    ap.add_argument("--elementwise", action="store_true",
                    help="only time the elementwise kernels (relu, pad, bf16 casts, transpose) in GB/s")
    ap.add_argument("--peak", action="store_true",
                    help="only print the measured MFMA peaks (fp32, bf16; zero, random and the reference's operands)")
    ap.add_argument("--vs-hipblaslt", action="store_true",
                    help="also time the vendor library on the same inputs and report it in config: torch.matmul "
                         "(hipBLASLt) for the matmul configs, torch's conv2d (MIOpen) for C4")
    ap.add_argument("--named-ops", action="store_true",
                    help="time every named operation of loop-explore --op-name with its default schedule")
    ap.add_argument("--named-dtype", default="float32", choices=["float32", "bfloat16"],
                    help="operand type of --named-ops (bfloat16: fp32 accumulation and output)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="launch only the 1 GiB copy kernel used to scale rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args(argv)
    if args.calibrate_copy:
        return _calibrate_copy(args.steps)
    if args.peak:
        return _print_peaks()
    if args.elementwise:
        return _elementwise(args.steps)
    if args.named_ops:
        return _named_ops(args.steps, args.warmup_ms, args.named_dtype)
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this build measures one GPU; a GEMM "
            "shards over GPUs by rows of A and C with B replicated, so one GPU's share is the "
            "same kernel at M / N_gpus rows.",
            file=sys.stderr,
        )
        return 2

    from xtc_amd.backends.hip import Backend
    from xtc_amd.runtimes.hip import capi
    from xtc_amd.runtimes.hip.device import HipDevice
    from xtc_amd.runtimes.hip.ndarray import DeviceArray

    cfg = args.config
    graph = workloads.graph(cfg)
    backend = Backend(graph)
    sch = workloads.apply_schedule(backend.get_scheduler(), cfg)
    module = backend.get_compiler(synchronize=False, schedule_policy="strict").compile(sch.schedule())

    dev = HipDevice(0)
    dev.init_device()
    dev.load_module(module)
    fn = dev.get_module_function(module, module.payload_name)
    fn.restype = None
    status = dev.module_symbol(module, f"{module.payload_name}_status")
    status.restype = ctypes.c_int

    host_in = workloads.inputs(cfg, graph)
    d_in = [DeviceArray.from_numpy(a, t.constant_dtype, dev) for a, t in zip(host_in, graph.inputs_types)]
    d_out = [DeviceArray(t.constant_shape, t.constant_dtype, dev) for t in graph.outputs_types]
    cargs = [ctypes.c_void_p(d.data) for d in (*d_in, *d_out)]

    def step() -> None:
        fn(*cargs)

    L = capi.lib()
    # parity spot check of the bench's own output (rows 0..7) in float64
    step()
    capi.check(L.xtc_hip_synchronize(), "synchronize")
    if status():
        raise SystemExit(f"payload failed: {dev.module_symbol(module, f'{module.payload_name}_message')()}")
    spot_err = None
    if cfg in ("C3a", "C3b", "C1", "C2"):
        out = d_out[0].numpy()
        a64, b64 = host_in[0][:8].astype(np.float64), host_in[1].astype(np.float64)
        ref = a64 @ b64
        k = host_in[0].shape[1]
        spot_err = float(np.abs(out[:8] - ref).max() / (np.sqrt(k) * np.abs(host_in[0]).max() * np.abs(host_in[1]).max()))
        tol = 1e-2 if cfg.startswith("C3") else 1e-4
        if not spot_err <= tol:
            raise SystemExit(f"parity spot check failed: scaled error {spot_err} > {tol}")
    elif cfg == "C4":
        # first image, first 8 output rows: relu(conv3x3(pad1(x)))
        x, w = host_in[0][0].astype(np.float64), host_in[1].astype(np.float64)
        xp = np.pad(x, ((1, 1), (1, 1), (0, 0)))
        ref = np.zeros((8, 56, 64))
        for r in range(3):
            for s in range(3):
                ref += np.einsum("hwc,cf->hwf", xp[r:r + 8, s:s + 56], w[r, s])
        ref = np.maximum(ref, 0.0)
        out = d_out[0].numpy()[0, :8]
        spot_err = float(np.abs(out - ref).max() / (np.sqrt(576) * np.abs(xp).max() * np.abs(w).max()))
        if not spot_err <= 1e-4:
            raise SystemExit(f"parity spot check failed: scaled error {spot_err} > 1e-4")
    elif cfg == "C5":
        # first 8 rows: relu(X W1) W2, the error scaled on the second GEMM
        x, w1, w2 = (a.astype(np.float64) for a in host_in[:3])
        h = np.maximum(x[:8] @ w1, 0.0)
        ref = h @ w2
        out = d_out[0].numpy()[:8]
        spot_err = float(np.abs(out - ref).max() / (np.sqrt(w2.shape[0]) * np.abs(h).max() * np.abs(w2).max()))
        if not spot_err <= 1e-4:
            raise SystemExit(f"parity spot check failed: scaled error {spot_err} > 1e-4")

    print(f"[bench] {cfg}: {args.warmup} warmup (at least {args.warmup_ms:g} ms) + {args.steps} timed steps",
          file=sys.stderr, flush=True)
    warmed = _warm(step, lambda: capi.check(L.xtc_hip_synchronize(), "synchronize"), args.warmup, args.warmup_ms)
    e0, e1 = L.xtc_hip_event_create(), L.xtc_hip_event_create()
    capi.check(L.xtc_hip_event_record(e0, None), "event")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    capi.check(L.xtc_hip_event_record(e1, None), "event")
    capi.check(L.xtc_hip_synchronize(), "synchronize")
    wall = time.perf_counter() - t0
    ms = ctypes.c_float()
    capi.check(L.xtc_hip_event_elapsed_ms(e0, e1, ctypes.byref(ms)), "elapsed")
    if status():
        raise SystemExit("payload reported an error during the timed region")
    kernel_s = ms.value * 1e-3 / args.steps
    step_s = wall / args.steps
    flops = workloads.flops(cfg)
    dtype = graph.inputs_types[0].constant_dtype
    kernels = "; ".join(f"{n}: {c.describe()}" for n, c in module.configs.items()) or None
    if cfg == "C3b":
        achieved = workloads.alg_bytes(cfg) / kernel_s / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    else:
        achieved = flops / kernel_s / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_TFLOPS[dtype], "unit": "TFLOP/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"] = _traffic(cfg)
    line = {
        "metric": "TFLOP/s + % of MFMA peak, matmul/conv2d on 1 MI355X vs MLIR-CPU baseline",
        "value": round(flops / step_s / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"bfloat16": "bf16 in, fp32 acc/out", "float32": "fp32"}[dtype],
        "data": "synthetic: seeded uniform/normal inputs of the BASELINE config",
        "config": {
            "workload": cfg,
            "graph": str(graph.name),
            "flop_per_step": flops,
            "kernel": kernels,
            "kernel_ms": round(kernel_s * 1e3, 4),
            "pct_of_peak": round(100 * roof["frac"], 2),
            "parity_spot_scaled_err": spot_err,
            "warmup_run": warmed,
        },
        "roofline": roof,
    }
    # the same schedule under XTC's own timing protocol (evaluate_perf.c:92-120):
    # per repeat, synchronous payload calls doubled until min_repeat_ms, time
    # per call, min and median over repeats; device time from HIP events and
    # host wall clock.  The protocol needs the synchronising payload (the
    # default compile): its loop measures host time.
    if not args.no_protocol:
        print(f"[bench] {cfg}: evaluate_perf protocol", file=sys.stderr, flush=True)
        line["config"]["xtc_protocol"] = _xtc_protocol(cfg, backend, sch, dev, cargs, flops, dtype)
    if not args.no_ceiling and cfg != "C3b":
        # the measured MFMA ceiling (register-only MFMA loop, xtc_hip_evaluate_flops):
        # on random operands the board's power limit holds it below the datasheet
        print(f"[bench] {cfg}: measured MFMA ceiling", file=sys.stderr, flush=True)
        ceil = {op: 2 * dev.evaluate_flops(dtype, op) / 1e12 for op in ("zero", "random")}
        line["config"]["mfma_ceiling"] = {
            "probe": "register-only MFMA loop, xtc_hip_evaluate_flops_operands",
            "zero_tflops": round(ceil["zero"], 1),
            "random_tflops": round(ceil["random"], 1),
            "kernel_frac_of_random_ceiling": round(roof["achieved"] / ceil["random"], 4),
        }
    if args.vs_hipblaslt and cfg in ("C1", "C2", "C3a", "C3b"):
        line["config"]["vendor"] = _vendor_matmul(host_in, dtype, args.steps, args.warmup, args.warmup_ms)
    if args.vs_hipblaslt and cfg == "C4":
        line["config"]["vendor"] = _vendor_conv(host_in, args.steps, args.warmup, args.warmup_ms)
    if not args.no_cpu:
        print(f"[bench] {cfg}: cpu baseline", file=sys.stderr, flush=True)
        try:
            line["cpu_baseline"] = _cpu_baseline(cfg)
        except Exception as err:  # the GPU figure stands without it
            line["cpu_baseline"] = {"value": None, "error": str(err)}
    print(json.dumps(line), flush=True)
    for d in (*d_in, *d_out):
        d.free()
    dev.unload_module(module)
    return 0


if __name__ == "__main__":
    sys.exit(main())
