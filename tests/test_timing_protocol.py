# SPDX-License-Identifier: BSD-3-Clause
"""The evaluate_perf timing protocol of libxtc_hip, pinned on the CPU.

xtc_hip_evaluate_perf restates src/xtc/csrcs/runtimes/host/evaluate_perf.c:
63-125: one warm-up call when number > 0; per repeat, batches of `number`
calls doubling until a batch lasts min_repeat_ms; the result is the last
batch's time (or counter delta) divided by its calls.  A stub payload that
counts its calls and sleeps a fixed time makes the call sequence
deterministic, so the checks below follow from that rule alone, and the same
stub is run through the reference's own evaluate_perf (built from its C
sources into oracle/_ref) to compare call counts, per-call means and the
host-counter results side by side.  No GPU is involved: without "gpu.*"
events the harness never touches the device.
"""

from __future__ import annotations

import ctypes
import time

import pytest

from oracle import cpu_baseline
from xtc_amd.runtimes.hip import capi

CALLBACK = ctypes.CFUNCTYPE(None)
SLEEP_S = 0.010


def _stub(sleep_s=SLEEP_S, spin=False):
    calls = []

    def f():
        calls.append(time.perf_counter())
        if spin:
            end = time.perf_counter() + sleep_s
            while time.perf_counter() < end:
                pass
        else:
            time.sleep(sleep_s)

    return CALLBACK(f), calls


def _ours(events, repeat, number, min_repeat_ms, fn):
    L = capi.lib()
    n = len(events)
    res = (ctypes.c_double * (repeat * max(1, n)))()
    names = (ctypes.c_char_p * max(1, n))(*[e.encode() for e in events])
    args = (ctypes.c_void_p * 1)()
    L.xtc_hip_evaluate_perf(res, n, names, repeat, number, min_repeat_ms, ctypes.cast(fn, ctypes.c_void_p), args, 0)
    assert L.xtc_hip_evaluate_status() == 0, capi.last_error()
    return list(res)


def _reference(events, repeat, number, min_repeat_ms, fn):
    ref = cpu_baseline.ref_runtime()
    n = len(events)
    res = (ctypes.c_double * (repeat * max(1, n)))()
    names = (ctypes.c_char_p * max(1, n))(*[e.encode() for e in events])
    args = (ctypes.c_void_p * 1)()
    ref.evaluate_perf(res, n, names, repeat, number, min_repeat_ms, ctypes.cast(fn, ctypes.c_void_p), args, 0)
    return list(res)


def _expected_calls(repeat, number, min_repeat_ms, per_call_s):
    """Calls the protocol makes when every call lasts per_call_s."""
    total = 1 if number > 0 else 0
    number = max(number, 1)
    for _ in range(repeat):
        attempts = number
        while True:
            total += attempts
            if attempts * per_call_s * 1000 >= min_repeat_ms:
                break
            attempts *= 2
    return total


def _harnesses():
    out = [("xtc_hip", _ours)]
    if cpu_baseline.ref_runtime() is not None:
        out.append(("reference", _reference))
    return out


# (repeat, number, min_repeat_ms): with calls of 10 ms every doubling step
# stays on its side of the threshold unless a call overshoots by 66 %, so the
# call count is deterministic
PROTOCOL_CASES = [(3, 1, 35), (2, 3, 50), (2, 0, 35), (4, 5, 0), (1, 2, 0)]


@pytest.mark.parametrize("repeat,number,min_ms", PROTOCOL_CASES)
def test_call_counts_and_per_call_means(repeat, number, min_ms):
    expect = _expected_calls(repeat, number, min_ms, SLEEP_S)
    counts = {}
    for name, run in _harnesses():
        fn, calls = _stub()
        res = run([], repeat, number, min_ms, fn)
        counts[name] = len(calls)
        assert len(calls) == expect, (name, len(calls), expect)
        assert len(res) == repeat
        for v in res:
            # the per-call mean of one batch, not its total or a count
            assert SLEEP_S <= v < SLEEP_S * 1.66, (name, v)
    assert len(set(counts.values())) == 1, counts


def test_batches_double_until_min_repeat_ms():
    # one warm-up call, then batches of 1, 2 and 4 calls (40 ms >= 35 ms)
    for name, run in _harnesses():
        fn, calls = _stub()
        run([], 1, 1, 35, fn)
        assert len(calls) == 1 + 1 + 2 + 4, name


def test_host_counters_match_the_reference():
    # busy-waiting stub: the software CPU clock counts ~SLEEP_S of user time
    # per call; names the kernel refuses (no hardware PMU in a VM) or that are
    # unknown read -1 in both harnesses
    events = ["clocks", "context_switches", "instructions", "cycles", "no_such_event"]
    results = {}
    for name, run in _harnesses():
        fn, _ = _stub(spin=True)
        results[name] = run(events, 2, 1, 20, fn)
    ours = results["xtc_hip"]
    assert ours[4] == -1 and ours[9] == -1
    for r in range(2):
        clocks = ours[r * len(events)]
        assert clocks == -1 or 0.5 * SLEEP_S * 1e9 <= clocks <= 2.0 * SLEEP_S * 1e9, clocks
    if "reference" in results:
        ref = results["reference"]
        for e in range(len(events)):
            for r in range(2):
                a, b = ours[r * len(events) + e], ref[r * len(events) + e]
                assert (a == -1) == (b == -1), (events[e], a, b)
        # same counter, same stub: per-call CPU clock agrees within 50 %
        if ours[0] != -1:
            assert 0.5 <= ours[0] / ref[0] <= 2.0


def test_invalid_arguments_set_the_status():
    L = capi.lib()
    fn, calls = _stub()
    res = (ctypes.c_double * 4)()
    args = (ctypes.c_void_p * 1)()
    L.xtc_hip_evaluate_perf(res, 0, None, 0, 1, 0, ctypes.cast(fn, ctypes.c_void_p), args, 0)
    assert L.xtc_hip_evaluate_status() != 0 and "invalid arguments" in capi.last_error()
    names = (ctypes.c_char_p * 65)(*([b"clocks"] * 65))
    L.xtc_hip_evaluate_perf(res, 65, names, 1, 1, 0, ctypes.cast(fn, ctypes.c_void_p), args, 0)
    assert L.xtc_hip_evaluate_status() != 0 and "at most 64" in capi.last_error()
    assert not calls
    # a valid call afterwards clears both the status and the message
    L.xtc_hip_evaluate_perf(res, 0, None, 1, 1, 0, ctypes.cast(fn, ctypes.c_void_p), args, 0)
    assert L.xtc_hip_evaluate_status() == 0 and capi.last_error() == "" and len(calls) == 2
