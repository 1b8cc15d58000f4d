# SPDX-License-Identifier: BSD-3-Clause
"""GPU hardware counters for `pmu_counters=["gpu.<name>", ...]`.

The evaluators accept, like the reference's (GPUEvaluator with CUPTI,
src/xtc/csrcs/runtimes/accelerator/gpu/perf_event_gpu.cpp:56-233):
  * "gpu.time" / "gpu.clocks": device time per call (HIP events, always on);
  * "gpu.cycles": GPU busy cycles (GRBM_GUI_ACTIVE);
  * "gpu.<counter>": any rocprofiler-sdk counter of the device (SQ_WAVES,
    FETCH_SIZE, ...), summed over the kernels of one call.
The last two need libxtc_hip_pmu.so's counter tool, which rocprofiler-sdk
accepts only before the ROCm runtime starts: call `enable()` before the
first GPU call of the process, or set XTC_HIP_PMU=1 (capi.lib() then
enables it when it loads the library).  While counters are collected every
dispatch is profiled and serialised, so times measured together with them
are perturbed, as under CUPTI.
"""

from __future__ import annotations

import ctypes
import threading

from .capi import LIB_PATH

__all__ = ["PMU_LIB_PATH", "PmuError", "enable", "registered", "ready", "available_counters", "is_hardware_counter"]

PMU_LIB_PATH = LIB_PATH.parent / "libxtc_hip_pmu.so"

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_registered = False

_SIGNATURES = {
    "xtc_hip_pmu_last_error": (ctypes.c_char_p, []),
    "xtc_hip_pmu_enable": (ctypes.c_int, []),
    "xtc_hip_pmu_ready": (ctypes.c_int, []),
    "xtc_hip_pmu_counter_count": (ctypes.c_int, [ctypes.c_int]),
    "xtc_hip_pmu_counter_name": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_char_p, ctypes.c_int]),
    "xtc_hip_pmu_open": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int)],
    ),
    "xtc_hip_pmu_start": (ctypes.c_int, []),
    "xtc_hip_pmu_stop": (ctypes.c_int, [ctypes.POINTER(ctypes.c_double), ctypes.c_int]),
    "xtc_hip_pmu_close": (None, []),
}


class PmuError(RuntimeError):
    """GPU counters could not be set up."""


def lib() -> ctypes.CDLL:
    """libxtc_hip_pmu.so, loaded with global symbols so that
    xtc_hip_evaluate_perf finds its entry points."""
    global _lib
    with _lock:
        if _lib is None:
            if not PMU_LIB_PATH.exists():
                raise PmuError(f"{PMU_LIB_PATH} is missing: build it with `python -m xtc_amd.csrc.build`")
            handle = ctypes.CDLL(str(PMU_LIB_PATH), mode=ctypes.RTLD_GLOBAL)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def _error() -> str:
    msg = lib().xtc_hip_pmu_last_error()
    return msg.decode() if msg else ""


def enable() -> None:
    """Registers the counter tool; raises PmuError once the ROCm runtime of
    this process has started (then only a new process can collect)."""
    global _registered
    if _registered:
        return
    if lib().xtc_hip_pmu_enable() != 0:
        raise PmuError(_error())
    _registered = True


def registered() -> bool:
    return _registered


def ready() -> bool:
    """True once the tool initialised with the runtime (after the first GPU call)."""
    return _registered and bool(lib().xtc_hip_pmu_ready())


def last_error() -> str:
    return _error() if _lib is not None else ""


def available_counters(device: int = 0) -> list[str]:
    """Counter names of GPU `device` (needs ready())."""
    L = lib()
    n = L.xtc_hip_pmu_counter_count(device)
    if n < 0:
        raise PmuError(f"no counters for GPU {device}: {_error() or 'tool not ready'}")
    buf = ctypes.create_string_buffer(256)
    names = []
    for i in range(n):
        if L.xtc_hip_pmu_counter_name(device, i, buf, len(buf)) == 0:
            names.append(buf.value.decode())
    return names


def is_hardware_counter(name: str) -> bool:
    return name.startswith("gpu.") and name not in ("gpu.time", "gpu.clocks")
