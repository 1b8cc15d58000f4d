# SPDX-License-Identifier: BSD-3-Clause
"""HipDevice: the AcceleratorDevice of the MI355X backend.

Re-implements, over libxtc_hip.so, what the reference's GPUDevice does over
the MLIR CUDA runtime (src/xtc/runtimes/accelerator/gpu/GPUDevice.py:33-353):
one process-wide device object, module loading with dlopen, device memory,
and the evaluate_perf timing protocol of the host runtime
(src/xtc/csrcs/runtimes/host/evaluate_perf.c:63-248).

Differences by design: host buffers are never registered for zero-copy
access (GPUDevice.py:327-347); tensors are copied into HBM so kernels read
device memory.  There is no CPU fallback: every call goes to the library,
which fails loudly when it is missing or no GPU is present.
"""

from __future__ import annotations

import ctypes
import os
import threading
from collections.abc import Callable
from typing import Any

from ...itf.runtime.accelerator import AcceleratorDevice
from . import capi

__all__ = ["HipDevice"]


class HipDevice(AcceleratorDevice):
    """Process-wide handle on one GPU (selected by `device`, default from
    XTC_HIP_DEVICE or 0)."""

    _instances: dict[int, "HipDevice"] = {}
    _lock = threading.Lock()

    def __new__(cls, device: int | None = None) -> "HipDevice":
        dev = int(os.environ.get("XTC_HIP_DEVICE", "0")) if device is None else int(device)
        with cls._lock:
            inst = cls._instances.get(dev)
            if inst is None:
                inst = super().__new__(cls)
                inst._device = dev
                inst._ready = False
                inst._modules: dict[str, ctypes.CDLL] = {}
                cls._instances[dev] = inst
            return inst

    def __init__(self, device: int | None = None) -> None:
        pass

    # ------------------------------------------------------------ identity

    def target_name(self) -> str:
        return "hip"

    def device_id(self) -> int:
        return self._device

    def device_name(self) -> str:
        self.init_device()
        buf = ctypes.create_string_buffer(256)
        capi.check(capi.lib().xtc_hip_device_name(buf, 256), "device_name")
        return buf.value.decode()

    def device_arch(self) -> str:
        self.init_device()
        buf = ctypes.create_string_buffer(256)
        capi.check(capi.lib().xtc_hip_device_arch(buf, 256), "device_arch")
        return buf.value.decode()

    def detect_accelerator(self) -> bool:
        if not capi.library_available():
            return False
        return capi.lib().xtc_hip_device_count() > self._device

    def init_device(self) -> None:
        if not self._ready:
            capi.check(capi.lib().xtc_hip_init(self._device), "xtc_hip_init")
            self._ready = True

    def deinit_device(self) -> None:
        if self._ready:
            capi.check(capi.lib().xtc_hip_synchronize(), "synchronize")

    # ------------------------------------------------------------- modules

    def load_module(self, module: Any) -> None:
        path = str(module.file_name)
        if path not in self._modules:
            capi.lib()  # libxtc_hip must be resident before the payload resolves it
            self._modules[path] = ctypes.CDLL(path, mode=ctypes.RTLD_LOCAL)

    def get_module_function(self, module: Any, function_name: str) -> Callable:
        handle = self._modules.get(str(module.file_name))
        if handle is None:
            raise RuntimeError(f"module {module.file_name} is not loaded")
        return getattr(handle, function_name)

    def module_symbol(self, module: Any, name: str) -> Any:
        handle = self._modules.get(str(module.file_name))
        return None if handle is None else getattr(handle, name, None)

    def unload_module(self, module: Any) -> None:
        path = str(module.file_name)
        handle = self._modules.pop(path, None)
        if handle is None:
            return
        release = getattr(handle, f"{module.payload_name}_release", None)
        if release is not None:
            release.restype = None
            release()
        dlclose = ctypes.CDLL(None).dlclose
        dlclose.argtypes = [ctypes.c_void_p]
        dlclose(handle._handle)

    # -------------------------------------------------------------- memory

    def memory_allocate(self, size_bytes: int) -> int:
        self.init_device()
        ptr = capi.lib().xtc_hip_malloc(max(1, int(size_bytes)))
        if not ptr:
            raise capi.HipError(f"xtc_hip_malloc({size_bytes}): {capi.last_error()}")
        return int(ptr)

    def memory_free(self, handle: Any) -> None:
        if handle:
            capi.check(capi.lib().xtc_hip_free(ctypes.c_void_p(int(handle))), "free")

    def memory_copy_to(self, acc_handle: Any, src: ctypes.c_void_p, size_bytes: int) -> None:
        capi.check(capi.lib().xtc_hip_memcpy_h2d(ctypes.c_void_p(int(acc_handle)), src, int(size_bytes)), "h2d")

    def memory_copy_from(self, acc_handle: Any, dst: ctypes.c_void_p, size_bytes: int) -> None:
        capi.check(capi.lib().xtc_hip_memcpy_d2h(dst, ctypes.c_void_p(int(acc_handle)), int(size_bytes)), "d2h")

    def memory_fill_zero(self, acc_handle: Any, size_bytes: int) -> None:
        capi.check(capi.lib().xtc_hip_memset_zero(ctypes.c_void_p(int(acc_handle)), int(size_bytes)), "fill_zero")

    def memory_data_pointer(self, acc_handle: Any) -> ctypes.c_void_p:
        return ctypes.c_void_p(int(acc_handle))

    # -------------------------------------------------------------- timing

    def evaluate_perf(
        self,
        pmu_events: list[str],
        repeat: int,
        number: int,
        min_repeat_ms: int,
        cfunc: Any,
        args: Any,
        nargs: int,
    ) -> list[float]:
        """Times `cfunc(*args)` with the evaluate_perf protocol.

        Without events: seconds per call (wall clock around synchronous
        calls).  Events, per call: "gpu.time" (device seconds, HIP events),
        "gpu.clocks" (device ns), "gpu.<counter>" (GPU hardware counters,
        xtc_amd.runtimes.hip.pmu), and the host counters "cycles", "clocks",
        "instructions", ... of perf_event_open; names that cannot be opened
        give -1.
        """
        self.init_device()
        nvals = max(1, len(pmu_events))
        results = (ctypes.c_double * (repeat * nvals))()
        names = (ctypes.c_char_p * max(1, len(pmu_events)))(*[e.encode() for e in pmu_events])
        fptr = ctypes.cast(cfunc, ctypes.c_void_p)
        argv = (ctypes.c_void_p * max(1, nargs))(*[ctypes.cast(a, ctypes.c_void_p).value if not isinstance(a, int) else a for a in list(args)[:nargs]])
        L = capi.lib()
        L.xtc_hip_evaluate_perf(results, len(pmu_events), names, repeat, number, min_repeat_ms, fptr, argv, nargs)
        if L.xtc_hip_evaluate_status():
            raise capi.HipError(capi.last_error())
        return [float(v) for v in results]

    def evaluate(self, results: Any, repeat: int, number: int, nargs: int, cfunc: Any, args: Any) -> None:
        vals = self.evaluate_perf([], repeat, number, 0, cfunc, args, nargs)
        for i, v in enumerate(vals):
            results[i] = v

    def evaluate_packed(self, *args: Any, **kwargs: Any) -> None:
        raise NotImplementedError("packed calling convention: HIP modules use bare pointers")

    def evaluate_packed_perf(self, *args: Any, **kwargs: Any) -> None:
        raise NotImplementedError("packed calling convention: HIP modules use bare pointers")

    def cndarray_new(self, ndim: int, shape: Any, dtype: Any, device: Any) -> Any:
        raise NotImplementedError("use xtc_amd.runtimes.hip.ndarray.DeviceArray")

    def cndarray_del(self, handle: Any) -> None:
        raise NotImplementedError("use xtc_amd.runtimes.hip.ndarray.DeviceArray")

    def cndarray_copy_from_data(self, handle: Any, data_handle: Any) -> None:
        raise NotImplementedError("use xtc_amd.runtimes.hip.ndarray.DeviceArray")

    def cndarray_copy_to_data(self, handle: Any, data_handle: Any) -> None:
        raise NotImplementedError("use xtc_amd.runtimes.hip.ndarray.DeviceArray")

    OPERANDS = {"reference": 0, "zero": 1, "random": 2}

    # measured peaks by (device, dtype, operands): the probe takes ~0.4 s
    _peaks: dict[tuple[int, str, str], float] = {}

    def evaluate_flops(self, dtype_name: str | bytes, operands: str = "reference") -> float:
        """Measured MFMA peak of the device in FMA/s (one XTC op per FMA):
        a register-only MFMA loop, operands the reference's integers
        1 + i % 127 (evaluate_flops.c:466-469), "zero" or "random".
        Measured once per process for each (device, dtype, operands).  A
        dtype the device has no MFMA probe for gives 0.0, as the reference's
        interface does for an unknown dtype; a failed probe raises."""
        name = dtype_name.decode() if isinstance(dtype_name, bytes) else dtype_name
        key = (self._device, name, operands)
        if key in self._peaks:
            return self._peaks[key]
        L = capi.lib()
        if L.xtc_hip_datasheet_flops(name.encode()) <= 0.0:
            return 0.0
        self.init_device()
        v = float(L.xtc_hip_evaluate_flops_operands(name.encode(), self.OPERANDS[operands]))
        if v <= 0.0:
            raise capi.HipError(capi.last_error() or f"evaluate_flops({name}) failed")
        self._peaks[key] = v
        return v

    @staticmethod
    def datasheet_flops(dtype_name: str) -> float:
        """Published dense MFMA peak of MI355X in FMA/s."""
        return float(capi.lib().xtc_hip_datasheet_flops(dtype_name.encode()))

    def __repr__(self) -> str:
        return f"HipDevice({self._device})"
