# SPDX-License-Identifier: BSD-3-Clause
"""HipEvaluator / HipExecutor.

Same kwargs, steps and result convention as the reference's GPUEvaluator
(src/xtc/targets/accelerator/gpu/GPUEvaluator.py:24-138) and
HostEvaluator (src/xtc/targets/host/HostEvaluator.py:28-120):
  repeat=1, number=1, min_repeat_ms=100, validate=False, parameters=None,
  init_zero=False, pmu_counters=[], np_inputs_spec, np_outputs_spec,
  reference_impl.
Steps: init device -> load payload -> inputs (np_init integers 1..9 unless
`parameters`: numpy arrays or NDArrays, on the host or the device) copied
to HBM -> optional validation against the graph's numpy interpreter with
np.allclose (src/xtc/utils/evaluation.py:129-145) -> timing with the
evaluate_perf protocol -> unload -> copy outputs back into caller-provided
arrays (numpy arrays, or NDArrays through copy_from_numpy).  Returns
(per-repeat seconds per call, code, msg); code 1 on a validation mismatch,
2 on a HIP/payload error.
With pmu_counters the results are, per repeat, one value per counter, per
call (src/xtc/csrcs/runtimes/host/evaluate_perf.c:63-125): "gpu.time" /
"gpu.clocks" from HIP events, "gpu.cycles" and "gpu.<counter>" from the
hardware counters of xtc_amd.runtimes.hip.pmu (-1 for a counter the device
does not have, as the reference reports an event it cannot open).

Differences by design: tensors live in HBM during timing (the reference maps
host memory for device access); `rtol`/`atol` may override np.allclose's
defaults, and `scaled_tolerance=t` replaces np.allclose by
max |got - ref| <= t * max |ref| (NaNs in the same places), the check for
non-integer inputs, whose fp32 sums differ from numpy's in the last bits
by summation order.  "gpu.time" / "gpu.clocks" pmu counters return device
time per call measured with HIP events.
"""

from __future__ import annotations

import ctypes
from typing import Any

import numpy as np

from ...itf.exec import Evaluator, Executor
from ...runtimes.hip import capi, pmu
from ...runtimes.hip.device import HipDevice
from ...runtimes.hip.ndarray import DeviceArray
from ...utils.bf16 import host_dtype
from ...utils.numpy import np_init

__all__ = ["HipEvaluator", "HipExecutor", "outputs_mismatch"]


def outputs_mismatch(ref: np.ndarray, got: np.ndarray, rtol: float, atol: float,
                     scaled_tolerance: float | None = None) -> str | None:
    """None when `got` passes the validation of `ref`, else what differs.
    Default: np.allclose(ref, got, rtol, atol) (src/xtc/utils/evaluation.py:
    129-145).  With scaled_tolerance t: NaN in the same places and
    max |got - ref| <= t * max |ref| over the rest."""
    diff = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    if scaled_tolerance is None:
        if np.allclose(ref, got, rtol=rtol, atol=atol):
            return None
        worst = np.unravel_index(int(np.nanargmax(diff / (np.abs(ref) + atol))), ref.shape)
        return (f"at {tuple(int(i) for i in worst)}: got {got[worst]!r}, expected {ref[worst]!r}; "
                f"max |diff| {np.nanmax(diff):.3g}")
    nan_ref, nan_got = np.isnan(ref), np.isnan(got)
    if not np.array_equal(nan_ref, nan_got):
        where = np.unravel_index(int(np.argmax(nan_ref != nan_got)), ref.shape)
        return f"at {tuple(int(i) for i in where)}: got {got[where]!r}, expected {ref[where]!r} (NaN)"
    ok = ~nan_ref
    if not ok.any():
        return None
    scale = float(np.max(np.abs(ref[ok].astype(np.float64))))
    err = float(np.max(diff[ok]))
    if err <= scaled_tolerance * scale:
        return None
    worst = np.unravel_index(int(np.argmax(np.where(ok, diff, -1.0))), ref.shape)
    return (f"at {tuple(int(i) for i in worst)}: got {got[worst]!r}, expected {ref[worst]!r}; "
            f"max |diff| / max |ref| = {err / scale if scale else float('inf'):.3g} > {scaled_tolerance:g}")


class HipEvaluator(Evaluator):
    def __init__(self, module: Any, **kwargs: Any) -> None:
        self._module = module
        self._device = HipDevice(getattr(module, "device", 0))
        self._repeat = int(kwargs.get("repeat", 1))
        self._number = int(kwargs.get("number", 1))
        self._min_repeat_ms = int(kwargs.get("min_repeat_ms", 100))
        self._validate = bool(kwargs.get("validate", False))
        self._parameters = kwargs.get("parameters")
        self._init_zero = bool(kwargs.get("init_zero", False))
        self._pmu_counters = list(kwargs.get("pmu_counters", []))
        self._np_inputs_spec = kwargs.get("np_inputs_spec", module._np_inputs_spec)
        self._np_outputs_spec = kwargs.get("np_outputs_spec", module._np_outputs_spec)
        self._reference_impl = kwargs.get("reference_impl", module._reference_impl)
        self._rtol = float(kwargs.get("rtol", 1e-5))
        self._atol = float(kwargs.get("atol", 1e-8))
        scaled = kwargs.get("scaled_tolerance")
        self._scaled_tolerance = None if scaled is None else float(scaled)
        if module.file_type != "shlib":
            raise ValueError("only shlib modules can be evaluated")

    @property
    def module(self) -> Any:
        return self._module

    def _host_parameters(
        self,
    ) -> tuple[list[np.ndarray], list[np.ndarray], list[str], list[str], list[list[int] | None]]:
        """Logical host arrays, dtypes and the inputs' layouts (a [1, 0]
        input is stored transposed on the device, as the reference's NDArray
        does for a layout spec, src/xtc/utils/evaluation.py:78-100)."""
        ins_spec = self._np_inputs_spec()
        outs_spec = self._np_outputs_spec()
        in_dt = [s["dtype"] for s in ins_spec]
        out_dt = [s["dtype"] for s in outs_spec]
        layouts = [s.get("layout") for s in ins_spec]
        if self._parameters is None:
            ins = [np_init(s["shape"], s["dtype"]) for s in ins_spec]
            make = np.zeros if self._init_zero else np.empty
            outs = [make(s["shape"], dtype=host_dtype(s["dtype"])) for s in outs_spec]
        else:
            ins = [np.asarray(getattr(a, "numpy", lambda a=a: a)()) for a in self._parameters[0]]
            outs = [np.asarray(getattr(a, "numpy", lambda a=a: a)()) for a in self._parameters[1]]
        return ins, outs, in_dt, out_dt, layouts

    def _status(self) -> tuple[int, str]:
        status = self._device.module_symbol(self._module, f"{self._module.payload_name}_status")
        if status is None:
            return 0, ""
        status.restype = ctypes.c_int
        rc = int(status())
        if rc == 0:
            return 0, ""
        msg = self._device.module_symbol(self._module, f"{self._module.payload_name}_message")
        msg.restype = ctypes.c_char_p
        return rc, (msg() or b"").decode()

    def evaluate(self) -> tuple[list[float], int, str]:
        if getattr(self._module, "schedule_error", None):
            return ([], 2, f"Error in compilation: schedule: {self._module.schedule_error}")
        dev = self._device
        hw = [c for c in self._pmu_counters if pmu.is_hardware_counter(c)]
        if hw and not pmu.registered():
            try:
                pmu.enable()
            except pmu.PmuError as err:
                return ([], 2, f"Error in execution: GPU counters {hw} need xtc_amd.runtimes.hip.pmu.enable() "
                               f"(or XTC_HIP_PMU=1) before the first GPU call of the process: {err}")
        dev.init_device()
        if hw and not pmu.ready():
            why = pmu.last_error() or "the counter tool did not initialise (the ROCm runtime of this process " \
                "started before xtc_amd.runtimes.hip.pmu.enable())"
            return ([], 2, f"Error in execution: GPU counters {hw} unavailable: {why}")
        dev.load_module(self._module)
        func = dev.get_module_function(self._module, self._module.payload_name)
        func.restype = None
        ins, outs, in_dt, out_dt, layouts = self._host_parameters()
        d_ins = [DeviceArray.from_numpy(a, dt, dev, lay) for a, dt, lay in zip(ins, in_dt, layouts)]
        d_outs = [DeviceArray(a.shape, dt, dev) for a, dt in zip(outs, out_dt)]
        if self._init_zero:
            for d in d_outs:
                d.fill_zero()
        args = [d.data for d in (*d_ins, *d_outs)]
        c_args = [ctypes.c_void_p(a) for a in args]
        result: tuple[list[float], int, str] = ([], 0, "")
        try:
            if self._validate:
                func(*c_args)
                rc, msg = self._status()
                if rc:
                    return ([], 2, f"Error in execution: {msg}")
                ref_outs = [np.empty(o.shape, host_dtype(dt)) for o, dt in zip(outs, out_dt)]
                self._reference_impl(*[a.copy() for a in ins], *ref_outs)
                for idx, (ref, d) in enumerate(zip(ref_outs, d_outs)):
                    got = d.numpy()
                    why = outputs_mismatch(ref, got, self._rtol, self._atol, self._scaled_tolerance)
                    if why is not None:
                        return ([], 1, f"Error in validation: outputs differ (output {idx}, {why})")
            fptr = ctypes.cast(func, ctypes.c_void_p)
            times = dev.evaluate_perf(
                self._pmu_counters, self._repeat, self._number, self._min_repeat_ms, fptr, args, len(args)
            )
            rc, msg = self._status()
            if rc:
                return ([], 2, f"Error in execution: {msg}")
            result = (times, 0, "")
            if self._parameters is not None:
                for dst, d in zip(self._parameters[1], d_outs):
                    if isinstance(dst, np.ndarray):
                        d.numpy(out=dst)
                    elif hasattr(dst, "copy_from_numpy"):  # an NDArray (xtc_amd.runtimes.types)
                        dst.copy_from_numpy(d.numpy())
        except capi.HipError as err:
            result = ([], 2, f"Error in execution: {err}")
        finally:
            for d in (*d_ins, *d_outs):
                d.free()
            dev.unload_module(self._module)
        return result


class HipExecutor(Executor):
    """Runs the payload once (Evaluator with repeat=1, number=1,
    min_repeat_ms=0; src/xtc/targets/accelerator/gpu/GPUEvaluator.py:120-138)."""

    def __init__(self, module: Any, **kwargs: Any) -> None:
        kwargs = {**kwargs, "repeat": 1, "number": 1, "min_repeat_ms": 0}
        self._evaluator = HipEvaluator(module, **kwargs)

    def execute(self) -> int:
        _, code, _ = self._evaluator.evaluate()
        return code

    @property
    def module(self) -> Any:
        return self._evaluator.module
