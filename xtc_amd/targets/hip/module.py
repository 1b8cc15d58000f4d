# SPDX-License-Identifier: BSD-3-Clause
"""HipModule: a compiled HIP payload (the analogue of
src/xtc/targets/accelerator/gpu/GPUModule.py:23-92 and
src/xtc/targets/host/HostModule.py:26-135)."""

from __future__ import annotations

import shutil
from pathlib import Path
from typing import Any, Callable

import numpy as np

from ...itf.comp import Module
from ...utils.bf16 import host_dtype

__all__ = ["HipModule", "graph_np_inputs_spec", "graph_np_outputs_spec", "graph_reference_impl"]


def _type_of(graph: Any, uid: str, inputs: bool) -> Any:
    if inputs:
        return graph.inputs_types[list(graph.inputs).index(uid)]
    return graph.outputs_types[list(graph.outputs).index(uid)]


def graph_np_inputs_spec(graph: Any) -> Callable[[], list[dict[str, Any]]]:
    """Shapes/dtypes of the graph inputs (src/xtc/utils/evaluation.py:21-46)."""

    def spec() -> list[dict[str, Any]]:
        return [
            {"shape": tuple(t.constant_shape), "dtype": t.constant_dtype, "device": t.device, "layout": t.layout}
            for t in (_type_of(graph, u, True) for u in graph.inputs)
        ]

    return spec


def graph_np_outputs_spec(graph: Any) -> Callable[[], list[dict[str, Any]]]:
    """Shapes/dtypes of the graph outputs (src/xtc/utils/evaluation.py:49-65)."""

    def spec() -> list[dict[str, Any]]:
        return [
            {"shape": tuple(t.constant_shape), "dtype": t.constant_dtype, "device": t.device}
            for t in (_type_of(graph, u, False) for u in graph.outputs)
        ]

    return spec


def graph_reference_impl(graph: Any) -> Callable[..., None]:
    """numpy interpreter of the graph writing into output arrays
    (src/xtc/utils/evaluation.py:68-75)."""
    from ...graphs.xtc.data import XTCTensor

    def run(*arrays: np.ndarray) -> None:
        n_in = len(graph.inputs)
        ins = [XTCTensor(a, type=_type_of(graph, u, True)) for a, u in zip(arrays[:n_in], graph.inputs)]
        outs = graph.forward(ins)
        for dst, res in zip(arrays[n_in:], outs):
            dst[...] = res.numpy().astype(dst.dtype, copy=False)

    return run


class HipModule(Module):
    def __init__(
        self,
        name: str,
        payload_name: str,
        file_name: str,
        graph: Any,
        plan: Any = None,
        configs: dict[str, Any] | None = None,
        source: str = "",
        device: int = 0,
        bare_ptr: bool = True,
        schedule_error: str | None = None,
    ) -> None:
        self._name = name
        self._payload_name = payload_name
        self._file_name = file_name
        self._graph = graph
        self.plan = plan
        self.configs = dict(configs or {})
        self.source = source
        self.device = device
        self._bare_ptr = bare_ptr
        # set when the schedule mapped onto no kernel (compile policy
        # "report"): the payload launches nothing and reports this message
        self.schedule_error = schedule_error
        self._np_inputs_spec = graph_np_inputs_spec(graph)
        self._np_outputs_spec = graph_np_outputs_spec(graph)
        self._reference_impl = graph_reference_impl(graph)

    @property
    def file_type(self) -> str:
        return "shlib"

    @property
    def name(self) -> str:
        return self._name

    @property
    def payload_name(self) -> str:
        return self._payload_name

    @property
    def file_name(self) -> str:
        return self._file_name

    @property
    def graph(self) -> Any:
        return self._graph

    def export(self) -> None:
        """Copies the payload next to the working directory as <name>.so."""
        dst = Path(f"{self._name}.so")
        if Path(self._file_name).resolve() != dst.resolve():
            shutil.copy(self._file_name, dst)

    def get_evaluator(self, **kwargs: Any) -> "Any":
        from .evaluator import HipEvaluator

        return HipEvaluator(self, **kwargs)

    def get_executor(self, **kwargs: Any) -> "Any":
        from .evaluator import HipExecutor

        return HipExecutor(self, **kwargs)

    def host_dtype(self, dtype: str) -> np.dtype:
        return host_dtype(dtype)
