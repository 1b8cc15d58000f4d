# SPDX-License-Identifier: BSD-3-Clause
"""Schedule exploration driver (the engine of `loop-explore`,
src/xtc/search/explore.py:200-873, src/xtc/search/pipeline.py:28-117,
src/xtc/search/callback.py:22-172).

Per sample: Backend(graph) -> get_scheduler() -> strategy.generate(sch, x)
-> schedule() -> get_compiler(...).compile() -> module.get_evaluator(...)
.evaluate(); time = min over repeats.  Compilation runs on a thread pool
(`jobs`), execution on one thread, as in the reference pipeline.  Results go
to a CSV with the reference's layout (sample columns, X, time, peak,
backend), optionally to a JSON-lines DB, and a `<output>.meta.json` run
manifest records the arguments.  Failed samples get time 0 and are logged,
and are not written to the CSV (callback.py:152-154).

Searches: "random", "exhaustive", "data", "default", and "iterative"
(src/xtc/search/explore.py:515-538): batches proposed by an optimizer
(xtc_amd/search/optimizers.py) that observes each batch's fraction of peak.

The exploring process also runs the GPU, so it starts no process once its
GPU runtime is up: the payloads' gcc runs in a CompileService (worker
processes of a fork server started before any GPU work), and the manifest's
`git rev-parse` runs before the first evaluation.  A Python caller that has
already run GPU work in its process calls CompileService.start_server()
before that work; otherwise Exploration(config)() on the HIP backend raises
instead of forking from a process whose GPU runtime is up.

With the HIP backend the strategy's samples are filtered to those that map
exactly onto a compiled kernel instance (schedule_policy "strict"), so every
measured point is the schedule it claims to be.
"""

from __future__ import annotations

import concurrent.futures as cf
import csv
import json
import logging
import os
import platform
import subprocess
import sys
import time
from dataclasses import dataclass, field, fields
from datetime import datetime, timezone
from importlib import import_module
from pathlib import Path
from typing import Any, Callable

import numpy as np

from .callback import DB_VERSION, CSVCallback, DBCallback, MemoryCallback, ResultCallBack, db_operator, db_strategy
from .strategies import Strategies

__all__ = ["ExplorationConfig", "Exploration", "CSVCallback", "DBCallback", "MemoryCallback", "ResultCallBack",
           "hip_sample_filter", "parse_x", "OPERATORS",
           "build_graph", "operation_dims", "config_graph", "random_parameters",
           "random_inputs_tolerance"]

logger = logging.getLogger("xtc_amd.search")


@dataclass
class ExplorationConfig:
    """Options of an exploration (src/xtc/search/explore.py:65-148).  The
    reference's fields are all here, with its defaults except `strategy`
    (tile_hip, the GPU-native space), `repeat` (5: the minimum of five
    timed repeats) and `backends` (hip).  `backend` is the one backend an
    `Exploration(graph, config)` runs; `Exploration(config)` builds the
    graph from `operator`/`dims`/`dtype` (or `op_name`, or `graph_file`)
    and runs every backend of `backends`."""

    backend: str = "hip"
    strategy: str = "tile_hip"
    strategy_kwargs: dict[str, Any] = field(default_factory=dict)
    search: str = "random"  # "random" | "exhaustive" | "data" | "default" | "iterative"
    trials: int = 100
    seed: int = 0
    optimizer: str = "random-forest-default"  # search "iterative"
    optimizer_config: str = ""  # YAML overrides of the optimizer preset
    batch: int = 1  # samples per optimizer proposal
    opt_level: int = 4  # 0-3: evaluate the strategy's default schedule at that level; 4: search
    data: str | None = None  # CSV of samples for search "data"
    repeat: int = 5
    number: int = 1
    min_repeat_ms: int = 100
    validate: bool = False
    pmu_counters: list[str] = field(default_factory=list)
    jobs: int = max(1, (os.cpu_count() or 2) // 2)
    output: str = "results.csv"
    db_file: str | None = None
    resume: bool = False
    append: bool = False
    peak_flops: float | None = None  # FMA/s; default: the device's dense MFMA peak
    compile_kwargs: dict[str, Any] = field(default_factory=dict)
    test: list[int] = field(default_factory=list)  # evaluate this one sample only
    execute: bool = True  # False: compile every sample, evaluate none
    quiet: bool = False  # no per-sample lines
    dump: bool = False  # print every payload's generated C source
    save_temps: bool = False  # keep payload sources under save_temps_dir/<ident>
    save_temps_dir: str = "./save_temps_dir"
    explore_dir: str | None = None  # where the payload libraries go (dump_file = <dir>/payload_<ident>)
    descript: str | None = None  # path to a descript YAML spec; replaces `strategy` when set
    # the graph, for Exploration(config): an operator of OPERATORS with its
    # dims (default: the operator's), a named operation's dims, or a file
    operator: str | None = "matmul"
    graph_file: str | None = None
    op_name: str | None = None
    func_name: str | None = None  # graph (payload) name, default to the operator
    dims: list[int] | None = None
    dtype: str = "float32"
    pad: int = 0  # conv2d: a pad2d producer on H and W (an extension)
    backends: list[str] = field(default_factory=lambda: ["hip"])
    # options of the reference's strategies (not tile_hip, which takes none)
    threads: int = 1
    max_unroll: int | None = None  # default 2^22: GPU tiles unroll further than the CPU bound of 256
    vec_size: int = 16
    # accepted for compatibility; they change nothing on this backend
    huge_pages: bool = True
    eval: str = "eval"
    bare_ptr: bool = False
    mlir_prefix: str | None = None
    use_tensors: bool = False
    progress_cls: str = "tqdm"
    debug_compile: bool = False  # log the payload compile commands
    eval_parameters: Any = None  # (inputs, outputs) numpy arrays for every evaluation
    random_inputs: int | None = None  # the seed of the CLI's eval_parameters (random_parameters), for the manifest
    # filled by Exploration(config).run(): (sample, code, time, backend) per sample
    results: list[Any] = field(default_factory=list)

    @classmethod
    def from_args(cls, args: Any = None, **overrides: Any) -> "ExplorationConfig":
        """A configuration from an argparse namespace (its attributes that
        name fields) and keyword overrides (src/xtc/search/explore.py:133-148)."""
        config = cls()
        names = {f for f in cls.__dataclass_fields__}
        if args is not None:
            for key, value in vars(args).items():
                if key in names:
                    setattr(config, key, value)
        for key, value in overrides.items():
            if key not in names:
                raise TypeError(f"unknown exploration configuration option: {key}")
            setattr(config, key, value)
        return config


# configuration fields left out of the run manifest: data, not options
_NOT_IN_MANIFEST = ("results", "eval_parameters")

# Operators of `operator` (src/xtc/search/explore.py:151-198): dimension
# names and default dims.
OPERATORS: dict[str, dict[str, Any]] = {
    "matmul": {"dims": ["i", "j", "k"], "default_dims": [512, 1024, 128]},
    "conv2d": {"dims": ["n", "h", "w", "f", "r", "s", "c", "SH", "SW"], "default_dims": [1, 112, 112, 64, 7, 7, 3, 2, 2]},
    "relu": {"dims": ["i"], "default_dims": [512 * 1024]},
}


def operation_dims(operator: str, name: str) -> list[int]:
    """Dims of a named operation: its loop sizes, then its params
    (src/xtc/search/explore.py:837-841)."""
    from ..artifacts import get_operation

    op = get_operation(operator, name)
    return [*op["dims"].values(), *op["params"].values()]


def build_graph(operator: str, dims: list[int], dtype: str, pad: int = 0, name: str | None = None) -> Any:
    """Graphs of the reference's operators, with the same tensor and node
    names and shapes (src/xtc/search/explore.py:218-256).  bfloat16
    matmul/conv accumulate and store fp32 (out_dtype extension).  `pad` > 0
    puts a pad2d producer on H and W in front of the conv (the C4 pattern);
    the padded input then has the reference's conv input shape.  `name` is
    the graph's (function's) name, default to the operator."""
    import xtc_amd.graphs.xtc.op as O

    extra = {"out_dtype": "float32"} if dtype == "bfloat16" else {}
    if operator == "matmul":
        i, j, k = dims
        a = O.tensor((i, k), dtype, name="A")
        b = O.tensor((k, j), dtype, name="B")
        with O.graph(name=name or "matmul") as gb:
            O.matmul(a, b, name="C", **extra)
        return gb.graph
    if operator == "conv2d":
        n, h, w, f, r, s, c, sh, sw = dims if len(dims) == 9 else (list(dims) + [1, 1])[:9]
        ih, iw = h * sh + r - 1 - 2 * pad, w * sw + s - 1 - 2 * pad
        x = O.tensor((n, ih, iw, c), dtype, name="A")
        wt = O.tensor((r, s, c, f), dtype, name="B")
        with O.graph(name=name or "conv2d") as gb:
            src = O.pad2d(x, padding=pad, axes=(1, 2), name="pad") if pad else x
            O.conv2d(src, wt, stride=(sh, sw), name="O", **extra)
        return gb.graph
    if operator == "relu":
        (i,) = dims
        x = O.tensor((i,), dtype, name="I")
        with O.graph(name=name or "relu") as gb:
            O.relu(x, threshold=0, name="O")
        return gb.graph
    raise ValueError(f"unknown operator {operator}")


def random_parameters(graph: Any, seed: int) -> tuple[list[np.ndarray], list[np.ndarray]]:
    """(inputs, outputs) for every evaluation of an exploration: seeded
    uniform[-1, 1) inputs in graph-input order, rounded to bfloat16 for
    bfloat16 tensors, and output buffers.  An extension: the reference
    evaluates on np_init integers (src/xtc/utils/numpy.py:12-19).  On MI355X
    the power a bf16 GEMM draws, hence its clock, depends on its operands, so
    a search meant for random data has to time it on random data."""
    from ..utils.bf16 import host_dtype, round_to_bf16

    rng = np.random.default_rng(seed)
    ins = []
    for t in graph.inputs_types:
        x = rng.uniform(-1.0, 1.0, tuple(t.constant_shape))
        if str(t.constant_dtype) == "bfloat16":
            x = round_to_bf16(x.astype(np.float32))
        ins.append(np.ascontiguousarray(x.astype(host_dtype(t.constant_dtype))))
    outs = [np.empty(tuple(t.constant_shape), dtype=host_dtype(t.constant_dtype)) for t in graph.outputs_types]
    return ins, outs


def random_inputs_tolerance(graph: Any) -> float:
    """Validation bound on random_parameters' inputs, as max |got - ref| /
    max |ref|: the payload and numpy sum in different orders, so on
    non-integer data they agree only to the accumulator's rounding.  1e-4
    for fp32 accumulation (bf16 or fp32 operands: a wrong kernel is off by
    O(1)), 1e-10 for float64, and 1e-2 when an output is stored in bfloat16,
    where two fp32 sums a few bits apart can round to neighbouring bf16
    values (one bf16 ulp is at most 2^-7 of the value)."""
    dtypes = {str(t.constant_dtype) for t in graph.outputs_types}
    if "bfloat16" in dtypes:
        return 1e-2
    return 1e-10 if dtypes == {"float64"} else 1e-4


def config_graph(config: ExplorationConfig) -> Any:
    """The graph an Exploration(config) explores: the graph file, else the
    operator with the named operation's dims, the given dims or its
    default ones."""
    if config.graph_file:
        import xtc_amd.graphs.xtc.op as O

        with O.graph() as gb:
            gb.load(config.graph_file)
        return gb.graph
    if not config.operator or config.operator not in OPERATORS:
        raise ValueError(f"unknown operator {config.operator!r}: one of {list(OPERATORS)}")
    if config.op_name:
        dims = operation_dims(config.operator, config.op_name)
    else:
        dims = list(config.dims) if config.dims else list(OPERATORS[config.operator]["default_dims"])
    return build_graph(config.operator, dims, config.dtype, config.pad, name=config.func_name or config.operator)


def parse_x(text: str) -> list[int]:
    """The X column back to a sample ('[1; 2; 3]' or '[1, 2, 3]')."""
    return [int(v) for v in json.loads(text.replace(";", ","))]


def hip_sample_filter(graph: Any, strategy_factory: Callable[..., Any]) -> Callable[[list[int]], bool]:
    """Predicate: does this sample's schedule map exactly onto a compiled
    kernel instance?  Builds the schedule on a scratch HipBackend."""
    from ..backends.hip import Backend
    from ..backends.hip.mapping import map_node
    from ..backends.hip.scheduler import ScheduleError

    backend = Backend(graph)
    probe = strategy_factory()
    cache: dict[tuple[int, ...], bool] = {}

    def ok(sample: list[int]) -> bool:
        key = tuple(sample)
        if key not in cache:
            sch = backend.get_scheduler()
            try:
                probe.generate(sch, list(sample))
                schedule = sch.schedule()
                for ln in backend.plan.launches:
                    if ln.kind in ("matmul", "conv2d"):
                        map_node(ln.attrs, ln.kind == "conv2d", schedule.node(ln.node), "strict")
                cache[key] = True
            except (ScheduleError, ValueError):
                cache[key] = False
        return cache[key]

    return ok


# GPU hardware counters per sample are switched off in the explorer: with
# them, loop-explore stalled until killed on MI355X (twice, the second time
# with the payload compiler moved out of the process), while the same
# counters collected by one HipEvaluator in a fresh process work.  The cause
# is not found, so the path raises instead of running.
EXPLORE_HW_COUNTERS_OFF = (
    "loop-explore: GPU hardware counters per sample ({names}) are switched off: explorations that collected "
    "them stalled on MI355X and the cause is not found.  gpu.time and gpu.clocks work here; a module's evaluator "
    "(HipEvaluator pmu_counters=[...]) collects hardware counters in a fresh process."
)


def check_explore_counters(names: list[str]) -> None:
    """Raises ValueError when `names` holds a GPU hardware counter."""
    from ..runtimes.hip.pmu import is_hardware_counter

    hw = [n for n in names if is_hardware_counter(n)]
    if hw:
        raise ValueError(EXPLORE_HW_COUNTERS_OFF.format(names=", ".join(hw)))


class Exploration:
    """An exploration, in either of two forms:

    * `Exploration(config)` (the reference's, src/xtc/search/explore.py:
      200-210, 864-873): the graph comes from the configuration
      (config_graph), every backend of `config.backends` is explored, and
      `run()` (or calling the object) returns and keeps in `results` and
      `config.results` one (sample, code, time, backend) per sample;
    * `Exploration(graph, config)`: `config.backend` on a given graph;
      `run()` returns (sample, times, code, message) per sample.
    """

    def __init__(self, graph: Any = None, config: ExplorationConfig | None = None) -> None:
        self.results: list[Any] = []
        if config is None and (graph is None or isinstance(graph, ExplorationConfig)):
            self.config = graph if graph is not None else ExplorationConfig()
            self.graph = None
            self.strategy = None
            self.peak_time_s = 0.0
            return
        assert config is not None, "Exploration(graph, config) needs a configuration"
        self.graph = graph
        self.config = config
        self._backend_mod = import_module(f"xtc_amd.backends.{config.backend}")
        factory = self._strategy_factory(graph, config)
        kwargs: dict[str, Any] = {}
        if config.backend == "hip" and (config.descript or self.strategy_name(config.strategy) != "tile_hip"):
            kwargs["sample_filter"] = hip_sample_filter(graph, factory)
        self.strategy = factory(**kwargs)
        self.peak_time_s = 0.0  # the graph's time at peak, set by run()

    # ---- the reference's static helpers (src/xtc/search/explore.py:211-261, 813-862)
    @staticmethod
    def xtc_load_graph(graph_file: str) -> Any:
        import xtc_amd.graphs.xtc.op as O

        with O.graph() as gb:
            gb.load(graph_file)
        return gb.graph

    @staticmethod
    def xtc_matmul_graph(i: int, j: int, k: int, dtype: str, name: str = "matmul") -> Any:
        return build_graph("matmul", [i, j, k], dtype, name=name)

    @staticmethod
    def xtc_relu_graph(i: int, dtype: str, name: str = "relu") -> Any:
        return build_graph("relu", [i], dtype, name=name)

    @staticmethod
    def xtc_conv2d_graph(n: int, h: int, w: int, f: int, r: int, s: int, c: int, SH: int, SW: int, dtype: str,
                         name: str = "conv2d") -> Any:
        return build_graph("conv2d", [n, h, w, f, r, s, c, SH, SW], dtype, name=name)

    @staticmethod
    def get_strategy_name(strategy: str) -> str:
        return Strategies.resolve_name(strategy)

    @staticmethod
    def get_operation_dims(operator: str, name: str) -> list[int]:
        return operation_dims(operator, name)

    @staticmethod
    def list_operations_dims(operator: str) -> None:
        from ..artifacts import get_operation, list_operations

        for _, name in list_operations(operator):
            op = get_operation(operator, name)
            print(f"{name}: {op['dims']}, {op['params']}")

    @staticmethod
    def list_operators() -> None:
        for name in OPERATORS:
            print(name)

    @staticmethod
    def list_strategies() -> None:
        for name in Strategies.names(include_aliases=True):
            print(name)

    @staticmethod
    def list_optimizers() -> None:
        from .optimizers import Optimizers

        for name in Optimizers.names():
            print(name)

    @staticmethod
    def strategy_name(strategy: str) -> str:
        """The registered name of `strategy`, whose arguments follow a colon
        (`prt:PPRPRP`; src/xtc/search/explore.py:813-834)."""
        return Strategies.resolve_name(strategy.split(":")[0])

    @staticmethod
    def _strategy_factory(graph: Any, config: ExplorationConfig) -> Callable[..., Any]:
        """Strategy constructor: a descript spec file replaces the named
        strategy; the reference's strategies get `threads`, `max_unroll`
        and `vec_size` (src/xtc/search/explore.py:817-834), tile_hip takes
        no option; `strategy_kwargs` override them."""
        if config.descript:
            from .descript_strategy import Strategy_Descript

            with open(config.descript) as f:
                spec = f.read()
            return lambda **kw: Strategy_Descript(graph, spec, **{**config.strategy_kwargs, **kw})
        name, *args = config.strategy.split(":")
        options: dict[str, Any] = {}
        if Strategies.resolve_name(name) != "tile_hip":
            options = {"threads": config.threads, "vec_size": config.vec_size,
                       "max_unroll": config.max_unroll if config.max_unroll is not None else 1 << 22}
        return lambda **kw: Strategies.create(name, graph, *args, **{**options, **config.strategy_kwargs, **kw})

    # ---- sample sources
    def samples(self) -> list[list[int]]:
        c = self.config
        if c.test:
            return [list(c.test)]
        # opt-level 0-3 evaluates the strategy's default schedule at that
        # level, whatever the search (src/xtc/search/explore.py:784-800)
        if c.opt_level in (0, 1, 2, 3):
            return [list(self.strategy.default_schedule(c.opt_level))]
        if c.search == "exhaustive":
            from itertools import islice

            return [list(x) for x in islice(self.strategy.exhaustive(), c.trials)]
        if c.search == "random":
            return [list(x) for x in self.strategy.sample(c.trials, seed=c.seed)]
        if c.search == "data":
            if not c.data:
                raise ValueError("search 'data' needs a data CSV")
            with open(c.data, newline="") as f:
                return [parse_x(row["X"]) for row in csv.DictReader(f)]
        if c.search == "default":
            return [list(self.strategy.default_schedule(2))]
        raise ValueError(f"unknown search {c.search!r}")

    # ---- one sample
    def compile_one(self, sample: list[int], ident: str = "0000") -> Any:
        c = self.config
        backend = self._backend_mod.Backend(self.graph)
        sch = backend.get_scheduler()
        self.strategy.generate(sch, sample)
        kwargs = {"shared_lib": True, **c.compile_kwargs}
        if c.explore_dir:
            kwargs.setdefault("dump_file", f"{c.explore_dir}/payload_{ident}")
        if c.dump:
            kwargs.setdefault("print_source_ir", True)
        if c.debug_compile:
            kwargs.setdefault("debug", True)
        if c.save_temps:
            kwargs.setdefault("save_temps", True)
            kwargs.setdefault("save_temps_dir", f"{c.save_temps_dir}/{ident}")
        if c.backend == "hip":
            kwargs.setdefault("schedule_policy", "strict")
        return backend.get_compiler(**kwargs).compile(sch.schedule())

    def counters(self) -> list[str]:
        """The pmu_counters each sample is evaluated with: the requested ones,
        with "gpu.time" added first when missing so that the time column
        stays a time.  Empty when none were requested (plain timing)."""
        req = list(self.config.pmu_counters)
        if req and "gpu.time" not in req:
            req = ["gpu.time", *req]
        return req

    def evaluate_one(self, module: Any) -> tuple[list[float], int, str]:
        c = self.config
        check_explore_counters(c.pmu_counters)
        extra = {}
        if c.random_inputs is not None:
            extra["scaled_tolerance"] = random_inputs_tolerance(self.graph if self.graph is not None else config_graph(c))
        return module.get_evaluator(
            repeat=c.repeat, number=c.number, min_repeat_ms=c.min_repeat_ms, validate=c.validate,
            pmu_counters=self.counters(), parameters=c.eval_parameters, **extra,
        ).evaluate()

    def split_counters(self, values: list[float]) -> tuple[list[float], dict[str, list[float]]]:
        """Evaluator values -> (times, {counter: per-repeat values}).  With
        counters the evaluator returns them repeat by repeat, in counter order
        (evaluate_perf's layout); the times are the "gpu.time" entries."""
        names = self.counters()
        if not names:
            return values, {}
        per = {name: values[i :: len(names)] for i, name in enumerate(names)}
        return per["gpu.time"], per

    def peak_time(self) -> float:
        """The graph's time at the device's MFMA peak for the graph's ops
        dtype (explore.py:619-625): bfloat16 for a bf16 matmul or conv even
        when it stores float32."""
        peak = self.config.peak_flops
        if peak is None and self.config.backend == "hip":
            from ..runtimes.hip.device import HipDevice

            peak = HipDevice().evaluate_flops(self.graph.ops_dtype())
        return self.graph.ops_count() / peak if peak else 0.0

    def write_manifest(self) -> None:
        try:
            commit = subprocess.run(["git", "rev-parse", "HEAD"], capture_output=True, text=True, check=True).stdout.strip()
        except (OSError, subprocess.CalledProcessError):
            commit = None
        meta = {
            "generatedAt": datetime.now(timezone.utc).isoformat(),
            "output": self.config.output,
            "sampleNames": self.strategy.sample_names,
            "gitCommit": commit,
            "python": {"version": sys.version, "executable": sys.executable},
            "platform": {"platform": sys.platform, "machine": platform.machine(), "cwd": os.getcwd()},
            "args": {f.name: (v if isinstance(v, (str, int, float, bool, list, dict, type(None))) else str(v))
                     for f in fields(self.config) if f.name not in _NOT_IN_MANIFEST
                     for v in [getattr(self.config, f.name)]},
        }
        Path(f"{self.config.output}.meta.json").write_text(json.dumps(meta, indent=2, sort_keys=True) + "\n")

    def _evaluate_compiled(
        self, sample: list[int], fut: Any, csv_cb: CSVCallback, db_cb: DBCallback | None
    ) -> tuple[list[int], list[float], int, str]:
        c = self.config
        extra: dict[str, Any] = {}
        if not c.execute:
            # compile only: a compile error is reported, nothing is timed or recorded
            try:
                fut.result()
                return (sample, [], 0, "compiled, not executed")
            except Exception as err:
                logger.warning("sample %s failed to compile: %s", sample, err)
                return (sample, [], 2, f"{type(err).__name__}: {err}")
        try:
            module = fut.result()
            extra = {"kernels": {k: v.describe() for k, v in getattr(module, "configs", {}).items()}, "error": ""}
            values, code, msg = self.evaluate_one(module)
            times, per_counter = self.split_counters(values) if code == 0 else ([], {})
            if per_counter:
                extra["counters"] = per_counter
        except Exception as err:  # a failed sample is recorded, not fatal
            times, code, msg = [], 2, f"{type(err).__name__}: {err}"
        if code:
            logger.warning("sample %s failed: %s", sample, msg)
        if code == 0 and not times:
            code, msg = 2, "the evaluator returned no time"
        # the callbacks' result tuple (src/xtc/search/callback.py): time is the minimum over the repeats
        result = (sample, code, min(times) if code == 0 else 0.0, c.backend)
        csv_cb(result)
        if db_cb:
            db_cb.record(result, {**extra, "error": msg})
        return (sample, times, code, msg)

    def _run_batch(
        self, pool: cf.ThreadPoolExecutor, todo: list[list[int]], csv_cb: CSVCallback, db_cb: DBCallback | None,
        done: int, total: int,
    ) -> list[tuple[list[int], list[float], int, str]]:
        futures = [pool.submit(self.compile_one, s, f"{done + i:04}") for i, s in enumerate(todo)]
        out = []
        for idx, (sample, fut) in enumerate(zip(todo, futures)):
            res = self._evaluate_compiled(sample, fut, csv_cb, db_cb)
            out.append(res)
            best = min(res[1]) if res[1] else 0.0
            if not self.config.quiet:
                logger.info("[%d/%d] %s -> %.3g s (%s)", done + idx + 1, total, sample, best, res[3] or "ok")
        return out

    def __call__(self) -> list[Any]:
        return self.run()

    def run(self) -> list[Any]:
        if self.graph is None:
            return self._run_config()
        return self._run_graph()

    def _run_config(self) -> list[tuple[list[int], int, float, str]]:
        """Exploration(config): every backend of config.backends on the
        configuration's graph; one (sample, code, time, backend) per sample,
        time the minimum over repeats (0 when the sample failed), and the
        best sample's line unless quiet (src/xtc/search/explore.py:764-811)."""
        from dataclasses import replace

        c = self.config
        graph = config_graph(c)
        out: list[tuple[list[int], int, float, str]] = []
        best: tuple[float, list[int], str, float] | None = None
        for backend in c.backends:
            sub = Exploration(graph, replace(c, backend=backend, results=[]))
            for sample, times, code, _ in sub.run():
                t = min(times) if code == 0 and times else 0.0
                out.append((list(sample), code, t, backend))
                if t > 0 and (best is None or t < best[0]):
                    best = (t, list(sample), backend, sub.peak_time_s / t if sub.peak_time_s else 0.0)
        if best is not None and not c.quiet:
            t, sample, backend, peak = best
            print(f"Schedule: {backend}: {sample}: time: {t * 1000:.2f} msecs, peak perf: {peak * 100:.2f}%",
                  flush=True)
        self.results = out
        c.results = out
        return out

    # ---- the exploration proper
    def _run_graph(self) -> list[tuple[list[int], list[float], int, str]]:
        from contextlib import nullcontext

        c = self.config
        service: Any = nullcontext()
        if c.backend == "hip":
            from ..backends.hip.compiler import CompileService

            service = CompileService(c.jobs)
        with service:
            self.write_manifest()  # runs git: before any GPU work
            results: list[tuple[list[int], list[float], int, str]] = []
            t0 = time.time()
            iterative = c.search == "iterative" and not c.test and c.opt_level not in (0, 1, 2, 3)
            samples: list[list[int]] = [] if iterative else self.samples()
            # compile-only runs never touch the GPU
            peak_time = self.peak_time() if c.execute else 0.0
            self.peak_time_s = peak_time
            if c.save_temps:
                Path(c.save_temps_dir).mkdir(parents=True, exist_ok=True)
                self.graph.dump(str(Path(c.save_temps_dir) / f"{self.graph.name}.graph.yaml"))
            csv_cb = CSVCallback(c.output, peak_time, self.strategy.sample_names, resume=c.resume, append=c.append)
            db_cb = None
            if c.db_file:
                db_cb = DBCallback(c.db_file, "gfx950", 1, "descript" if c.descript else self.strategy_name(c.strategy))
                db_cb.set_graph(self.graph)
            try:
                with cf.ThreadPoolExecutor(max_workers=max(1, c.jobs)) as pool:
                    if iterative:
                        results = self._run_iterative(pool, csv_cb, db_cb, peak_time)
                    else:
                        todo = [s for s in samples if (c.backend, tuple(s)) not in csv_cb.seen]
                        results = self._run_batch(pool, todo, csv_cb, db_cb, 0, len(todo))
            finally:
                csv_cb.close()
                if db_cb:
                    db_cb.close()
            if not c.quiet:
                logger.info("explored %d samples in %.1f s", len(results), time.time() - t0)
        return results

    def _run_iterative(
        self, pool: cf.ThreadPoolExecutor, csv_cb: CSVCallback, db_cb: DBCallback | None, peak_time: float
    ) -> list[tuple[list[int], list[float], int, str]]:
        """Batches of `batch` samples proposed by the optimizer, which then
        observes each one's fraction of peak (peak_time / time, 0 when the
        sample failed), for `trials` samples in all
        (src/xtc/search/explore.py:515-538)."""
        from .optimizers import Optimizers

        c = self.config
        opt = Optimizers.from_name(c.optimizer)(
            lambda n, seed: self.strategy.sample(n, seed=seed), c.batch, c.seed, c.optimizer_config
        )
        results: list[tuple[list[int], list[float], int, str]] = []
        # a strategy that can name the library's own choice for the graph
        # (tile_hip) puts it in the first batch in place of the optimizer's
        # last pick: the optimizer then learns from it, and the search never
        # ends below the default; the optimizer's draws are unchanged
        start = [list(self.strategy.default_schedule(2))] if getattr(self.strategy, "starts_from_default", False) else []
        for step in range(0, c.trials, c.batch):
            size = min(c.batch, c.trials - step)
            first = start if step == 0 else []
            batch = first + [list(x) for x in opt.suggest()[: size - len(first)]]
            got = self._run_batch(pool, batch, csv_cb, db_cb, step, c.trials)
            results.extend(got)
            opt.observe(batch, [peak_time / min(t) if code == 0 and t and min(t) > 0 else 0.0 for _, t, code, _ in got])
        opt.finished()
        return results
