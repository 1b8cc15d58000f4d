# SPDX-License-Identifier: BSD-3-Clause
"""Compiler of the HIP backend: Schedule -> payload shared object.

The payload follows the reference's module convention
(src/xtc/backends/mlir/MlirGraphBackend.py:125-171,
src/xtc/backends/mlir/MlirTarget/MlirLLVMTarget.py:311): a shared object
exporting `void <graph.name>(void *in0, ..., void *out0, ...)` taking bare
device pointers to dense row-major tensors, inputs first.  Its body is a
short sequence of calls into libxtc_hip (one per kernel launch of the plan,
each with its kernel instance fixed by the schedule), then a stream
synchronisation, because callers time the payload with a wall clock around
the call (src/xtc/csrcs/runtimes/host/evaluate_perf.c:92-120).

The GPU kernels themselves are compiled once into libxtc_hip.so, so a
schedule compiles in ~0.1 s of host C (the MLIR backend spends ~1-3 s per
sample in mlir-translate/opt/llc/cc).  Side symbols give the payload an
error channel the reference lacks: `<name>_status()`, `<name>_message()`,
and `<name>_release()` frees the intermediate-tensor workspace.

Compile kwargs (src/xtc/search/explore.py:365-391): shared_lib, dump_file,
bare_ptr (always True, as the MLIR compiler forces it), debug,
print_source_ir (prints the generated C), save_temps,
save_temps_dir, target ("hip" or a HipDevice), selected_device, and the
extensions schedule_policy and synchronize (False: the payload returns with
its kernels queued).

schedule_policy says what happens to a schedule that maps onto no compiled
kernel instance (mapping.py):
  * "report" (default): compile() still returns a module, but its payload
    launches nothing and reports the mapping error through
    `<name>_status()` / `<name>_message()`; its evaluator returns code 2
    with that message.  The reference's explorer calls compile() without a
    policy and records a sample with code != 0 as failed
    (src/xtc/search/explore.py:415-427), so it never times a kernel other
    than the one the sample names;
  * "strict": compile() raises ScheduleError;
  * "nearest" (opt-in): the closest compiled instance in log2 distance,
    recorded as exact=False in the module's configs.
"""

from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import tempfile
import threading
from pathlib import Path
from typing import TYPE_CHECKING, Any

from ...itf.comp import Compiler
from ...runtimes.hip import capi
from ...utils.bf16 import itemsize
from .lowering import Launch, Plan
from .mapping import GemmConfig, SplitConfig, map_node
from .scheduler import HipSchedule, ScheduleError

if TYPE_CHECKING:
    from ...targets.hip.module import HipModule
    from .backend import HipBackend

__all__ = ["HipCompiler", "CompileService", "generate_payload"]

_DTYPE_ENUM = {"float32": "XTC_HIP_F32", "bfloat16": "XTC_HIP_BF16", "float64": "XTC_HIP_F64"}
# bytes of the operands and of the output/bias of a GEMM launch per operand dtype
_IN_BYTES = {"float32": 4, "bfloat16": 2, "float64": 8}
_OUT_BYTES = {"float32": 4, "bfloat16": 4, "float64": 8}
_cache_lock = threading.Lock()


def _cache_dir() -> Path:
    base = os.environ.get("XTC_AMD_CACHE") or os.path.join(tempfile.gettempdir(), f"xtc_amd-{os.getuid()}")
    path = Path(base) / "modules"
    path.mkdir(parents=True, exist_ok=True)
    return path


def _c_float(v: float) -> str:
    if v != v:
        return "(0.0f/0.0f)"
    if v in (float("inf"), float("-inf")):
        return "(1.0f/0.0f)" if v > 0 else "(-1.0f/0.0f)"
    return f"{float(v)!r}f"


def _c_double(v: float) -> str:
    """`v` as a C double literal: repr round-trips a Python float exactly."""
    if v != v:
        return "(0.0/0.0)"
    if v in (float("inf"), float("-inf")):
        return "(1.0/0.0)" if v > 0 else "(-1.0/0.0)"
    return f"{float(v)!r}"


def _ptr(plan: Plan, uid: str) -> str:
    b = plan.buffer(uid)
    if b.kind in ("input", "output"):
        return f"a{b.arg_index}"
    return f"(void *)(ws + {b.offset})"


def _c_string(text: str) -> str:
    """`text` as a C string literal (printable ASCII, escaped)."""
    out = []
    for ch in text:
        if ch in '\\"':
            out.append("\\" + ch)
        elif 32 <= ord(ch) < 127:
            out.append(ch)
        else:
            out.append(" ")
    return '"' + "".join(out) + '"'


def generate_payload(
    plan: Plan,
    configs: dict[str, GemmConfig | SplitConfig],
    payload: str,
    device: int,
    synchronize: bool = True,
    error: str | None = None,
) -> str:
    """C source of the payload for `plan` with the kernel instances `configs`.

    With `synchronize=False` the payload returns once its kernels are queued
    on the library stream (for back-to-back throughput measurement); the
    default waits for them, as XTC's wall-clock timing requires.  With
    `error` (a schedule that maps onto no kernel) the payload launches
    nothing and reports status 2 with that message."""
    nargs = len(plan.args)
    params = ", ".join(f"void *a{i}" for i in range(nargs)) or "void"
    out: list[str] = [
        "/* generated by xtc_amd.backends.hip.compiler */",
        "#include <stdint.h>",
        "#include <stdio.h>",
        '#include "xtc_hip.h"',
        "",
        "static int g_init = 0;",
        "static int g_status = 0;",
        "static char g_msg[1024];",
        "static void *g_ws = 0;",
        f"static const uint64_t g_ws_bytes = {plan.workspace_bytes}ull;",
        "",
        f"int {payload}_status(void) {{ return g_status; }}",
        f"const char *{payload}_message(void) {{ return g_msg; }}",
        f"void {payload}_release(void) {{ if (g_ws) {{ xtc_hip_free(g_ws); g_ws = 0; }} }}",
        "",
        "static void record(int rc, const char *where) {",
        "  g_status = rc;",
        '  snprintf(g_msg, sizeof(g_msg), "%s: %s", where, xtc_hip_last_error());',
        "}",
        "",
    ]
    if error is not None:
        out.append(f"void {payload}({params}) {{")
        for i in range(nargs):
            out.append(f"  (void)a{i};")
        out.append("  g_status = 2;")
        out.append(f'  snprintf(g_msg, sizeof(g_msg), "%s", {_c_string("schedule: " + error)});')
        out.append("}")
        return "\n".join(out) + "\n"
    body: list[str] = []
    for idx, ln in enumerate(plan.launches):
        body.extend(_emit_launch(plan, ln, configs.get(ln.node), idx))
    out.append(f"void {payload}({params}) {{")
    out.append("  int rc = 0;")
    out.append("  char *ws = 0;")
    out.append(f"  if (!g_init) {{ if ((rc = xtc_hip_init({device}))) {{ record(rc, \"init\"); return; }} g_init = 1; }}")
    out.append("  if (g_ws_bytes && !g_ws) {")
    out.append("    g_ws = xtc_hip_malloc(g_ws_bytes);")
    out.append('    if (!g_ws) { record(1, "workspace"); return; }')
    out.append("  }")
    out.append("  ws = (char *)g_ws;")
    out.append("  (void)ws;")
    out.extend(body)
    if synchronize:
        out.append('  if ((rc = xtc_hip_synchronize())) { record(rc, "synchronize"); return; }')
    out.append("  g_status = 0;")
    out.append("}")
    return "\n".join(out) + "\n"


def _emit_split_matmul(plan: Plan, ln: Launch, cfg: SplitConfig) -> list[str]:
    """One xtc_hip_matmul per piece, on the strided sub-views: rows m0.. of
    A (columns of A^T), columns n0.. of B (rows of B^T), the block of C at
    (m0, n0) and bias from n0; strides are the whole operands'."""
    a = ln.attrs
    M, N, K = a["M"], a["N"], a["K"]
    esz = _IN_BYTES[a["dtype"]]
    osz = _OUT_BYTES[a["dtype"]]
    ta, tb = bool(a.get("trans_a")), bool(a.get("trans_b"))
    lda, ldb = (M if ta else K), (K if tb else N)
    A, B = _ptr(plan, ln.inputs[0]), _ptr(plan, ln.inputs[1])
    C = _ptr(plan, ln.output)
    bias = _ptr(plan, a["bias"]) if a.get("bias") else None
    lines: list[str] = []
    for p in cfg.pieces:
        c = p.config
        a_off = p.m0 * esz if ta else p.m0 * lda * esz
        b_off = p.n0 * ldb * esz if tb else p.n0 * esz
        c_off = (p.m0 * N + p.n0) * osz
        tile = f"{{{c.bm}, {c.bn}, {c.bk}, {c.wgm}, {c.wgn}}}"
        lines.append(
            f"  {{ static const xtc_hip_matmul_desc d = {{{_DTYPE_ENUM[a['dtype']]}, {p.M}, {p.N}, {K}, "
            f"{lda}, {ldb}, {N}, {tile}, {c.split_k}, {c.group_m}, {c.xcd_remap}, {1 if a['relu'] else 0}, "
            f"{_c_float(a['threshold'])}, 0, {1 if ta else 0}, {1 if tb else 0}, {c.stages}, "
            f"{_c_double(a['threshold'])}}};"
        )
        bias_arg = f"(const void *)((const char *){bias} + {p.n0 * osz}ull)" if bias else "0"
        call = (f"xtc_hip_matmul(&d, (const char *){A} + {a_off}ull, (const char *){B} + {b_off}ull, "
                f"(void *)((char *){C} + {c_off}ull), {bias_arg})")
        where = f'"matmul {ln.node} rows {p.m0}+{p.M} cols {p.n0}+{p.N}"'
        lines.append(f"    if ((rc = {call})) {{ record(rc, {where}); return; }} }}")
    return lines


def _emit_launch(plan: Plan, ln: Launch, cfg: GemmConfig | SplitConfig | None, idx: int) -> list[str]:
    a = ln.attrs
    dst = _ptr(plan, ln.output)
    where = f'"{ln.kind} {ln.node}"'
    lines: list[str] = [f"  /* {ln.kind} {ln.node}{' + ' + ', '.join(ln.absorbed) if ln.absorbed else ''} */"]
    if isinstance(cfg, SplitConfig):
        assert ln.kind == "matmul"
        return lines + _emit_split_matmul(plan, ln, cfg)
    if ln.kind in ("matmul", "conv2d"):
        assert cfg is not None
        bias = _ptr(plan, a["bias"]) if a.get("bias") else "0"
        tile = f"{{{cfg.bm}, {cfg.bn}, {cfg.bk}, {cfg.wgm}, {cfg.wgn}}}"
        common = (
            f"{tile}, {cfg.split_k}, {cfg.group_m}, {cfg.xcd_remap}, "
            f"{1 if a['relu'] else 0}, {_c_float(a['threshold'])}, 0"
        )
        if ln.kind == "matmul":
            trans = (f", {1 if a.get('trans_a') else 0}, {1 if a.get('trans_b') else 0}, {cfg.stages}, "
                     f"{_c_double(a['threshold'])}")
            lines.append(
                f"  {{ static const xtc_hip_matmul_desc d = {{{_DTYPE_ENUM[a['dtype']]}, "
                f"{a['M']}, {a['N']}, {a['K']}, 0, 0, 0, {common}{trans}}};"
            )
            call = f"xtc_hip_matmul(&d, {_ptr(plan, ln.inputs[0])}, {_ptr(plan, ln.inputs[1])}, (void *){dst}, (const void *){bias})"
        else:
            pt, pb, pl, pr = a["pads"]
            lines.append(
                f"  {{ static const xtc_hip_conv2d_desc d = {{{_DTYPE_ENUM[a['dtype']]}, "
                f"{a['NB']}, {a['H']}, {a['W']}, {a['C']}, {a['F']}, {a['R']}, {a['S']}, "
                f"{a['stride'][0]}, {a['stride'][1]}, {pt}, {pb}, {pl}, {pr}, {_c_float(a['pad_value'])}, "
                f"{common}, {_c_double(a['threshold'])}, {_c_double(a['pad_value'])}}};"
            )
            call = f"xtc_hip_conv2d(&d, {_ptr(plan, ln.inputs[0])}, {_ptr(plan, ln.inputs[1])}, (void *){dst}, (const void *){bias})"
        lines.append(f"    if ((rc = {call})) {{ record(rc, {where}); return; }} }}")
    elif ln.kind == "relu":
        if a.get("dtype") == "float64":
            lines.append(
                f"  if ((rc = xtc_hip_relu_f64((const double *){_ptr(plan, ln.inputs[0])}, (double *){dst}, "
                f"{a['n']}ull, {_c_double(a['threshold'])}, 0))) {{ record(rc, {where}); return; }}"
            )
        else:
            lines.append(
                f"  if ((rc = xtc_hip_relu((const float *){_ptr(plan, ln.inputs[0])}, (float *){dst}, "
                f"{a['n']}ull, {_c_float(a['threshold'])}, 0))) {{ record(rc, {where}); return; }}"
            )
    elif ln.kind == "pad":
        nd = len(a["shape"])
        shape = ", ".join(str(d) for d in a["shape"])
        before = ", ".join(str(p[0]) for p in a["pads"])
        after = ", ".join(str(p[1]) for p in a["pads"])
        lines.append(f"  {{ static const int64_t s[{nd}] = {{{shape}}}, b[{nd}] = {{{before}}}, e[{nd}] = {{{after}}};")
        if a.get("dtype") == "float64":
            lines.append(
                f"    if ((rc = xtc_hip_pad_f64((const double *){_ptr(plan, ln.inputs[0])}, (double *){dst}, {nd}, s, "
                f"b, e, {_c_double(a['value'])}, 0))) {{ record(rc, {where}); return; }} }}"
            )
        else:
            lines.append(
                f"    if ((rc = xtc_hip_pad((const float *){_ptr(plan, ln.inputs[0])}, (float *){dst}, {nd}, s, b, e, "
                f"{_c_float(a['value'])}, 0))) {{ record(rc, {where}); return; }} }}"
            )
    elif ln.kind == "unpad":
        nd = len(a["shape"])
        shape = ", ".join(str(d) for d in a["shape"])
        before = ", ".join(str(p[0]) for p in a["pads"])
        after = ", ".join(str(p[1]) for p in a["pads"])
        lines.append(f"  {{ static const int64_t s[{nd}] = {{{shape}}}, b[{nd}] = {{{before}}}, e[{nd}] = {{{after}}};")
        lines.append(
            f"    if ((rc = xtc_hip_unpad({_ptr(plan, ln.inputs[0])}, {dst}, {a['elem']}, {nd}, s, b, e, 0))) "
            f"{{ record(rc, {where}); return; }} }}"
        )
    elif ln.kind == "cast":
        lines.append(
            f"  if ((rc = xtc_hip_cast_f32_to_bf16((const float *){_ptr(plan, ln.inputs[0])}, (uint16_t *){dst}, "
            f"{a['n']}ull, 0))) {{ record(rc, {where}); return; }}"
        )
    elif ln.kind == "copy":
        nbytes = plan.buffer(ln.output).nbytes
        lines.append(
            f"  if ((rc = xtc_hip_memcpy_d2d({dst}, {_ptr(plan, ln.inputs[0])}, {nbytes}ull))) "
            f"{{ record(rc, {where}); return; }}"
        )
    else:
        raise ScheduleError(f"no code generator for launch kind {ln.kind}")
    return lines


def _cc() -> str:
    return os.environ.get("CC") or shutil.which("gcc") or shutil.which("cc") or "cc"


class CompileService:
    """Runs the payloads' C compiler in worker processes of a fork server.

    A process that runs GPU work must not fork once its ROCm runtime has
    started: fork() copies a process whose runtime (and, with GPU counters,
    rocprofiler-sdk) threads may hold locks at that moment, and a fork
    handler or the child can then wait for a lock that no thread will ever
    release.  A compile that runs gcc through subprocess from a thread while
    another thread dispatches kernels does exactly that.  Inside
    `with CompileService(jobs):` build_shared_object hands its gcc run to
    workers that the fork server (a fresh interpreter started by this
    constructor, before any GPU work of the caller) forks from itself, so the
    calling process starts no process after this point.
    """

    _server_started = False

    def __init__(self, jobs: int = 1) -> None:
        import multiprocessing
        from concurrent.futures import ProcessPoolExecutor

        if not CompileService._server_started and capi.library_available() and capi.lib().xtc_hip_stream():
            raise RuntimeError(
                "CompileService: this process has already initialised the GPU (xtc_hip_init ran), so starting the "
                "compiler's fork server now would fork a process whose GPU runtime is up. Call "
                "CompileService.start_server() before the first GPU call (loop-explore's command line does), then "
                "run the exploration."
            )
        ctx = multiprocessing.get_context("forkserver")
        CompileService.start_server()  # the only process this one starts
        self._pool = ProcessPoolExecutor(max_workers=max(1, jobs), mp_context=ctx)
        self._previous: CompileService | None = None

    @staticmethod
    def start_server() -> None:
        """Starts the fork server now (idempotent): for programs that load
        the GPU libraries or register GPU tools before they build a
        CompileService.  A process that explores on the GPU from Python
        after its own GPU work must call this before that work."""
        from multiprocessing import forkserver

        forkserver.ensure_running()
        CompileService._server_started = True

    def build(self, source: str, out_path: Path | None, keep_dir: Path | None) -> Path:
        fut = self._pool.submit(
            _build_in_worker, source, str(out_path) if out_path else None, str(keep_dir) if keep_dir else None
        )
        return Path(fut.result())

    def close(self) -> None:
        self._pool.shutdown(wait=True)

    def __enter__(self) -> "CompileService":
        global _service
        self._previous, _service = _service, self
        return self

    def __exit__(self, *exc: Any) -> None:
        global _service
        _service = self._previous
        self.close()


_service: CompileService | None = None


def _build_in_worker(source: str, out_path: str | None, keep_dir: str | None) -> str:
    return str(build_shared_object(source, Path(out_path) if out_path else None, Path(keep_dir) if keep_dir else None))


def build_shared_object(source: str, out_path: Path | None, keep_dir: Path | None = None) -> Path:
    """Compiles `source` into a shared object linked to libxtc_hip.so.

    Objects are cached by content hash (atomic rename, so concurrent
    compilations of the same schedule are safe); `out_path` receives a copy.
    Inside a CompileService the compiler runs in its workers.
    """
    if _service is not None:
        return _service.build(source, out_path, keep_dir)
    lib = capi.LIB_PATH
    if not lib.exists():
        raise capi.HipError(f"{lib} is missing: build it with `python -m xtc_amd.csrc.build`")
    flags = ["-O2", "-std=c11", "-shared", "-fPIC", f"-I{capi.INCLUDE_PATH}"]
    link = [f"-L{lib.parent}", "-lxtc_hip", f"-Wl,-rpath,{lib.parent}"]
    key = hashlib.sha256("\0".join([source, *flags, *link, str(lib.stat().st_mtime_ns)]).encode()).hexdigest()[:24]
    cached = _cache_dir() / f"{key}.so"
    with _cache_lock:
        if not cached.exists():
            work = Path(tempfile.mkdtemp(prefix="xtc_hip_", dir=str(_cache_dir())))
            try:
                src = work / "payload.c"
                src.write_text(source)
                tmp = work / "payload.so"
                res = subprocess.run([_cc(), *flags, str(src), "-o", str(tmp), *link], capture_output=True, text=True)
                if res.returncode != 0:
                    raise RuntimeError(f"payload compilation failed:\n{res.stderr[-4000:]}\n--- source ---\n{source}")
                os.replace(tmp, cached)
            finally:
                shutil.rmtree(work, ignore_errors=True)
    if keep_dir is not None:
        # kept whether or not the object came from the cache
        keep_dir.mkdir(parents=True, exist_ok=True)
        (keep_dir / f"{key}.c").write_text(source)
    if out_path is None:
        return cached
    out_path.parent.mkdir(parents=True, exist_ok=True)
    tmp_out = out_path.with_name(out_path.name + f".tmp{os.getpid()}")
    shutil.copy(cached, tmp_out)
    os.replace(tmp_out, out_path)
    return out_path


class HipCompiler(Compiler):
    def __init__(self, backend: "HipBackend", **kwargs: Any) -> None:
        self._backend = backend
        target = kwargs.get("target")
        if target is not None and not (
            (isinstance(target, str) and target in ("hip", "rocm", "gfx950", "mi355x"))
            or getattr(target, "target_name", lambda: "")() == "hip"
        ):
            raise ValueError(f"HIP backend: unsupported target {target!r}")
        self._device = int(kwargs.get("selected_device", getattr(target, "device_id", lambda: 0)()))
        self._shared_lib = bool(kwargs.get("shared_lib", True))
        self._dump_file = kwargs.get("dump_file")
        # The payload takes bare device pointers whatever is asked: the
        # reference's explorer passes bare_ptr=False by default
        # (src/xtc/search/explore.py:98,368) and its MLIR compiler overrides
        # it to True the same way (src/xtc/backends/mlir/MlirCompiler.py:45)
        self._bare_ptr = True
        self._debug = bool(kwargs.get("debug", False))
        self._print_source = bool(kwargs.get("print_source_ir", False))
        self._save_temps = bool(kwargs.get("save_temps", False))
        self._save_temps_dir = kwargs.get("save_temps_dir")
        self._policy = kwargs.get("schedule_policy", "report")
        self._synchronize = bool(kwargs.get("synchronize", True))
        if self._policy not in ("report", "strict", "nearest"):
            raise ValueError(f"schedule_policy must be 'report', 'strict' or 'nearest', not {self._policy!r}")

    @property
    def backend(self) -> "HipBackend":
        return self._backend

    def kernel_configs(self, schedule: HipSchedule) -> dict[str, GemmConfig | SplitConfig]:
        """The kernel instance of every matmul/conv2d launch under `schedule`
        (one per segment for a matmul whose schedule splits i or j)."""
        policy = "nearest" if self._policy == "nearest" else "strict"
        configs: dict[str, GemmConfig | SplitConfig] = {}
        for ln in self._backend.plan.launches:
            if ln.kind in ("matmul", "conv2d"):
                configs[ln.node] = map_node(ln.attrs, ln.kind == "conv2d", schedule.node(ln.node), policy)
        return configs

    def check_fusions(self, schedule: HipSchedule) -> None:
        """fuse_producer_at(axis, input_idx) (src/xtc/itf/schd/scheduler.py:217-233)
        asks for the producer of a node input to be computed inside the node.
        The HIP backend fuses a pad/pad2d over H and W into conv2d input 0 (the
        implicit-GEMM and direct-conv loaders read the pad value outside the
        image); any other request is an error rather than silently ignored."""
        graph = self._backend.graph
        by_name = {n.name: n for uid, n in graph.nodes.items() if uid not in graph.inputs}
        absorbed = {ln.node: set(ln.absorbed) for ln in self._backend.plan.launches}
        for ns in schedule.schedule_impl:
            for loop, idx in ns.fused:
                node = by_name.get(ns.node_name)
                where = f"fuse_producer_at({loop!r}, {idx}) on {ns.node_name}"
                if node is None or not 0 <= idx < len(node.inputs):
                    raise ScheduleError(f"{where}: the node has no input {idx}")
                uid = node.inputs[idx]
                if uid in graph.inputs:
                    raise ScheduleError(f"{where}: input {idx} is a graph input, there is no producer to fuse")
                producer = graph.nodes[uid]
                if producer.name not in absorbed.get(ns.node_name, set()):
                    raise ScheduleError(
                        f"{where}: the HIP backend cannot fuse {producer.operation.name} {producer.name} there "
                        "(it fuses a pad/pad2d over H and W into conv2d input 0)"
                    )

    def compile(self, schedule: Any) -> "HipModule":
        from ...targets.hip.module import HipModule

        if not isinstance(schedule, HipSchedule):
            raise TypeError(f"HIP compiler needs a HipSchedule, got {type(schedule).__name__}")
        plan = self._backend.plan
        self.check_fusions(schedule)
        payload = self._backend.payload_name
        error = None
        try:
            configs = self.kernel_configs(schedule)
        except ScheduleError as err:
            if self._policy != "report":
                raise
            configs, error = {}, str(err)
        source = generate_payload(plan, configs, payload, self._device, self._synchronize, error)
        if self._print_source:
            print(source, flush=True)
        out = None
        if self._dump_file:
            out = Path(str(self._dump_file) + ".so")
        keep = None
        if self._save_temps:
            keep = Path(self._save_temps_dir or ".")
        path = build_shared_object(source, out, keep)
        if self._debug:
            for name, cfg in configs.items():
                print(f"[xtc_amd] {name}: {cfg.describe()}", flush=True)
        return HipModule(
            name=self._backend.graph.name or payload,
            payload_name=payload,
            file_name=str(path),
            graph=self._backend.graph,
            plan=plan,
            configs=configs,
            source=source,
            device=self._device,
            schedule_error=error,
        )
