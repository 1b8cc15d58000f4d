# SPDX-License-Identifier: BSD-3-Clause
"""The reference's unit tests (tests/pytest/unit/*, tests/pytest/graphs/),
replayed on this package's restatements: the sample-space estimators and
unique sampling of the search, the result callbacks, the compile/execute
pipeline, the NDArray runtime type, the interface modules and graph
serialization.  The input/expected values are the reference tests' own;
the test code is this package's.
"""

from __future__ import annotations

import csv
import time
from itertools import islice
from pathlib import Path
from types import SimpleNamespace as NS

import numpy as np
import pytest

from xtc_amd.utils.algorithms import sample_uniques
from xtc_amd.utils.math import (
    estimate_count_prob_smooth,
    estimate_unique_num_chao1,
    estimate_unique_prob_good_turing,
)

RTOL, ATOL = 1e-3, 1e-6


def _close(got: float, want: float) -> bool:
    return abs(got - want) <= RTOL * want + ATOL


# ---------------------------------------------------- unit/math/test_estimates.py

# (count, samples, kwargs, expected): additive smoothing
@pytest.mark.parametrize("count,samples,kw,want", [
    (0, 0, {}, 1), (0, 1, {}, 1 / 2), (1, 1, {}, 1), (1, 10, {}, 2 / 11), (1, 100, {}, 2 / 101),
    (10, 10, {}, 1), (10, 100, {}, 11 / 101), (10, 1000, {}, 11 / 1001),
    (0, 0, {"alpha": 0}, 0), (0, 1, {"alpha": 0}, 0), (0, 0, {"alpha": 2}, 1), (0, 1, {"alpha": 2}, 2 / 3),
])
def test_estimate_count_prob_smooth(count, samples, kw, want):
    assert _close(estimate_count_prob_smooth(count, samples, **kw), want)


# (samples, seen once, expected): probability that the next draw is new
@pytest.mark.parametrize("samples,once,want", [
    (0, 0, 1), (1, 0, 1 / 2), (10, 1, 2 / 11), (100, 1, 2 / 101), (1000, 1, 2 / 1001),
    (10, 10, 1), (100, 10, 11 / 101), (1000, 10, 11 / 1001),
])
def test_estimate_unique_prob_good_turing(samples, once, want):
    assert _close(estimate_unique_prob_good_turing(samples, once), want)


# (uniques, seen once, seen twice, expected richness)
@pytest.mark.parametrize("uniques,once,twice,want", [
    (0, 0, 0, 0), (1, 0, 0, 1), (100, 0, 0, 100), (1, 1, 0, 1), (2, 1, 1, 2), (2, 2, 0, 3), (3, 2, 1, 4),
    (9, 8, 1, 23), (100, 8, 1, 114),
])
def test_estimate_unique_num_chao1(uniques, once, twice, want):
    assert estimate_unique_num_chao1(uniques, once, twice) == want


def test_estimators_reject_impossible_counts():
    with pytest.raises(ValueError):
        estimate_count_prob_smooth(3, 2)
    with pytest.raises(ValueError):
        estimate_unique_prob_good_turing(2, 3)
    with pytest.raises(ValueError):
        estimate_unique_num_chao1(2, 2, 1)


# ------------------------------------------- unit/algorithms/test_sample_uniques.py

def _sampler(stream: list):
    """A draw function over a fixed stream: up to n items per call, None
    standing for a draw that produced no valid sample."""
    it = iter(stream)

    def draw(n: int):
        return [s for s in islice(it, n) if s is not None]

    return draw


# (stream, requested, expected count, kwargs)
@pytest.mark.parametrize("stream,num,want,kw", [
    ([], 100, 0, {}),
    ([None] * 100 + [1], 100, 1, {}),
    ([None] * 100 + [1], 100, 0, {"prob": 1 / 100}),
    ([None] * 5000 + [1], 100, 0, {}),
    ([None] * 5000 + [1], 100, 1, {"prob": 1 / 10000}),
    ([None] * 100 + [1] + [None] * 100 + [2] + [None] * 100 + [3], 100, 3, {}),
    ([1] * 101 + [None] * 100 + [2] + [None] * 100 + [3], 100, 3, {}),
    ([None] * 100 + [1] + [None] * 100 + [1] + [None] * 100 + [2], 100, 2, {}),
    ([None] * 100 + [1], 1, 1, {}),
    ([None] * 100 + [1] + [None] * 100 + [2], 2, 2, {}),
])
def test_sample_uniques(stream, num, want, kw):
    got = sample_uniques(_sampler(stream), num, **kw)
    assert len(got) == want and len(set(got)) == len(got)


# --------------------------------------- unit/cli/test_explore_csv_callback.py

def _rows(path: Path) -> list[list[str]]:
    with path.open(newline="") as f:
        return list(csv.reader(f))


def _existing(path: Path, row: list) -> None:
    with path.open("w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["M", "N", "X", "time", "peak", "backend"])
        w.writerow(row)


def test_csv_callback_resume_skips_recorded_pairs(tmp_path):
    from xtc_amd.search.callback import CSVCallback

    out = tmp_path / "r.csv"
    _existing(out, [8, 16, "[8; 16]", 2.0, 0.5, "mlir"])
    cb = CSVCallback(str(out), peak_time=1.0, sample_names=["M", "N"], resume=True)
    cb(([8, 16], 0, 3.0, "mlir"))  # already in the file for this backend
    cb(([8, 16], 0, 2.5, "tvm"))  # another backend
    cb(([8, 32], 0, 3.0, "mlir"))  # another sample
    cb.close()
    rows = _rows(out)
    assert rows[0] == ["M", "N", "X", "time", "peak", "backend"] and len(rows) == 4
    assert rows[1][-3:] == ["2.0", "0.5", "mlir"]
    assert rows[2][:2] == ["8", "16"] and rows[2][-3:] == ["2.5", "0.4", "tvm"]
    assert rows[3][:2] == ["8", "32"] and rows[3][-1] == "mlir"


def test_csv_callback_default_rewrites_and_skips_failures(tmp_path):
    from xtc_amd.search.callback import CSVCallback

    out = tmp_path / "r.csv"
    _existing(out, [9, 9, "[9; 9]", 8.0, 0.25, "mlir"])
    cb = CSVCallback(str(out), peak_time=2.0, sample_names=["M", "N"])
    cb(([2, 3], 0, 6.0, "mlir"))
    cb(([4, 4], 2, 0.0, "mlir"))  # a failed sample is not written
    cb.close()
    rows = _rows(out)
    assert len(rows) == 2 and rows[1][:2] == ["2", "3"] and rows[1][-1] == "mlir"


def test_csv_callback_append(tmp_path):
    from xtc_amd.search.callback import CSVCallback

    out = tmp_path / "r.csv"
    _existing(out, [4, 4, "[4; 4]", 10.0, 0.1, "mlir"])
    cb = CSVCallback(str(out), peak_time=1.0, sample_names=["M", "N"], append=True)
    cb(([4, 4], 0, 1.6, "mlir"))  # duplicates are kept in append mode
    cb.close()
    rows = _rows(out)
    assert len(rows) == 3 and rows[1][:2] == rows[2][:2] == ["4", "4"]
    fresh = tmp_path / "new.csv"
    cb = CSVCallback(str(fresh), peak_time=2.0, sample_names=["M", "N"], append=True)
    cb(([2, 3], 0, 8.0, "mlir"))
    cb.close()
    assert _rows(fresh) == [["M", "N", "X", "time", "peak", "backend"], ["2", "3", "[2; 3]", "8.0", "0.25", "mlir"]]


def test_memory_and_db_callbacks(tmp_path):
    import json

    import xtc_amd.graphs.xtc.op as O
    from xtc_amd.search.callback import DBCallback, MemoryCallback

    mem = MemoryCallback()
    mem(([1, 2], 0, 1e-3, "hip"))
    assert mem.results == [([1, 2], 0, 1e-3, "hip")]
    a, b = O.tensor((4, 4), "float32"), O.tensor((4, 4), "float32")
    with O.graph(name="mm") as gb:
        O.matmul(a, b)
    db = DBCallback(str(tmp_path / "db.jsonl"), "gfx950", 1, "tile_hip")
    db.set_graph(gb.graph)
    db(([1, 2], 0, 1e-3, "hip"))
    db(([3, 4], 2, 5.0, "hip"))  # a failed sample records time 0
    recs = [json.loads(line) for line in open(tmp_path / "db.jsonl")]
    assert [r["results"] for r in recs] == [[0, [1e-3]], [2, [0.0]]]
    assert recs[0]["compiler"][-3:] == ["gfx950", 1, "hip"] and recs[0]["operator"][0] == "xtc.graph"
    assert recs[0]["version"] == ["v0.2"] and recs[0]["strategy"][2] == "tile_hip"


# --------------------------------------------------- unit/search/test_pipeline.py

def _compile(p):
    assert p.input == f"Input {p.id}"
    time.sleep(0.01)
    return NS(id=p.id, compiled=f"Compiled {p.id}")


def _execute(c):
    assert c.compiled == f"Compiled {c.id}"
    time.sleep(0.02)
    return NS(id=c.id, executed=f"Executed {c.id}")


@pytest.mark.parametrize("compile_jobs,execute_jobs,ntasks", [(1, 1, 4), (0, 0, 4), (3, 4, 11)])
def test_pipeline_order_and_results(compile_jobs, execute_jobs, ntasks):
    from xtc_amd.search.pipeline import CompileExecutePipeline

    pipe = CompileExecutePipeline(compile_func=_compile, execute_func=_execute, compile_jobs=compile_jobs,
                                  execute_jobs=execute_jobs)
    tasks = pipe.run(NS(id=i, input=f"Input {i}") for i in range(ntasks))
    assert [t.id for t in tasks] == list(range(ntasks))
    assert all(t.comp_result.compiled == f"Compiled {t.id}" for t in tasks)
    assert all(t.exec_result.executed == f"Executed {t.id}" for t in tasks)
    assert all(t.comp_time > 0 and t.exec_time > 0 and t.exec_stamp >= t.comp_stamp + t.comp_time for t in tasks)


def test_pipeline_compiles_ahead_of_execution():
    """With one execute job, task k+1 is compiled while task k executes."""
    from xtc_amd.search.pipeline import CompileExecutePipeline

    tasks = CompileExecutePipeline(_compile, _execute, compile_jobs=2, execute_jobs=1).run(
        NS(id=i, input=f"Input {i}") for i in range(6))
    overlapped = [t.id for t, nxt in zip(tasks, tasks[1:]) if nxt.comp_stamp < t.exec_stamp + t.exec_time]
    assert len(overlapped) >= 4, overlapped


def test_pipeline_raises_at_the_failing_task():
    from xtc_amd.search.pipeline import CompileExecutePipeline

    def bad(p):
        if p == 2:
            raise RuntimeError("no kernel for 2")
        return p

    gen = CompileExecutePipeline(bad, lambda c: c, compile_jobs=2).generate(range(5))
    assert [next(gen).id, next(gen).id] == [0, 1]
    with pytest.raises(RuntimeError, match="no kernel for 2"):
        next(gen)


# ------------------------------------------------- unit/runtimes/test_ndarray.py

def test_ndarray_aligned_host_copy():
    from xtc_amd.runtimes.types.ndarray import NDArray

    try:
        NDArray.set_alloc_alignment(2 * 1024 * 1024)
        x = np.arange(100 * 200).reshape(100, 200).astype("float32")
        a = NDArray(x)
        assert (a.dims, a.shape, a.dtype, a.size) == (2, (100, 200), np.dtype("float32"), 20000)
        assert a.data % (2 * 1024 * 1024) == 0 and not a.is_on_device()
        assert np.array_equal(a.numpy(), x)
    finally:
        NDArray.set_alloc_alignment(256)


def test_ndarray_layout_and_copies():
    from xtc_amd.runtimes.types.ndarray import NDArray

    x = np.arange(6.0).reshape(2, 3)
    t = NDArray(x, layout=[1, 0])
    assert t.shape == (3, 2) and t.is_transposed() and np.array_equal(t.numpy(), x)
    t.copy_from_numpy(x + 1)
    assert np.array_equal(t.numpy(), x + 1)
    out = np.empty((2, 3), np.float64)
    plain = NDArray(x)
    assert plain.numpy(out=out) is out and np.array_equal(out, x)
    with pytest.raises(ValueError):
        NDArray(np.zeros(3, dtype=np.float16))
    with pytest.raises(ValueError):
        NDArray.set_alloc_alignment(3)
    with pytest.raises(ValueError):
        t.copy_from_numpy(np.zeros((3, 2)))


# ------------------------------------------------------ unit/itf/test_abstract.py

def test_interface_modules():
    from xtc_amd.itf.back.backend import Backend
    from xtc_amd.itf.comp.compiler import Compiler
    from xtc_amd.itf.data.tensor import Tensor, TensorType
    from xtc_amd.itf.graph.graph import Graph
    from xtc_amd.itf.graph.node import Node
    from xtc_amd.itf.operator.operator import Operator
    from xtc_amd.itf.schd.schedule import Schedule
    from xtc_amd.itf.schd.scheduler import Scheduler

    from xtc_amd.itf.exec.evaluator import Evaluator
    from xtc_amd.itf.exec.executor import Executor
    from xtc_amd.itf.search.optimizer import Optimizer
    from xtc_amd.itf.search.strategy import Strategy

    for abc in (Backend, Compiler, Tensor, TensorType, Graph, Node, Operator, Schedule, Scheduler, Evaluator,
                Executor, Strategy, Optimizer):
        with pytest.raises(TypeError):
            abc()


# ------------------------------------------- pytest/graphs/test_graph_serialization.py

def test_graph_serialization_round_trips(tmp_path):
    import xtc_amd.graphs.xtc.op as O

    golden = Path(__file__).parent / "golden" / "graphs"
    for name in ("matmul", "conv2d"):
        with O.graph() as gb:
            gb.load(golden / f"{name}.graph.yaml")
        assert gb.graph.name == name
    # dict, string and file round trips
    a, b = O.tensor((4, 512), "float32", name="A"), O.tensor((512, 32), "float32", name="B")
    with O.graph(name="matmul_relu") as gb:
        O.relu(O.matmul(a, b, name="matmul"), name="relu")
    d = gb.graph.to_dict()
    with O.graph() as gb2:
        gb2.from_dict(d)
    assert d and d == gb2.graph.to_dict()
    i, w = O.tensor((1, 8, 8, 3), "float32", name="I"), O.tensor((5, 5, 3, 16), "float32", name="W")
    with O.graph(name="pad_conv2d_nhwc_mini") as gb:
        O.conv2d(O.pad(i, padding={1: 2, 2: (2, 2)}, name="pad"), w, stride=(2, 2), name="conv")
    text = gb.graph.dumps()
    with O.graph(name="other") as gb2:
        gb2.loads(text)
    assert text and text == gb2.graph.dumps()
    gb.graph.dump(str(tmp_path / "g.yaml"))
    with O.graph() as gb3:
        gb3.load(str(tmp_path / "g.yaml"))
    assert gb.graph.to_dict() == gb3.graph.to_dict()
    # nested subgraphs and an output chosen by the user survive the dict form
    ts = [O.tensor() for _ in range(5)]

    def fc(x, wt, n):
        return O.matmul(O.reshape(x, shape=(1, -1)), O.reshape(wt, shape=(-1, n)))

    with O.graph(name="mlp4") as gb:
        with O.graph(name="l1"):
            l1 = O.relu(fc(ts[0], ts[1], 512))
        with O.graph(name="l2"):
            l2 = O.relu(fc(l1, ts[2], 256))
        with O.graph(name="l3"):
            l3 = O.relu(fc(l2, ts[3], 128))
        with O.graph(name="l4"):
            l4 = fc(l3, ts[4], 10)
        O.reshape(l4, shape=(-1,))
        O.outputs(l1)
    d = gb.graph.to_dict()
    with O.graph() as gb2:
        gb2.from_dict(d)
    assert d and d == gb2.graph.to_dict()
