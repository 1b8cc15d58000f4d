# SPDX-License-Identifier: BSD-3-Clause
"""Graph DSL and operator semantics against the reference's graph tests.

tests/golden/graph_prints.json holds the expected output (FileCheck patterns)
of each of the reference's tests/filecheck/graphs/test_*.py.  Each case here
builds the same graph with xtc_amd's DSL, runs the same prints and matches
them line by line.  The "Outputs:" lines also pin the oracle: the oracle's
float64 restatement of the same graph, formatted the same way, must print
the reference's values.
"""

from __future__ import annotations

import json
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import xtc_amd.graphs.xtc.op as O
import xtc_amd.graphs.xtc.ty as T
from oracle import reference as R
from xtc_amd.utils.numpy import np_init

ROOT = Path(__file__).resolve().parent.parent
PRINTS = json.loads((Path(__file__).parent / "golden" / "graph_prints.json").read_text())


def _match(output: str, patterns: list[str]) -> None:
    """FileCheck semantics for a CHECK followed by CHECK-NEXTs: the first
    pattern is found on some line, each next one on the line after; leading
    and trailing whitespace is not significant."""
    lines = [l.strip() for l in output.splitlines()]
    starts = [i for i, l in enumerate(lines) if patterns[0] in l]
    assert starts, f"first pattern {patterns[0]!r} not found in:\n{output}"
    i = starts[0]
    for j, pat in enumerate(patterns):
        assert i + j < len(lines), f"output ended before pattern {j}: {pat!r}"
        assert pat in lines[i + j], f"line {i + j}: expected {pat!r}, got {lines[i + j]!r}"


def _inputs(types):
    return [T.Tensor(np_init(t.constant_shape, t.constant_dtype) - 5) for t in types]


def _run_matmul() -> str:
    x, y = O.tensor(), O.tensor()
    with O.graph(name="matmul") as gb:
        O.matmul(x, y)
    g = gb.graph
    print(g)
    types = [T.TensorType((5, 3), "float32"), T.TensorType((3, 4), "float32")]
    print(g.forward_types(types))
    inps = _inputs(types)
    print(f"Inputs: {inps}")
    print(f"Outputs: {g.forward(inps)}")


def _run_matmul_relu() -> None:
    x, y = O.tensor(), O.tensor()
    with O.graph(name="matmul_relu") as gb:
        O.relu(O.matmul(x, y))
    g = gb.graph
    print(g)
    types = [T.TensorType((5, 3), "float32"), T.TensorType((3, 4), "float32")]
    print(f"outputs: {g.forward_types(types)}")
    print(g)
    inps = _inputs(types)
    print(f"Inputs: {inps}")
    print(f"Outputs: {g.forward(inps)}")


def _run_relu() -> None:
    x = O.tensor()
    with O.graph(name="relu") as gb:
        O.relu(x)
    g = gb.graph
    print(g)
    types = [T.TensorType((1, 5, 6), "float32")]
    print(g.forward_types(types))
    inps = _inputs(types)
    print(f"Inputs: {inps}")
    print(f"Outputs: {g.forward(inps)}")


def _run_conv_relu() -> None:
    i, k = O.tensor(), O.tensor()
    with O.graph(name="conv_relu") as gb:
        p = O.pad2d(i, padding=2, axes=(1, 2))
        t = O.transpose(k, axes=(1, 2, 3, 0))
        O.relu(O.conv2d(p, t, stride=(2, 2)), threshold=0.1)
    g = gb.graph
    print(g)
    types = [T.TensorType((2, 6, 6, 3), "float32"), T.TensorType((8, 5, 5, 3), "float32")]
    g.forward_types(types)
    print(g)
    inps = _inputs(types)
    print(f"Inputs: {inps}")
    print(f"Outputs: {g.forward(inps)}")


def _mlp_weights():
    size = 32 * 32 * 3
    return [(1, size), (size, 512), (512, 256), (256, 128), (128, 10)]


def _run_mlp() -> None:
    img, w1, w2, w3, w4 = (O.tensor(shape=s, dtype="float32") for s in _mlp_weights())
    with O.graph(name="mlp4") as gb:
        with O.graph(name="l1"):
            l1 = O.relu(O.matmul(img, w1))
        with O.graph(name="l2"):
            l2 = O.relu(O.matmul(l1, w2))
        with O.graph(name="l3"):
            l3 = O.relu(O.matmul(l2, w3))
        with O.graph(name="l4"):
            O.matmul(l3, w4)
    g = gb.graph
    print(g)
    inps = _inputs([n.forward_types([])[0] for n in g.inputs_nodes])
    print(f"Inputs: {inps}")
    print(f"Outputs: {g.forward(inps)}")


def _run_mlp_fc() -> None:
    img, w1, w2, w3, w4 = (O.tensor() for _ in range(5))

    def fc(i, w, nout):
        return O.matmul(O.reshape(i, shape=(1, -1)), O.reshape(w, shape=(-1, nout)))

    with O.graph(name="mlp4") as gb:
        with O.graph(name="l1"):
            l1 = O.relu(fc(img, w1, 512))
        with O.graph(name="l2"):
            l2 = O.relu(fc(l1, w2, 256))
        with O.graph(name="l3"):
            l3 = O.relu(fc(l2, w3, 128))
        with O.graph(name="l4"):
            l4 = fc(l3, w4, 10)
        O.reshape(l4, shape=(-1,))
    g = gb.graph
    print(g)
    shapes = [(32, 32, 3)] + _mlp_weights()[1:]
    types = [T.TensorType(s, "float32") for s in shapes]
    print(g.forward_types(types))
    inps = _inputs(types)
    print(f"Inputs: {inps}")
    print(f"Outputs: {g.forward(inps)}")


def _run_subgraphs() -> None:
    x, y = O.tensor(), O.tensor()
    with O.graph(name="matmul_relu") as mrb:
        with O.graph(name="matmul") as mb:
            z = O.matmul(x, y)
        with O.graph(name="relu") as rb:
            O.relu(z)
    print(mrb.graph)
    print(mb.graph)
    print(rb.graph)


CASES = {
    "test_matmul": _run_matmul,
    "test_matmul_relu": _run_matmul_relu,
    "test_relu": _run_relu,
    "test_conv_relu": _run_conv_relu,
    "test_mlp": _run_mlp,
    "test_mlp_fc": _run_mlp_fc,
    "test_subgraphs": _run_subgraphs,
}


def test_every_reference_graph_test_is_replayed():
    assert set(CASES) == set(PRINTS)


@pytest.mark.parametrize("name", sorted(CASES))
def test_reference_graph_transcript(name):
    # Node ids (%0, %1, ...) number from 0 in each process, and each of the
    # reference's tests is one process: so is each case here.
    code = f"import tests.test_graphs as t; t.CASES[{name!r}]()"
    res = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    _match(res.stdout, PRINTS[name])


def _outputs_line(name: str) -> str:
    (line,) = [l for l in PRINTS[name] if l.startswith("Outputs:")]
    return line


def _oracle_line(arr: np.ndarray) -> str:
    return f"Outputs: {[T.Tensor(np.asarray(arr, dtype=np.float32))]}"


def _oracle_inputs(shapes):
    return [np_init(s, "float32").astype(np.float64) - 5 for s in shapes]


def test_oracle_matmul_matches_reference_print():
    a, b = _oracle_inputs([(5, 3), (3, 4)])
    assert _oracle_line(R.matmul(a, b)) == _outputs_line("test_matmul")
    assert _oracle_line(R.relu(R.matmul(a, b))) == _outputs_line("test_matmul_relu")


def test_oracle_relu_matches_reference_print():
    (x,) = _oracle_inputs([(1, 5, 6)])
    assert _oracle_line(R.relu(x)) == _outputs_line("test_relu")


def test_oracle_conv_relu_matches_reference_print():
    x, k = _oracle_inputs([(2, 6, 6, 3), (8, 5, 5, 3)])
    p = R.pad(x, R.pad2d_padding(4, 2, axes=(1, 2)))
    w = np.transpose(k, (1, 2, 3, 0))
    out = R.relu(R.conv2d(p, w, stride=(2, 2)), threshold=0.1)
    assert out.shape == (2, 3, 3, 8)
    assert _oracle_line(out) == _outputs_line("test_conv_relu")
    np.testing.assert_array_equal(R.conv2d(p, w, (2, 2)), R.conv2d_direct(p, w, (2, 2)))


def test_oracle_mlp_matches_reference_print():
    xs = _oracle_inputs(_mlp_weights())
    h = xs[0]
    for w in xs[1:4]:
        h = R.relu(R.matmul(h, w))
    out = R.matmul(h, xs[4])
    assert _oracle_line(out) == _outputs_line("test_mlp")
    # the fc form flattens a 32x32x3 image into the same row
    img = np_init((32, 32, 3), "float32").astype(np.float64) - 5
    assert _oracle_line(out.reshape(-1)) == _outputs_line("test_mlp_fc")
    np.testing.assert_array_equal(img.reshape(1, -1), xs[0])


def test_forward_types_and_ops_count():
    a = O.tensor((64, 32), "float32")
    b = O.tensor((32, 16), "float32")
    with O.graph(name="mm") as gb:
        O.relu(O.matmul(a, b))
    g = gb.graph
    assert [str(t) for t in g.outputs_types] == ["64x16xfloat32"]
    # per node: the product of its iteration space (operation.py:76-81), i.e.
    # i*j*k multiply-accumulates for the matmul and one op per relu element
    assert g.ops_count() == 64 * 16 * 32 + 64 * 16
    assert g.ops_dtype() == "float32"


def test_graph_yaml_round_trip(tmp_path):
    i = O.tensor((2, 6, 6, 3), "float32", name="I")
    k = O.tensor((8, 5, 5, 3), "float32", name="K")
    with O.graph(name="conv_relu") as gb:
        p = O.pad2d(i, padding=2, axes=(1, 2))
        t = O.transpose(k, axes=(1, 2, 3, 0))
        O.relu(O.conv2d(p, t, stride=(2, 2)), threshold=0.1)
    g = gb.graph
    path = tmp_path / "g.yaml"
    g.dump(str(path))
    with O.graph() as gb2:
        O.graph.load(str(path))
    g2 = gb2.graph

    def canon(text: str) -> str:
        # a loaded graph gets fresh ids: compare up to a renaming of %N
        ids: dict[str, str] = {}
        return re.sub(r"%\d+", lambda m: ids.setdefault(m.group(0), f"%{len(ids)}"), text)

    assert canon(str(g2)) == canon(str(g))
    inps = _inputs([T.TensorType((2, 6, 6, 3), "float32"), T.TensorType((8, 5, 5, 3), "float32")])
    np.testing.assert_array_equal(g2.forward(inps)[0].numpy(), g.forward(inps)[0].numpy())


# The reference's own graph files (tests/graphs/*.graph.yaml, loaded by
# tests/pytest/graphs/test_graph_serialization.py:8-19), kept as data.
REF_GRAPHS = Path(__file__).resolve().parent / "golden" / "graphs"


@pytest.mark.parametrize("opname,ins,outs", [
    ("matmul", ["512x128xfloat32", "128x1024xfloat32"], ["512x1024xfloat32"]),
    ("conv2d", ["1x230x230x3xfloat32", "7x7x3x64xfloat32"], ["1x112x112x64xfloat32"]),
])
def test_reference_graph_files_load_and_compile(opname, ins, outs):
    import yaml

    from xtc_amd.backends.hip import Backend

    path = REF_GRAPHS / f"{opname}.graph.yaml"
    with O.graph() as gb:
        gb.load(path)
    graph = gb.graph
    assert graph.name == opname
    assert [str(t) for t in graph.inputs_types] == ins and [str(t) for t in graph.outputs_types] == outs
    # the same document back, but for the digest of the operator classes
    # (ops_version hashes the registering module's names)
    data = yaml.safe_load(path.read_text())
    mine = graph.to_dict()
    assert {k: v for k, v in mine.items() if k != "ops_version"} == {k: v for k, v in data.items() if k != "ops_version"}
    with O.graph() as gb2:
        gb2.loads(graph.dumps())
    assert gb2.graph.to_dict() == mine
    backend = Backend(graph)
    module = backend.get_compiler().compile(backend.get_scheduler().schedule())
    assert module.schedule_error is None and len(module.configs) == 1
