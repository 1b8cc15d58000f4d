# SPDX-License-Identifier: BSD-3-Clause
"""pad / pad2d / unpad around matmul and conv2d, against the reference's
padding tests (tests/filecheck/backends/padding/test_*.py).

tests/golden/padding_graph_prints.json holds, per reference test, the graph
print its FileCheck lines expect and whether its validated run ends with
`CODE: 0`, and the error backends/invalid/test_pad2d_invalid.py expects.  Each case here builds the same graph with xtc_amd's DSL (the
same calls and argument forms as the reference test), matches the print on
the CPU, checks the launch plan, and on the GPU compiles it with the
reference test's scheduler choice and runs the executor with validate=True
(np_init inputs, np.allclose against graph.forward): code 0, as the
reference's MLIR and TVM runs print.  The seeded GPU case compares the
pad -> matmul -> unpad output with the float64 oracle.
"""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import xtc_amd.graphs.xtc.op as O
from oracle import reference as R

ROOT = Path(__file__).resolve().parent.parent
_FIXTURE = json.loads((Path(__file__).parent / "golden" / "padding_graph_prints.json").read_text())
INVALID = _FIXTURE.pop("test_pad2d_invalid")["error"]
PRINTS = _FIXTURE

N, H, W, F, RR, S, C, SH, SW = 1, 8, 8, 16, 5, 5, 3, 2, 2
I_, J_, K_ = 14, 14, 14


def _conv(pad_call, frsc: bool = False):
    a = O.tensor((N, H, W, C), "float32", name="I")
    b = O.tensor((F, RR, S, C) if frsc else (RR, S, C, F), "float32", name="W")
    with O.graph(name="pad_conv2d_nhwc_mini") as gb:
        p = pad_call(a)
        w = O.transpose(b, axes=(1, 2, 3, 0)) if frsc else b
        O.conv2d(p, w, stride=(SH, SW), name="conv")
    return gb.graph


def _matmul(pad_a, pad_b, unpad_padding):
    a = O.tensor((I_, K_), "float32", name="A")
    b = O.tensor((K_, J_), "float32", name="B")
    with O.graph(name="pad_matmul_unpad") as gb:
        p1 = pad_a(a)
        p2 = pad_b(b)
        m = O.matmul(p1, p2, name="matmul_padded")
        O.unpad(m, padding=unpad_padding, name="C")
    return gb.graph


# reference test (without its _mlir / _tvm suffix) -> (graph builder, default_node of its scheduler)
BUILDERS = {
    "test_gen_pad_dict_conv2d": (lambda: _conv(lambda a: O.pad(a, padding={1: 2, 2: (2, 2)}, name="pad")), None),
    "test_gen_pad_int_matmul_unpad": (
        lambda: _matmul(lambda a: O.pad(a, padding=2, name="A_pad"), lambda b: O.pad(b, padding=2, name="B_pad"), 2),
        "matmul_padded",
    ),
    "test_gen_pad_tuple_conv2d": (lambda: _conv(lambda a: O.pad(a, padding=(0, 2, (2, 2), 0), name="pad")), None),
    "test_gen_pad_tuple_matmul_unpad": (
        lambda: _matmul(lambda a: O.pad(a, padding=(0, 2), name="A_pad"),
                        lambda b: O.pad(b, padding=(0, 2), name="B_pad"), (0, 2)),
        "matmul_padded",
    ),
    "test_pad2d_dict_matmul_unpad": (
        lambda: _matmul(lambda a: O.pad2d(a, padding={-2: (0, 2), -1: (0, 2)}, name="A_pad"),
                        lambda b: O.pad2d(b, padding=(0, 2), axes=(-2, -1), name="B_pad"),
                        {-2: (0, 2), -1: (0, 2)}),
        "matmul_padded",
    ),
    "test_pad_constant_conv2d": (
        lambda: _conv(lambda a: O.pad2d(a, padding=2, axes=(1, 2), constant_value=3, name="pad")), None),
    "test_pad_conv2d_frsc": (lambda: _conv(lambda a: O.pad2d(a, padding=2, axes=(1, 2), name="pad"), frsc=True), None),
    "test_pad_conv2d": (lambda: _conv(lambda a: O.pad2d(a, padding=2, axes=(1, 2), name="pad")), None),
    "test_pad_matmul_unpad": (
        lambda: _matmul(lambda a: O.pad2d(a, padding=(0, 2), axes=(-2, -1), name="A_pad"),
                        lambda b: O.pad2d(b, padding=(0, 2), axes=(-2, -1), name="B_pad"),
                        {-2: (0, 2), -1: (0, 2)}),
        "matmul_padded",
    ),
    "test_pad_tuple_matmul_unpad": (
        lambda: _matmul(lambda a: O.pad2d(a, padding=(0, 2, 0, 2), axes=(-2, -1), name="A_pad"),
                        lambda b: O.pad2d(b, padding=((0, 2), (0, 2)), axes=(-2, -1), name="B_pad"),
                        {-2: (0, 2), -1: (0, 2)}),
        "matmul_padded",
    ),
}
# transpose runs only on the reference's TVM backend (no MLIR variant of the
# test exists); this backend, like the MLIR one, has no standalone transpose
NOT_LOWERED = {"test_pad_conv2d_frsc"}


def _base(stem: str) -> str:
    return stem.rsplit("_", 1)[0]


def _match(output: str, patterns: list[str]) -> None:
    lines = [l.strip() for l in output.splitlines()]
    assert patterns[0] in lines, f"{patterns[0]!r} not in:\n{output}"
    i = lines.index(patterns[0])
    for j, pat in enumerate(patterns):
        assert i + j < len(lines) and pat in lines[i + j], f"line {j}: expected {pat!r} in:\n{output}"


def test_every_reference_padding_test_has_a_builder():
    assert {_base(k) for k in PRINTS} == set(BUILDERS)
    assert len(PRINTS) == 18 and all(v["code0"] for v in PRINTS.values())


def test_invalid_pad2d_padding_reports_the_reference_message():
    """backends/invalid/test_pad2d_invalid.py: a one-axis dict for pad2d.
    The reference fails an assert; this DSL raises ValueError with the same
    text."""
    exc_name, message = INVALID.split(": ", 1)
    assert exc_name == "AssertionError"
    a = O.tensor((I_, K_), "float32", name="A")
    with pytest.raises(ValueError) as info:
        with O.graph(name="pad_matmul_unpad"):
            O.pad2d(a, padding={-2: 2}, name="A_pad")
    assert str(info.value) == message


@pytest.fixture(scope="module")
def fresh_prints():
    """Each builder's print from a fresh interpreter: value ids count from
    %0 per process, as in the reference's one-process-per-test runs."""
    cache: dict[str, str] = {}

    def get(base: str) -> str:
        if base not in cache:
            code = ("import sys; sys.path.insert(0, 'tests'); from test_padding_graphs import BUILDERS; "
                    f"print(BUILDERS[{base!r}][0]())")
            res = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True, timeout=120)
            assert res.returncode == 0, res.stderr[-2000:]
            cache[base] = res.stdout
        return cache[base]

    return get


@pytest.mark.parametrize("stem", sorted(PRINTS))
def test_padding_graph_prints(stem, fresh_prints):
    _match(fresh_prints(_base(stem)), PRINTS[stem]["graph"])


@pytest.mark.parametrize("base", sorted(BUILDERS))
def test_padding_graph_plans(base):
    from xtc_amd.backends.hip.lowering import UnsupportedGraph, lower_graph

    build, _ = BUILDERS[base]
    g = build()
    if base in NOT_LOWERED:
        with pytest.raises(UnsupportedGraph, match="transpose"):
            lower_graph(g)
        return
    kinds = [ln.kind for ln in lower_graph(g).launches]
    if "conv2d" in base:
        assert kinds == ["conv2d"], kinds  # the pad over H and W is folded into the conv loader
    else:
        assert kinds == ["pad", "pad", "matmul", "unpad"], kinds
        un = lower_graph(g).launches[-1]
        expect = R.pad2d_padding(2, 2, axes=(0, 1)) if "int" in base else [(0, 2), (0, 2)]
        assert un.attrs["pads"] == expect and un.attrs["elem"] == 4 and tuple(un.attrs["shape"]) == (
            I_ + sum(expect[0]), J_ + sum(expect[1]))


@pytest.mark.gpu
@pytest.mark.parametrize("base", sorted(set(BUILDERS) - NOT_LOWERED))
def test_padding_graphs_execute_validated(base):
    """The reference test's own run: its scheduler choice, executor with
    validate=True on np_init inputs; it prints CODE: 0."""
    from xtc_amd.backends.hip import Backend

    build, node = BUILDERS[base]
    backend = Backend(build())
    sch = backend.get_scheduler(default_node=node) if node else backend.get_scheduler()
    module = backend.get_compiler(shared_lib=True).compile(sch.schedule())
    assert module.get_executor(validate=True).execute() == 0


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float32", "float64"])
def test_pad_matmul_unpad_seeded(dtype):
    """Seeded inputs through pad -> matmul -> unpad against the float64
    oracle: the crop keeps the 14x14 interior of the 17x17 product."""
    from xtc_amd.backends.hip import Backend

    rng = np.random.default_rng(11)
    x = rng.uniform(-1, 1, (I_, K_)).astype(dtype)
    y = rng.uniform(-1, 1, (K_, J_)).astype(dtype)
    a = O.tensor(x.shape, dtype, name="A")
    b = O.tensor(y.shape, dtype, name="B")
    with O.graph(name="pad_matmul_unpad_seeded") as gb:
        m = O.matmul(O.pad2d(a, padding=(1, 2), axes=(-2, -1)), O.pad2d(b, padding=(1, 2), axes=(-2, -1)))
        O.unpad(m, padding={-2: (1, 2), -1: (1, 2)}, name="C")
    backend = Backend(gb.graph)
    module = backend.get_compiler().compile(backend.get_scheduler().schedule())
    out = np.empty((I_, J_), dtype)
    _, code, msg = module.get_evaluator(parameters=([x, y], [out]), repeat=1, number=1, min_repeat_ms=0).evaluate()
    assert code == 0, msg
    pads = [(1, 2), (1, 2)]
    expect = R.unpad(R.matmul(R.pad(x.astype(np.float64), pads), R.pad(y.astype(np.float64), pads)), pads)
    tol = 1e-12 if dtype == "float64" else 1e-5
    assert np.max(np.abs(out - expect)) <= tol * np.max(np.abs(expect))


@pytest.mark.gpu
def test_unpad_of_a_bf16_output():
    """A bf16 matmul output (stored as 16-bit words after the cast kernel)
    cropped by unpad: the crop moves 2-byte elements; validate=True on
    np_init inputs compares with graph.forward, which rounds the same exact
    sums to bf16."""
    from xtc_amd.backends.hip import Backend
    from xtc_amd.backends.hip.lowering import lower_graph

    a = O.tensor((30, 64), "bfloat16", name="A")
    b = O.tensor((64, 48), "bfloat16", name="B")
    with O.graph(name="matmul_bf16_unpad") as gb:
        O.unpad(O.matmul(a, b, name="M"), padding={-2: (1, 3), -1: (2, 2)}, name="C")
    plan = lower_graph(gb.graph)
    assert [ln.kind for ln in plan.launches] == ["matmul", "cast", "unpad"] and plan.launches[-1].attrs["elem"] == 2
    backend = Backend(gb.graph)
    module = backend.get_compiler().compile(backend.get_scheduler().schedule())
    assert module.get_executor(validate=True).execute() == 0
