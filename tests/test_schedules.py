# SPDX-License-Identifier: BSD-3-Clause
"""Schedule description layer: loop nests, validation and descript specs.

tests/golden/schedule_prints.json holds the expected output (FileCheck
patterns, per prefix) of the reference's tests/filecheck/schedules/
test_descript_pretty_print.py, test_get_descript.py,
test_low_level_validation.py and test_descript_parsing_errors.py.  The same
specifications / scheduler calls are replayed here against xtc_amd's
descript module and the HIP scheduler.
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest

import xtc_amd.graphs.xtc.op as O
from xtc_amd.backends.hip import Backend
from xtc_amd.backends.hip.mapping import map_gemm
from xtc_amd.schedules.descript import (
    Descript,
    ScheduleInterpreter,
    ScheduleParser,
    YAMLParser,
    descript_scheduler,
    instantiate,
)
from xtc_amd.schedules.exceptions import ScheduleInterpretError, ScheduleParseError, ScheduleValidationError

PRINTS = json.loads((Path(__file__).parent / "golden" / "schedule_prints.json").read_text())


def _expect(file: str, prefix: str) -> list[str]:
    return [l.strip() for l in PRINTS[file][prefix]]


def _lines(text: str) -> list[str]:
    return [l.strip() for l in text.splitlines()]


def _matmul(i=4, j=32, k=512, dtype="float32"):
    a = O.tensor((i, k), dtype, name="A")
    b = O.tensor((k, j), dtype, name="B")
    with O.graph(name="matmul") as gb:
        O.matmul(a, b, name="C")
    return gb.graph


# ------------------------------------------------- descript -> loop nest prints

PRETTY = {
    "SIMPLE": {"i": {}, "k": {}, "j": {}},
    "TILED": {"i": {}, "k": {}, "j": {}, "j#16": {}},
    "VECTORIZED": {"i": {}, "k": {}, "j": {}, "j#16": {"vectorize": True}},
    "FULL": {"i": {"parallelize": True}, "k": {}, "j": {}, "j#32": {}, "j#16": {"vectorize": True, "unroll": 4}},
    "SPLIT": {"i": {}, "j[:128]": {"k": {}, "k#32": {}}, "j[128:]": {"k": {}, "k#16": {"vectorize": True}}},
    "BUFFER": {"i": {"parallelize": True}, "k": {"buffer": "default"}, "j": {"buffer": "shared"}, "j#16": {"vectorize": True}},
    "PACK": {"i": {"parallelize": True}, "k": {"pack": (0, "default", False)}, "j": {"pack": (1, "shared", True)},
             "j#16": {"vectorize": True}},
}


@pytest.mark.parametrize("prefix", sorted(PRETTY))
def test_descript_pretty_print(prefix):
    ast = ScheduleParser().parse(PRETTY[prefix])
    nest = ScheduleInterpreter(["i", "j", "k"]).interpret(ast, root="C")
    assert _lines(nest.root_node.pretty_print()) == _expect("test_descript_pretty_print", prefix)


def test_every_reference_pretty_print_case_is_replayed():
    assert set(PRETTY) == set(PRINTS["test_descript_pretty_print"])


# ------------------------------------------------- scheduler -> loop nest

def test_scheduler_loop_nest_prints():
    expect = _expect("test_get_descript", "MLIR")
    sep = expect.index("---")
    b = Backend(_matmul())
    sch = b.get_scheduler()
    sch.set_dims(["I", "J", "K"])
    sch.tile("I", {"I0": 2})
    sch.tile("J", {"J0": 16})
    sch.interchange(["K", "I", "J", "I0", "J0"])
    sch.unroll({"I0": 2})
    sch.vectorize(["J0"])
    assert _lines(sch.get_loop_nest().root_node.pretty_print()) == expect[:sep]

    sch2 = Backend(_matmul()).get_scheduler()
    sch2.set_dims(["I", "J", "K"])
    sch2.split("I", {"I_lo": 0, "I_hi": 2})
    sch2.tile("J", {"J0": 16}, root="./I_lo")
    sch2.tile("J", {"J0": 16}, root="./I_hi")
    sch2.interchange(["K", "I_lo", "I_hi"])
    sch2.interchange(["J", "J0"], root="./I_lo")
    sch2.interchange(["J", "J0"], root="./I_hi")
    assert _lines(sch2.get_loop_nest().root_node.pretty_print()) == expect[sep + 1:]


def _validation_case(name):
    sch = Backend(_matmul()).get_scheduler()
    sch.set_dims(["I", "J", "K"])
    if name == "VALID":
        sch.tile("I", {"I0": 2})
        sch.tile("J", {"J0": 16})
        sch.interchange(["K", "I", "J", "I0", "J0"])
        sch.vectorize(["J0"])
    elif name == "UNUSED-DIM":
        sch.tile("I", {"I0": 2})
        sch.interchange(["I", "J", "I0"])
    elif name == "VECT":
        sch.tile("I", {"I0": 2})
        sch.tile("J", {"J0": 16})
        sch.interchange(["K", "I", "J", "J0", "I0"])
        sch.vectorize(["J0"])
    elif name == "ORDER":
        sch.tile("I", {"I0": 2})
        sch.tile("J", {"J0": 16})
        sch.interchange(["K", "I0", "I", "J", "J0"])
    elif name == "SIZE":
        sch.tile("I", {"I0": 4})
        sch.tile("I", {"I00": 8})
        sch.tile("J", {"J0": 16})
        sch.interchange(["K", "I", "J", "I0", "I00", "J0"])
    return sch.get_loop_nest()


@pytest.mark.parametrize("name", ["VALID", "UNUSED-DIM", "VECT", "ORDER", "SIZE"])
def test_low_level_validation(name):
    (expect,) = _expect("test_low_level_validation", name)
    nest = _validation_case(name)
    if name == "VALID":
        nest.check()
        assert expect == "ok"
        return
    with pytest.raises(ScheduleValidationError) as err:
        nest.check()
    assert expect in " ".join(str(err.value).split())


# ------------------------------------------------- descript parse errors

@pytest.mark.parametrize("which", ["UNROLL", "PARALLELIZE", "VECTORIZE"])
def test_descript_parsing_errors(which):
    (expect,) = _expect("test_descript_parsing_errors", which)
    key = {"UNROLL": "K", "PARALLELIZE": "I", "VECTORIZE": "J"}[which]
    spec = {"I": {}, "K": {}, "J": {}}
    spec[key] = {which.lower(): ["hello"]}
    sch = Backend(_matmul()).get_scheduler()
    with pytest.raises(ScheduleParseError) as err:
        descript_scheduler(scheduler=sch, node_name="C", abstract_dims=["I", "J", "K"], spec=spec)
    assert str(err.value) == expect


def test_interpretation_errors():
    it = ScheduleInterpreter(["i", "j", "k"])
    p = ScheduleParser()
    with pytest.raises(ScheduleInterpretError, match="jumps from 10 to 12"):
        it.interpret(p.parse({"i[0:10]": {"j": {}}, "i[12:]": {"j": {}}}), "C")
    with pytest.raises(ScheduleInterpretError, match="not a defined axis"):
        it.interpret(p.parse({"q": {}}), "C")
    with pytest.raises(ScheduleInterpretError, match="strictly positive"):
        it.interpret(p.parse({"i": {}, "i#0": {}}), "C")
    with pytest.raises(ScheduleParseError, match="Unknown annotation"):
        p.parse({"i": {"fast": True}})


# ------------------------------------------------- descript on the HIP backend

def test_descript_drives_the_hip_kernel_choice():
    g = _matmul(8192, 8192, 8192, "bfloat16")
    b = Backend(g)
    sch = b.get_scheduler()
    descript_scheduler(
        scheduler=sch,
        node_name="C",
        abstract_dims=["i", "j", "k"],
        spec={"i": {"parallelize": True}, "j": {"parallelize": True}, "k": {},
              "i#256": {}, "j#256": {}, "k#64": {}, "i#128": {}, "j#64": {"vectorize": True}},
    )
    (ln,) = [l for l in b.plan.launches if l.kind == "matmul"]
    cfg = map_gemm(ln.attrs, False, sch.schedule().node("C"), "strict")
    assert cfg.tile == (256, 256, 64, 2, 4) and cfg.split_k == 1
    nest = sch.get_loop_nest()
    nest.check()
    assert _lines(nest.root_node.pretty_print())[:3] == ["loop i  // parallelized", "loop j  // parallelized", "loop k"]


def test_yaml_spec_equals_dict_spec():
    text = """
i: parallelize
k:
j:
j#32:
j#16: vectorize unroll=4
"""
    d = YAMLParser().parse(text)
    assert d == {"i": {"parallelize": None}, "k": {}, "j": {}, "j#32": {}, "j#16": {"vectorize": None, "unroll": 4}}
    a = Descript(["i", "j", "k"]).loop_nest("C", text).root_node.pretty_print()
    assert _lines(a) == _expect("test_descript_pretty_print", "FULL")
    # a size entry makes the key a tile
    assert YAMLParser().parse("j: {size: 16, vectorize: true}") == {"j#16": {"vectorize": True}}


def test_parameters_constraints_and_samples():
    desc = Descript(["i", "j", "k"], abstract_dim_sizes={"i": 64, "j": 64, "k": 64})
    spec = {"i": {}, "j": {}, "k": {}, "i#ti": {}, "k#tk": {"unroll": "u"}, "j#tj": {"vectorize": "v"}}
    nest = desc.loop_nest("C", spec)
    assert "ti || {64}" in nest.constraints and "v in {0, 1}" in nest.constraints and "u || tk" in nest.constraints
    concrete = instantiate(nest, {"ti": 16, "tj": 8, "tk": 32, "v": 1, "u": 4})
    node = concrete.root_node
    assert node.tiles["i"] == {"i0": 16} and node.tiles["j"] == {"j0": 8} and node.unroll == {"k0": 4}
    assert node.vectorize == ["j0"]
    assert instantiate(nest, {"ti": 16, "tj": 8, "tk": 32, "v": 0, "u": 4}).root_node.vectorize == []
    with pytest.raises(ScheduleValidationError, match="does not hold"):
        instantiate(nest, {"ti": 5, "tj": 8, "tk": 32, "v": 1, "u": 4})  # 5 does not divide 64
    with pytest.raises(ScheduleValidationError, match="no value"):
        instantiate(nest, {"ti": 16})
    # the sample reaches the scheduler
    g = _matmul(64, 64, 64)
    sch = Backend(g).get_scheduler()
    descript_scheduler(sch, "C", ["i", "j", "k"], spec, abstract_dim_sizes={"i": 64, "j": 64, "k": 64},
                       sample={"ti": 16, "tj": 8, "tk": 32, "v": 1, "u": 4})
    (s,) = sch.schedule().schedule_impl
    assert s.tiles == {"i": {"i0": 16}, "j": {"j0": 8}, "k": {"k0": 32}} and s.vectorization == ["./j0"]


def test_split_segments_reach_the_scheduler():
    sch = Backend(_matmul(50, 64, 64)).get_scheduler()
    descript_scheduler(
        sch, "C", ["i", "j", "k"],
        {"k": {}, "i": {}, "i#10": {}, "i[0:5]": {"i#5": {}, "j": {}}, "i[5:]": {"i#5": {}, "j": {}}},
    )
    nest = sch.get_loop_nest()
    text = _lines(nest.root_node.pretty_print())
    assert text[:3] == ["loop k", "loop i", "tile(i, 10)"]
    assert "split(i, 0, 5)" in text and "split(i, 5, ...)" in text
