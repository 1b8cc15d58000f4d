# SPDX-License-Identifier: BSD-3-Clause
"""The descript-spec search strategy (`loop-explore --descript`), on the CPU.

Golden vectors: the reference's strategy tests
(tests/filecheck/search/test_matmul_descript_*.py) print the sorted
constraint list of a spec on a 21x32x12 matmul and the number of distinct
samples that `sample(100)` returns; both are checked here for the same
specs.  The legal sets are also pinned by brute force over the parameters'
ranges, with the constraints evaluated independently of the solver."""

from __future__ import annotations

import itertools

import pytest

import xtc_amd.graphs.xtc.op as O
from xtc_amd.backends.hip import Backend
from xtc_amd.schedules.descript import check_constraints
from xtc_amd.schedules.exceptions import ScheduleValidationError
from xtc_amd.search.descript_strategy import Strategy_Descript


def _mm(i=21, j=32, k=12):
    a = O.tensor((i, k), "float32", name="A")
    b = O.tensor((k, j), "float32", name="B")
    with O.graph(name="matmul") as gb:
        O.matmul(a, b, name="C")
    return gb.graph


# (spec, extra constraints, expected sorted constraints, expected count of sample(100))
GOLDEN = {
    # test_matmul_descript_simple.py:12-27 (and test_matmul_descript_yaml_simple.py)
    "simple": ({"k": {}, "i": {}, "j": {}, "i#i1": {}, "j#j1": {}, "j#j2": {}}, [],
               ["i1 || {21}", "j1 || {32}", "j2 || {32, j1}"], 84),
    # test_matmul_descript_3axes.py:12-26
    "3axes": ({"j": {}, "k": {}, "i": {}, "j#jR": {}, "k#kR": {}, "i#iR": {}}, [],
              ["iR || {21}", "jR || {32}", "kR || {12}"], 100),
    # test_matmul_descript_goto.py:12-28
    "goto": ({"j": {"parallelize": "j_parallel"}, "k": {}, "i": {"pack": (1, None, True)},
              "j#jL3": {"pack": (0, None, True)}, "i#iL2": {}, "k#kL1": {"unroll": "k_unroll"},
              "i#iR": {"unroll": None}, "j#jR": {"vectorize": "j_vectorise"}}, ["iR * jR <= 56"],
             ["iL2 || {21}", "iR * jR <= 56", "iR || {21, iL2}", "jL3 || {32}", "jR || {32, jL3}",
              "j_parallel in {0, 1}", "j_vectorise in {0, 1}", "kL1 || {12}", "k_unroll || kL1"], 100),
    # test_matmul_descript_split.py:12-34
    "split": ({"j": {}, "k": {}, "i": {}, "i#iL3": {}, "i#7": {}, "j#jDDR": {},
               "i[:5]": {"i#iR1": {"unroll": None}, "j#jR1": {"parallelize": None}},
               "i[5:]": {"i#iR2": {"unroll": None}, "j#jR2": {"parallelize": None}}}, [],
              ["iL3 || {21}", "iR1 || {21, iL3, 7}", "iR2 || {21, iL3, 7}", "jDDR || {32}", "jR1 || {32, jDDR}",
               "jR2 || {32, jDDR}"], 100),
    # test_matmul_descript_split_in_split.py:12-37
    "split_in_split": ({"j": {}, "k": {}, "i": {}, "i#iL2": {}, "j#jDDR": {},
                        "i[:6]": {"i#3": {}, "i[:2:]": {"i#iR1": {"unroll": True}, "j#jR1": {"vectorize": True}},
                                  "i[:iS:]": {"i#iR3": {}, "j#jR3": {}}},
                        "i[6:]": {"i#iR2": {"unroll": True}, "j#jR2": {"vectorize": True}}}, [],
                       ["iL2 || {21}", "iR1 || {21, iL2, 3}", "iR2 || {21, iL2}", "iR3 || {21, iL2, 3}", "iS + 2 == 3",
                        "i_1_ + 6 == iL2", "i_1_ <= iL2", "jDDR || {32}", "jR1 || {32, jDDR}", "jR2 || {32, jDDR}",
                        "jR3 || {32, jDDR}"], 100),
    # test_matmul_descript_yaml_split.py:12-33
    "yaml_split": ("""
    j:
    k:
    i:
    i#iL3:
    i#iL2:
    j#jDDR:
    i[:iS]:
            i#iR1: unroll
            j#jR1: vectorize
            k#SR:
    i[iS:]:
            i#iR2: unroll
            j#jR2: unroll
""", [], ["SR || {12}", "iL2 || {21, iL3}", "iL3 || {21}", "iR1 || {21, iL3, iL2}", "iR2 || {21, iL3, iL2}",
          "iS <= iL2", "i_1_ + iS == iL2", "i_1_ <= iL2", "jDDR || {32}", "jR1 || {32, jDDR}", "jR2 || {32, jDDR}"],
        100),
}


@pytest.mark.parametrize("name", list(GOLDEN))
def test_reference_constraints_and_sample_counts(name):
    spec, extra, constraints, count = GOLDEN[name]
    s = Strategy_Descript(_mm(), spec, constraints=extra)
    assert sorted(s._constraints) == constraints
    xs = list(s.sample(100, seed=0))
    assert len(xs) == count and len({tuple(x) for x in xs}) == count
    for x in xs:
        check_constraints(constraints, s.sample_to_dict(x))


def _holds(constraints: list[str], env: dict[str, int]) -> bool:
    try:
        check_constraints(constraints, env)
        return True
    except ScheduleValidationError:
        return False


def _div(n: int) -> list[int]:
    return [d for d in range(1, n + 1) if n % d == 0]


def test_enumeration_equals_brute_force():
    """`simple`: every (i1, j1, j2) in 1..32^3 that satisfies the constraints;
    `goto`: every assignment of its tiles over the divisors of the sizes they
    divide (21, 32, 12) and of its switches over {0, 1}."""
    spec, extra, constraints, _ = GOLDEN["simple"]
    s = Strategy_Descript(_mm(), spec, constraints=extra)
    brute = {x for x in itertools.product(range(1, 33), repeat=3) if _holds(constraints, dict(zip(s.sample_names, x)))}
    assert {tuple(x) for x in s.exhaustive()} == brute
    # 4 divisors of 21, times the sum over j1 | 32 of the divisors of j1
    assert len(brute) == 4 * (1 + 2 + 3 + 4 + 5 + 6)

    spec, extra, constraints, _ = GOLDEN["goto"]
    s = Strategy_Descript(_mm(), spec, constraints=extra)
    ranges = {"iR": _div(21), "iL2": _div(21), "jR": _div(32), "jL3": _div(32), "kL1": _div(12), "k_unroll": _div(12),
              "j_parallel": [0, 1], "j_vectorise": [0, 1]}
    names = s.sample_names
    brute = {x for x in itertools.product(*(ranges[n] for n in names)) if _holds(constraints, dict(zip(names, x)))}
    assert {tuple(x) for x in s.exhaustive()} == brute and len(brute) > 1000


def test_split_in_split_count_in_closed_form():
    """iS + 2 == 3 fixes iS = 1; i_1_ + 6 == iL2 with i_1_ >= 1 leaves
    iL2 in {7, 21}; iR1, iR3 divide gcd(21, iL2, 3) and iR2 divides iL2;
    jR1..3 divide jDDR | 32.  So 2 * (1*1*2 + 2*2*4) / 2 ... written out:
    (iL2=7: 1*1*2) + (iL2=21: 2*2*4) = 18 i-choices, and
    sum over jDDR | 32 of d(jDDR)^3 = 1+8+27+64+125+216 = 441 j-choices."""
    spec, extra, constraints, _ = GOLDEN["split_in_split"]
    s = Strategy_Descript(_mm(), spec, constraints=extra)
    xs = [s.sample_to_dict(x) for x in s.exhaustive()]
    assert len(xs) == 18 * 441
    assert {x["iS"] for x in xs} == {1} and {(x["iL2"], x["i_1_"]) for x in xs} == {(7, 1), (21, 15)}


def test_partial_tile_goto_spec_samples_satisfy_its_constraints():
    """test_matmul_descript_yaml_goto.py: a 1024^3 matmul with partial tiles
    and the spec's own register/cache constraints; the space is too large to
    enumerate, so samples come from randomised draws."""
    spec = """
    constraints:
        - 1 + nvr + nvr * mr <= 32
        - nr == 16 * nvr
        - nvr * mr >= 8
        - nvr * mr * kr <= 256
        - kc * nr <= 8192
        - kc * mc <= 262144
        - kc * nc <= 9437184
    j:
    k:
    B: pack
    i:
    A: pack
    j#nc:
    i#mc:
    k#kc: unroll=kr
    i#mr: unroll full
    j#nr: vectorize full
"""
    s = Strategy_Descript(_mm(1024, 1024, 1024), spec, partial_tiles=True, partial_unrolls=True)
    assert sorted(s._constraints) == [
        "1 + nvr + nvr * mr <= 32", "kc * mc <= 262144", "kc * nc <= 9437184", "kc * nr <= 8192", "kc <= 1024",
        "kr <= kc", "mc <= 1024", "mr || {1024, mc}", "nc <= 1024", "nr == 16 * nvr", "nr || {1024, nc}",
        "nvr * mr * kr <= 256", "nvr * mr >= 8"]
    xs = list(s.sample(100, seed=0))
    assert len({tuple(x) for x in xs}) == 100
    for x in xs:
        env = s.sample_to_dict(x)
        # the constraints, restated as Python
        assert 1 + env["nvr"] + env["nvr"] * env["mr"] <= 32 and env["nr"] == 16 * env["nvr"]
        assert env["nvr"] * env["mr"] >= 8 and env["nvr"] * env["mr"] * env["kr"] <= 256
        assert env["kc"] * env["nr"] <= 8192 and env["kc"] * env["mc"] <= 262144 and env["kr"] <= env["kc"]
        assert 1024 % env["mr"] == 0 and env["mc"] % env["mr"] == 0 and env["nc"] % env["nr"] == 0
    assert list(s.sample(5, seed=3)) == list(s.sample(5, seed=3))


def test_samples_are_seeded_and_generate_schedules():
    spec, extra, _, _ = GOLDEN["split"]
    g = _mm()
    s = Strategy_Descript(g, spec, constraints=extra)
    assert list(s.sample(10, seed=1)) == list(s.sample(10, seed=1))
    assert list(s.sample(10, seed=1)) != list(s.sample(10, seed=2))
    # iL3 = 1 satisfies the constraints, but the fixed inner tile i#7 then
    # exceeds it and the nest is refused when applied, as in the reference
    x = next(x for x in s.exhaustive() if s.sample_to_dict(x)["iL3"] >= 7)
    sch = Backend(g).get_scheduler()
    s.generate(sch, x)
    env = s.sample_to_dict(x)
    node = sch.schedule().node("C")
    assert node.tiles["i"]["i0"] == env["iL3"] and node.tiles["j"]["j0"] == env["jDDR"]
    assert [seg.start for seg in node.segments] == [0, 5]
    # the split cuts each 7-row tile, which one launch per segment cannot do
    from xtc_amd.backends.hip.mapping import map_node
    from xtc_amd.backends.hip.scheduler import ScheduleError

    with pytest.raises(ScheduleError, match="inside its tiles"):
        map_node({"M": 21, "N": 32, "K": 12}, False, node, "strict")


def test_hip_filter_keeps_samples_that_map_to_compiled_kernels():
    """Through the explorer, the HIP legality filter keeps only samples whose
    tiles are compiled kernel instances."""
    from xtc_amd.backends.hip.mapping import map_node
    from xtc_amd.search.explore import hip_sample_filter

    g = _mm(512, 512, 512)
    spec = {"i": {}, "j": {}, "k": {}, "i#bm": {}, "j#bn": {}, "k#bk": {}, "i#wm": {}, "j#wn": {}}
    make = lambda **kw: Strategy_Descript(g, spec, **kw)  # noqa: E731
    s = make(sample_filter=hip_sample_filter(g, make))
    xs = list(s.sample(20, seed=0))
    assert 0 < len(xs) <= 20
    backend = Backend(g)
    for x in xs:
        sch = backend.get_scheduler()
        s.generate(sch, x)
        (ln,) = [l for l in backend.plan.launches if l.kind == "matmul"]
        map_node(ln.attrs, False, sch.schedule().node("C"), "strict")
    assert s.stats["filtered"] > 0


def test_reference_import_path_and_dict_samples():
    """The reference imports the strategy from xtc.search.strategies and
    applies dict samples (src/xtc/search/strategies.py:1031-1185)."""
    from xtc_amd.search.strategies import Strategy_Descript as S, Strategy_Descript_Explore

    assert S is Strategy_Descript and Strategy_Descript_Explore is Strategy_Descript
    spec, extra, _, _ = GOLDEN["simple"]
    g = _mm()
    s = S(g, spec, constraints=extra, initialize=False)
    x = s.default_schedule()
    a, b = Backend(g).get_scheduler(), Backend(g).get_scheduler()
    s.generate(a, x)
    s.generate(b, s.sample_to_dict(x))
    assert str(a.schedule()) == str(b.schedule())

