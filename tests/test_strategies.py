# SPDX-License-Identifier: BSD-3-Clause
"""Search spaces against the reference's golden transcripts.

tests/golden/strategy_transcripts.json holds, for each of the reference's
strategy tests (tests/filecheck/search/test_*.py), the strategy, its
arguments, the graph and the expected default schedules (O0-O3), sample
sequences (exhaustive prefix or seeded random draw) and filter statistics.
Replaying them pins the enumeration order, the filters and the seeded
sampling stream, which loop-explore results depend on.
"""

from __future__ import annotations

import json
from itertools import islice
from pathlib import Path

import pytest

import xtc_amd.graphs.xtc.op as O
from xtc_amd.search import strategies as S
from xtc_amd.utils.math import divisors_list, factors_enumeration, factors_to_sizes, sizes_to_factors

TRANSCRIPTS = json.loads((Path(__file__).parent / "golden" / "strategy_transcripts.json").read_text())


def _graph(kind):
    if kind == "matmul":
        a = O.tensor((21, 12), "float32")
        b = O.tensor((12, 32), "float32")
        with O.graph(name="matmul") as gb:
            O.matmul(a, b)
        return gb.graph
    B, H, W, F, R, Sz, C = 2, 4, 4, 32, 7, 7, 3
    a = O.tensor((B, H + R - 1, W + Sz - 1, C), "float32")
    w = O.tensor((R, Sz, C, F), "float32")
    with O.graph(name="matmul") as gb:
        O.conv2d(a, w, stride=(2, 2))
    return gb.graph


@pytest.mark.parametrize("name", sorted(TRANSCRIPTS))
def test_transcript(name):
    rec = TRANSCRIPTS[name]
    strategy = getattr(S, rec["strategy"])(_graph(rec["graph"]), **rec["kwargs"])
    for call, args in rec["calls"]:
        if call == "print_all_opt_schedules":
            for level, expect in rec["defaults"].items():
                assert strategy.default_schedule(int(level)) == expect, f"O{level}"
        elif call == "print_exhaustive_samples":
            got = list(islice(strategy.exhaustive(), args[0]))
            assert got == rec["samples"]
            assert dict(strategy.stats) == rec["stats"]
        elif call == "print_random_samples":
            got = list(strategy.sample(num=args[0]))
            assert got == rec["samples"]
            assert dict(strategy.stats) == rec["stats"]


def test_math_helpers_documented_examples():
    # examples stated in src/xtc/utils/math.py docstrings
    assert divisors_list(112) == [1, 2, 4, 7, 8, 14, 16, 28, 56, 112]
    assert factors_enumeration(97, 2) == [[1, 1], [1, 97], [97, 1]]
    assert factors_enumeration(28, 2)[:8] == [[1, 1], [1, 2], [1, 4], [1, 7], [1, 14], [1, 28], [2, 1], [2, 2]]
    assert len(factors_enumeration(28, 2)) == 18
    assert factors_to_sizes([4, 1, 2, 2]) == [16, 4, 4, 2]
    assert sizes_to_factors([16, 4, 4, 2]) == [4, 1, 2, 2]
    for n in (1, 12, 360, 8192):
        for f in factors_enumeration(n, 3):
            assert n % (f[0] * f[1] * f[2]) == 0


def test_registry_names_and_aliases():
    assert S.Strategies.resolve_name("tile7dvr") == "tile_pprprp_vr"
    assert S.Strategies.from_name("tile4d") is S.Strategy_P1
    with pytest.raises(ValueError):
        S.Strategies.registration("nope")
    g = _graph("matmul")
    st = S.Strategies.create("tile_oo", g, max_unroll=8)
    assert st.sample_names == ["x0", "x1", "x2"]


def test_generate_records_schedule():
    from xtc_amd.backends.hip import Backend

    g = _graph("matmul")
    st = S.Strategy_PPRPRP(g, max_unroll=8, threads=4)
    # P P R P R P: i and j get three tile levels, k one
    assert st.sample_names == [f"x{i}" for i in range(7)]
    sch = Backend(g).get_scheduler()
    # factors outer->inner: i (1, 3, 7), j (2, 8, 2), k (3)
    st.generate(sch, [1, 3, 7, 2, 8, 2, 3])
    (s,) = sch.schedule().schedule_impl
    assert s.tiles["i"] == {"i1": 21, "i2": 21, "i3": 7}
    assert s.tiles["j"] == {"j1": 32, "j2": 16, "j3": 2}
    assert s.tiles["k"] == {"k1": 3}
    assert s.permutation["."] == ["./" + a for a in ["i", "j", "i1", "j1", "k", "i2", "j2", "k1", "i3", "j3"]]
    assert s.parallelization == ["./i", "./j"]
    assert s.vectorization == ["./j3"]


def test_sample_filter_extension():
    g = _graph("matmul")
    keep = lambda x: x[0] == 3  # noqa: E731
    st = S.Strategy_OO(g, max_unroll=8, sample_filter=keep)
    assert all(x[0] == 3 for x in st.exhaustive())
    assert all(x[0] == 3 for x in st.sample(5, seed=1))
