# SPDX-License-Identifier: BSD-3-Clause
"""loop-explore driver on the CPU: graphs of the CLI, the CSV/DB/manifest
outputs, resume, and the HIP legality filter.  Evaluation is replaced by a
stub (no GPU here); compilation runs for real."""

from __future__ import annotations

import csv
import json

import numpy as np
import pytest

from xtc_amd.backends.hip import Backend
from xtc_amd.backends.hip.mapping import map_gemm
from xtc_amd.cli.explore import DEFAULT_DIMS, build_graph
from xtc_amd.search.explore import Exploration, ExplorationConfig, hip_sample_filter, parse_x
from xtc_amd.search.strategies import Strategies


def test_cli_graphs_follow_the_reference_shapes():
    g = build_graph("conv2d", DEFAULT_DIMS["conv2d"], "float32")
    # input (n, h*SH + r - 1, w*SW + s - 1, c) (explore.py:253)
    assert [str(t) for t in g.inputs_types] == ["1x230x230x3xfloat32", "7x7x3x64xfloat32"]
    assert [str(t) for t in g.outputs_types] == ["1x112x112x64xfloat32"]
    g = build_graph("conv2d", [8, 56, 56, 64, 3, 3, 64, 1, 1], "float32", pad=1)
    assert [str(t) for t in g.inputs_types][0] == "8x56x56x64xfloat32"
    assert [str(t) for t in g.outputs_types] == ["8x56x56x64xfloat32"]
    g = build_graph("matmul", [16, 8192, 8192], "bfloat16")
    assert [str(t) for t in g.outputs_types] == ["16x8192xfloat32"]
    assert build_graph("relu", [1024], "float32").ops_count() == 1024


def test_bf16_graphs_count_and_peak_in_their_operand_dtype(monkeypatch):
    # a bf16 matmul or conv that stores fp32 computes in bf16: its ops dtype,
    # hence the peak the explorer divides by, is bfloat16, and a pad2d in
    # front of a bf16 conv is counted together with the conv, as the
    # reference counts every node of the first node's dtype (graph.py:190-205)
    g = build_graph("matmul", [16, 8192, 8192], "bfloat16")
    assert g.ops_dtype() == "bfloat16" and g.ops_count() == 16 * 8192 * 8192
    g = build_graph("conv2d", [1, 8, 8, 64, 3, 3, 64, 1, 1], "bfloat16", pad=1)
    assert g.ops_dtype() == "bfloat16" and g.ops_count() == 8 * 8 * 64 * 9 * 64 + 10 * 10 * 64
    seen = []

    class _Dev:
        def evaluate_flops(self, dtype):
            seen.append(dtype)
            return 1e15

    import xtc_amd.runtimes.hip.device as device

    monkeypatch.setattr(device, "HipDevice", _Dev)
    ex = Exploration(build_graph("matmul", [8192, 8192, 8192], "bfloat16"), ExplorationConfig())
    assert ex.peak_time() == pytest.approx(8192**3 / 1e15) and seen == ["bfloat16"]


def _stub(monkeypatch, calls):
    def evaluate_one(self, module):
        calls.append(module.configs)
        return [2e-3, 1e-3], 0, ""

    monkeypatch.setattr(Exploration, "evaluate_one", evaluate_one)


def test_run_writes_csv_db_manifest_and_resumes(tmp_path, monkeypatch):
    calls = []
    _stub(monkeypatch, calls)
    g = build_graph("matmul", [512, 512, 512], "float32")
    out = tmp_path / "r.csv"
    cfg = ExplorationConfig(trials=5, seed=3, output=str(out), db_file=str(tmp_path / "r.jsonl"),
                            peak_flops=1e12, jobs=2)
    res = Exploration(g, cfg).run()
    assert len(res) == 5 and all(code == 0 for _, _, code, _ in res)
    rows = list(csv.DictReader(open(out)))
    assert list(rows[0]) == ["bm", "wm", "bn", "wn", "bk", "split_k", "stages", "X", "time", "peak", "backend"]
    assert len(rows) == 5 and all(float(r["time"]) == 1e-3 for r in rows)
    # peak = ops_count / peak_flops / time
    assert float(rows[0]["peak"]) == pytest.approx(512**3 / 1e12 / 1e-3)
    assert all(r["X"].count(";") == 6 and "," not in r["X"] for r in rows)
    db = [json.loads(l) for l in open(tmp_path / "r.jsonl")]
    assert len(db) == 5 and all(d["kernels"]["C"].startswith("gemm<float32>") for d in db)
    # results-DB record of the reference (callback.py:46-60, query_results.py:78-123)
    d = db[0]
    assert d["version"] == ["v0.2"] and d["results"] == [0, [1e-3]]
    assert d["compiler"][0] == "xtc" and d["compiler"][2:] == ["gfx950", 1, "hip"]
    assert d["operator"][0] == "xtc.graph" and len(d["operator"][1]) == 40 and "name" not in d["operator"][2]
    assert d["strategy"][0] == "xtc.strategy" and d["strategy"][2] == "tile_hip"
    assert [x["schedule"] for x in db] == [parse_x(r["X"]) for r in rows]
    meta = json.loads((tmp_path / "r.csv.meta.json").read_text())
    assert meta["sampleNames"] == ["bm", "wm", "bn", "wn", "bk", "split_k", "stages"] and meta["args"]["trials"] == 5
    # every sampled schedule compiled to exactly the kernel it names, at the
    # pipeline depth it names (0 in the config = the kernel's default depth)
    from xtc_amd.backends.hip.mapping import pipeline_depths

    (ln,) = Backend(g).plan.launches
    for sample, conf in zip([parse_x(r["X"]) for r in rows], calls):
        (c,) = conf.values()
        bm, wm, bn, wn, bk, sk, st = sample
        assert (c.bm, c.bn, c.bk, c.bm // c.wgm, c.bn // c.wgn, c.split_k, c.exact) == (bm, bn, bk, wm, wn, sk, True)
        default = pipeline_depths(ln.attrs, False, c.tile, sk)[0]
        assert c.stages == (0 if st == default else st)
    # resume: the same samples are not run again
    calls.clear()
    cfg.resume = True
    Exploration(g, cfg).run()
    assert calls == [] and len(list(csv.DictReader(open(out)))) == 5
    # data search replays the CSV's samples
    cfg2 = ExplorationConfig(search="data", data=str(out), output=str(tmp_path / "d.csv"), peak_flops=1e12)
    assert sorted(map(tuple, Exploration(g, cfg2).samples())) == sorted(tuple(parse_x(r["X"])) for r in rows)


def test_failed_sample_is_recorded_not_written(tmp_path, monkeypatch):
    def evaluate_one(self, module):
        return [], 1, "validation failed"

    monkeypatch.setattr(Exploration, "evaluate_one", evaluate_one)
    g = build_graph("matmul", [256, 256, 256], "float32")
    cfg = ExplorationConfig(trials=2, output=str(tmp_path / "f.csv"), db_file=str(tmp_path / "f.jsonl"), peak_flops=1e12)
    res = Exploration(g, cfg).run()
    assert [code for _, _, code, _ in res] == [1, 1]
    assert list(csv.DictReader(open(tmp_path / "f.csv"))) == []
    recs = [json.loads(l) for l in open(tmp_path / "f.jsonl")]
    assert [r["error"] for r in recs] == ["validation failed"] * 2
    assert [r["results"] for r in recs] == [[1, [0.0]]] * 2


def test_cpu_strategy_samples_are_filtered_to_compiled_kernels():
    g = build_graph("matmul", [1024, 1024, 1024], "float32")
    # the CLI's HIP default unroll bound; 256 (the CPU default) excludes every GPU-sized tile
    ok = hip_sample_filter(g, lambda: Strategies.create("tile_oo", g, max_unroll=1 << 22))
    st = Strategies.create("tile_oo", g, max_unroll=1 << 22, sample_filter=ok)
    samples = list(st.sample(8, seed=0))
    assert len(samples) == 8
    from xtc_amd.backends.hip import Backend

    for x in samples:
        b = Backend(g)
        sch = b.get_scheduler()
        st.generate(sch, list(x))
        (ln,) = b.plan.launches
        assert map_gemm(ln.attrs, False, sch.schedule().node(ln.node), "strict").exact


def test_tile_hip_conv_points_map_exactly():
    from xtc_amd.backends.hip import Backend

    g = build_graph("conv2d", [8, 56, 56, 64, 3, 3, 64, 1, 1], "float32", pad=1)
    st = Strategies.create("tile_hip", g)
    points = list(st.exhaustive())
    assert len(points) > 10 and all(p[5] == 1 for p in points)
    for x in points:
        b = Backend(g)
        sch = b.get_scheduler()
        st.generate(sch, list(x))
        (ln,) = [l for l in b.plan.launches if l.kind == "conv2d"]
        cfg = map_gemm(ln.attrs, True, sch.schedule().node(ln.node), "strict")
        assert (cfg.bm, cfg.bm // cfg.wgm, cfg.bn, cfg.bn // cfg.wgn, cfg.bk) == tuple(x[:5])
    # the default point is the library's own choice
    assert st.default_schedule(2)[5] >= 1


def test_pmu_counters_are_split_from_the_times(tmp_path, monkeypatch):
    # with counters the evaluator returns repeat x counters values, repeat by
    # repeat in counter order; the CSV time is the min of the gpu.time ones
    # (added first when not requested) and the DB record keeps every counter
    seen = []

    def evaluate_one(self, module):
        seen.append(self.counters())
        #        repeat 0           repeat 1
        return [3e-3, 256.0, 9.0, 2e-3, 256.0, 7.0], 0, ""

    monkeypatch.setattr(Exploration, "evaluate_one", evaluate_one)
    g = build_graph("matmul", [256, 256, 256], "float32")
    cfg = ExplorationConfig(trials=2, seed=1, output=str(tmp_path / "p.csv"), db_file=str(tmp_path / "p.jsonl"),
                            peak_flops=1e12, pmu_counters=["gpu.SQ_WAVES", "gpu.cycles"], jobs=1)
    res = Exploration(g, cfg).run()
    assert seen == [["gpu.time", "gpu.SQ_WAVES", "gpu.cycles"]] * 2
    assert [t for _, t, _, _ in res] == [[3e-3, 2e-3]] * 2
    rows = list(csv.DictReader(open(tmp_path / "p.csv")))
    assert [float(r["time"]) for r in rows] == [2e-3, 2e-3]
    recs = [json.loads(l) for l in open(tmp_path / "p.jsonl")]
    assert recs[0]["results"] == [0, [2e-3]]
    assert recs[0]["counters"] == {"gpu.time": [3e-3, 2e-3], "gpu.SQ_WAVES": [256.0, 256.0], "gpu.cycles": [9.0, 7.0]}
    # no counters requested: plain timing, values untouched
    cfg.pmu_counters = []
    ex = Exploration(g, cfg)
    assert ex.counters() == [] and ex.split_counters([1.0, 2.0]) == ([1.0, 2.0], {})
    # gpu.time requested explicitly keeps its place
    cfg.pmu_counters = ["gpu.cycles", "gpu.time"]
    assert Exploration(g, cfg).split_counters([5.0, 1e-3, 6.0, 2e-3]) == (
        [1e-3, 2e-3], {"gpu.cycles": [5.0, 6.0], "gpu.time": [1e-3, 2e-3]})


# ---------------------------------------------------------------- no fork after the GPU starts

def test_no_process_starts_after_the_device(tmp_path, monkeypatch):
    # A fake device: evaluation "starts the GPU runtime" on first use.  Every
    # way this process could start another one (fork, posix_spawn, the
    # fork_exec behind subprocess and multiprocessing) is recorded together
    # with whether the device had started; compilation must still happen.
    import _posixsubprocess
    import os

    from xtc_amd.runtimes.hip.device import HipDevice

    state = {"gpu": False}
    spawns = []

    def fake_init(self):
        state["gpu"] = True

    def evaluate_one(self, module):
        HipDevice(0).init_device()
        assert os.path.exists(module.file_name)
        return [1e-3], 0, ""

    def record(name, real):
        def wrapper(*a, **k):
            spawns.append((name, state["gpu"]))
            return real(*a, **k)

        return wrapper

    monkeypatch.setattr(HipDevice, "init_device", fake_init)
    monkeypatch.setattr(Exploration, "evaluate_one", evaluate_one)
    monkeypatch.setattr(_posixsubprocess, "fork_exec", record("fork_exec", _posixsubprocess.fork_exec))
    monkeypatch.setattr(os, "fork", record("fork", os.fork))
    monkeypatch.setattr(os, "posix_spawn", record("posix_spawn", os.posix_spawn))
    g = build_graph("matmul", [384, 384, 384], "float32")
    for search in ("random", "iterative"):
        cfg = ExplorationConfig(search=search, trials=6, batch=2, optimizer="random", seed=5,
                                output=str(tmp_path / f"{search}.csv"), peak_flops=1e12, jobs=3)
        res = Exploration(g, cfg).run()
        assert len(res) == 6 and all(code == 0 for _, _, code, _ in res), res
        assert state["gpu"]
        assert not [s for s in spawns if s[1]], spawns
        state["gpu"] = False
    # the recorder sees what subprocess starts in this process
    import subprocess

    subprocess.run(["true"], check=True)
    assert ("fork_exec", False) in spawns


# ---------------------------------------------------------------- iterative search and optimizers

def test_iterative_search_records_every_batch(tmp_path, monkeypatch):
    times = {}

    def evaluate_one(self, module):
        (c,) = module.configs.values()
        # larger tiles "run faster": a smooth objective for the forest
        t = 1e-3 / (c.bm * c.bn)
        times[(c.bm, c.bn)] = t
        return [t], 0, ""

    monkeypatch.setattr(Exploration, "evaluate_one", evaluate_one)
    g = build_graph("matmul", [1024, 1024, 1024], "float32")
    cfg = ExplorationConfig(search="iterative", trials=7, batch=3, optimizer="random-forest-default", seed=1,
                            output=str(tmp_path / "it.csv"), db_file=str(tmp_path / "it.jsonl"), peak_flops=1e12,
                            jobs=2)
    res = Exploration(g, cfg).run()
    assert len(res) == 7 and all(code == 0 for _, _, code, _ in res)
    assert len([json.loads(l) for l in open(tmp_path / "it.jsonl")]) == 7
    rows = list(csv.DictReader(open(tmp_path / "it.csv")))
    assert 1 <= len(rows) <= 7  # repeated proposals are written once


def test_iterative_tile_hip_search_starts_from_the_library_default(tmp_path, monkeypatch):
    # tile_hip puts the library's own schedule in the first batch, so the
    # search never ends below it; the reference's strategies do not
    _stub(monkeypatch, [])
    g = build_graph("matmul", [1024, 1024, 1024], "float32")
    cfg = ExplorationConfig(search="iterative", strategy="tile_hip", trials=5, batch=3, seed=2, peak_flops=1e12,
                            output=str(tmp_path / "h.csv"), jobs=1)
    ex = Exploration(g, cfg)
    res = ex.run()
    assert len(res) == 5 and res[0][0] == list(ex.strategy.default_schedule(2))
    ex2 = Exploration(g, ExplorationConfig(search="iterative", strategy="tile_oo", trials=3, batch=3, seed=2,
                                           peak_flops=1e12, output=str(tmp_path / "o.csv"), jobs=1))
    assert not getattr(ex2.strategy, "starts_from_default", False)
    assert len(ex2.run()) == 3


def _grid_sampler(n, seed):
    import numpy as np

    rng = np.random.default_rng(seed)
    for _ in range(n):
        yield [int(v) for v in rng.integers(0, 16, size=2)]


def test_random_optimizer_draws_one_seed_per_batch():
    import random

    from xtc_amd.search.optimizers import Optimizers

    opt = Optimizers.from_name("random")(_grid_sampler, 4, 7)
    r = random.Random(7)
    for _ in range(3):
        assert opt.suggest() == list(_grid_sampler(4, r.randint(0, 2**32 - 1)))


def test_random_forest_optimizer_protocol_and_convergence(tmp_path):
    import random

    from xtc_amd.search.optimizers import Optimizers

    def peak(x):  # fraction of peak, best at (11, 4)
        return 1.0 / (1.0 + (x[0] - 11) ** 2 + (x[1] - 4) ** 2)

    make = Optimizers.from_name("random-forest-default")
    opt = make(_grid_sampler, 4, 3)
    # before update_first (= batch) observations: 4 random picks among
    # batch_candidates fresh samples, one seed draw for the candidates
    r = random.Random(3)
    cands = list(_grid_sampler(1000, r.randint(0, 2**32 - 1)))
    first = opt.suggest()
    assert first == r.choices(cands, k=4)
    opt.observe(first, [peak(x) for x in first])
    assert opt.fitted_on == 4
    fits = [opt.fitted_on]
    for _ in range(9):
        xs = opt.suggest()
        assert len(xs) == 4
        opt.observe(xs, [peak(x) for x in xs])
        fits.append(opt.fitted_on)
    # refit every update_period (= batch) observations
    assert fits == list(range(4, 44, 4))
    assert opt.best_y == max(opt.y) and peak(opt.best_x) == opt.best_y
    # 40 evaluations of a 256-point grid find the optimum's neighbourhood
    assert abs(opt.best_x[0] - 11) + abs(opt.best_x[1] - 4) <= 2, opt.best_x
    # same seed, same proposals
    again = make(_grid_sampler, 4, 3)
    assert again.suggest() == first
    # a YAML file overrides the preset
    conf = tmp_path / "rf.yaml"
    conf.write_text("beta: 0.5\nupdate_first: 8\n")
    tuned = make(_grid_sampler, 4, 3, str(conf))
    assert tuned.beta == 0.5 and tuned.update_first == 8 and tuned.alpha == 0.7
    with pytest.raises(ValueError, match="unknown optimizer"):
        Optimizers.from_name("bayes")


def test_explorer_refuses_gpu_hardware_counters(tmp_path):
    from xtc_amd.cli.explore import main
    from xtc_amd.search.explore import check_explore_counters

    check_explore_counters(["gpu.time", "gpu.clocks"])
    with pytest.raises(ValueError, match="switched off"):
        check_explore_counters(["gpu.time", "gpu.SQ_WAVES"])
    assert main(["--pmu-counters", "gpu.cycles", "--output", str(tmp_path / "x.csv")]) == 2
    assert not (tmp_path / "x.csv").exists()


# ---------------------------------------------------------------- the reference's remaining CLI flags

def test_cli_listing_flags(capsys):
    from xtc_amd.cli.explore import main

    assert main(["--operator-list"]) == 0
    assert capsys.readouterr().out.split() == ["matmul", "conv2d", "relu"]
    assert main(["--strategy-list"]) == 0
    assert "tile_hip" in capsys.readouterr().out.split()
    assert main(["--operator", "conv2d", "--op-name-list"]) == 0
    out = capsys.readouterr().out.splitlines()
    # src/xtc/artifacts: 32 layers of Yolo9000/MobileNet/ResNet18, then 17 of SqueezeNet/AlexNet
    assert len(out) == 49 and out[0].startswith("Yolo9000_00: {'n': 1, 'h': 544")
    assert "ResNet18_04: {'n': 1, 'h': 56, 'w': 56, 'f': 128, 'r': 3, 's': 3, 'c': 64}, {'SH': 2, 'SW': 2}" in out


def test_named_operations_follow_the_reference_registry():
    from xtc_amd.artifacts import get_operation, has_operation, list_operations
    from xtc_amd.cli.explore import _operation_dims

    assert _operation_dims("conv2d", "resnet18_04") == [1, 56, 56, 128, 3, 3, 64, 2, 2]
    assert _operation_dims("matmul", "Gemma9B_FC") == [3584, 14336, 3584]
    assert get_operation("matmul", "AlexNet_FC6")["dims"] == {"i": 1, "j": 4096, "k": 9216}
    assert len(list_operations("matmul")) == 27 and has_operation("conv2d", "SQUEEZENET_21")
    with pytest.raises(ValueError, match="not registered"):
        get_operation("matmul", "ResNet18_04")
    g = build_graph("conv2d", _operation_dims("conv2d", "ResNet18_01"), "float32", name="rn18_01")
    assert g.name == "rn18_01"
    assert [str(t) for t in g.inputs_types] == ["1x454x454x3xfloat32", "7x7x3x64xfloat32"]


def test_cli_rejects_resume_with_append(tmp_path):
    from xtc_amd.cli.explore import main

    with pytest.raises(SystemExit):
        main(["--resume", "--append", "--output", str(tmp_path / "x.csv")])


def test_cli_compile_only_runs_record_nothing(tmp_path, capsys):
    """--no-execute compiles each sample (payload libraries under
    --explore-dir, sources under --save-temps-dir) and evaluates none; the
    CSV keeps its header only."""
    from xtc_amd.cli.explore import main

    out = tmp_path / "r.csv"
    temps = tmp_path / "temps"
    rc = main(["--operator", "matmul", "--dims", "256", "256", "256", "--trials", "3", "--no-execute", "--quiet",
               "--output", str(out), "--explore-dir", str(tmp_path), "--save-temps", "--save-temps-dir", str(temps),
               "--func-name", "mm256", "--jobs", "2"])
    assert rc == 0
    assert len(list(csv.DictReader(open(out)))) == 0
    assert (temps / "mm256.graph.yaml").exists()
    assert sorted(p.name for p in temps.iterdir() if p.is_dir()) == ["0000", "0001", "0002"]
    assert capsys.readouterr().out == ""


def test_cli_opt_level_and_test_evaluate_one_schedule(tmp_path, monkeypatch, capsys):
    from xtc_amd.cli.explore import main

    seen = []

    def evaluate_one(self, module):
        seen.append(module)
        return [1e-3], 0, ""

    monkeypatch.setattr(Exploration, "evaluate_one", evaluate_one)
    # the reference evaluates the default schedule at --opt-level 0-3
    assert main(["--operator", "matmul", "--dims", "256", "256", "256", "--opt-level", "2", "--peak-flops", "1e12",
                 "--output", str(tmp_path / "a.csv")]) == 0
    assert len(seen) == 1
    assert capsys.readouterr().out.startswith("Schedule: hip: [")
    g = build_graph("matmul", [256, 256, 256], "float32")
    x = Strategies.create("tile_hip", g).default_schedule(2)
    assert main(["--operator", "matmul", "--dims", "256", "256", "256", "--test", *map(str, x), "--quiet", "--peak-flops", "1e12",
                 "--output", str(tmp_path / "b.csv")]) == 0
    rows = list(csv.DictReader(open(tmp_path / "b.csv")))
    assert len(seen) == 2 and len(rows) == 1 and parse_x(rows[0]["X"]) == list(x)


def test_cli_descript_spec_replaces_the_strategy(tmp_path, monkeypatch):
    """--descript: the spec's parameters are the CSV columns, and every
    sample kept by the HIP filter compiles to a kernel instance."""
    from xtc_amd.cli.explore import main

    monkeypatch.setattr(Exploration, "evaluate_one", lambda self, module: ([1e-3], 0, ""))
    spec = tmp_path / "spec.yaml"
    spec.write_text("i:\nj:\nk:\ni#bm:\nj#bn:\nk#bk:\ni#wm:\nj#wn:\n")
    out = tmp_path / "d.csv"
    assert main(["--operator", "matmul", "--dims", "512", "512", "512", "--descript", str(spec), "--trials", "4", "--peak-flops", "1e12",
                 "--quiet", "--output", str(out), "--db-file", str(tmp_path / "d.jsonl"), "--jobs", "2"]) == 0
    rows = list(csv.DictReader(open(out)))
    assert list(rows[0])[:5] == ["bm", "bn", "bk", "wm", "wn"] and len(rows) == 4
    db = [json.loads(l) for l in open(tmp_path / "d.jsonl")]
    assert all(d["strategy"][2] == "descript" and d["kernels"]["C"].startswith("gemm<float32>") for d in db)


# ---------------------------------------------------------------- the reference's Python form

def test_exploration_from_a_configuration(tmp_path, monkeypatch, capsys):
    """Exploration(config): the graph from the configuration's operator and
    dims, every backend of `backends`, results as (sample, code, time,
    backend) in the return value, `results` and `config.results`, and the
    reference's closing line (src/xtc/search/explore.py:200-210, 764-873;
    docs/tutorials/explore_optimizers.py:199-227)."""
    monkeypatch.setattr(Exploration, "evaluate_one", lambda self, module: ([2e-4, 1e-4], 0, ""))
    config = ExplorationConfig(operator="matmul", dims=[256, 256, 256], backends=["hip"], strategy="tile_hip",
                               search="random", trials=3, seed=0, output=str(tmp_path / "r.csv"), peak_flops=1e12,
                               func_name="mm")
    exploration = Exploration(config)
    res = exploration()
    assert res is exploration.results and config.results == res and len(res) == 3
    assert all(code == 0 and t == 1e-4 and backend == "hip" and len(x) == 7 for x, code, t, backend in res)
    assert capsys.readouterr().out.startswith("Schedule: hip: [")
    rows = list(csv.DictReader(open(tmp_path / "r.csv")))
    assert len(rows) == 3 and float(rows[0]["peak"]) == pytest.approx(256**3 / 1e12 / 1e-4)
    # a named operation's dims, opt-level 0-3: one default schedule
    config = ExplorationConfig(operator="conv2d", op_name="ResNet18_12", opt_level=2, quiet=True,
                               output=str(tmp_path / "n.csv"), peak_flops=1e12)
    (res,) = Exploration(config).run()
    assert res[1] == 0 and capsys.readouterr().out == ""
    # a reference strategy with its scheme argument (prt:<scheme>), filtered to compiled kernels
    config = ExplorationConfig(operator="matmul", dims=[512, 512, 512], strategy="prt:PPRPRP", trials=2, quiet=True,
                               output=str(tmp_path / "p.csv"), peak_flops=1e12)
    assert [code for _, code, _, _ in Exploration(config).run()] == [0, 0]


def test_exploration_config_from_args():
    import argparse

    ns = argparse.Namespace(operator="conv2d", trials=7, search="exhaustive", not_a_field=1)
    c = ExplorationConfig.from_args(ns, seed=3)
    assert (c.operator, c.trials, c.search, c.seed) == ("conv2d", 7, "exhaustive", 3)
    with pytest.raises(TypeError, match="unknown exploration configuration option"):
        ExplorationConfig.from_args(None, trialz=1)


def test_random_inputs_give_seeded_uniform_parameters(tmp_path, monkeypatch):
    from xtc_amd.search.explore import random_parameters
    from xtc_amd.utils.bf16 import round_to_bf16

    g = build_graph("matmul", [64, 32, 48], "bfloat16")
    (a, b), (c,) = random_parameters(g, 7)
    assert a.shape == (64, 48) and b.shape == (48, 32) and c.shape == (64, 32)
    assert a.dtype == np.float32 and c.dtype == np.float32
    assert np.array_equal(a, round_to_bf16(a)) and -1.0 <= a.min() and a.max() <= 1.0
    a2, _ = random_parameters(g, 7)[0]
    assert np.array_equal(a, a2) and not np.array_equal(a, random_parameters(g, 8)[0][0])
    # the CLI hands them to every evaluation and records the seed in the manifest
    seen = []

    def evaluate_one(self, module):
        seen.append(self.config.eval_parameters)
        return [1e-3], 0, ""

    monkeypatch.setattr(Exploration, "evaluate_one", evaluate_one)
    from xtc_amd.cli.explore import main

    out = tmp_path / "r.csv"
    assert main(["--operator", "matmul", "--dims", "64", "32", "48", "--dtype", "bfloat16", "--trials", "2",
                 "--random-inputs", "7", "--peak-flops", "1e12", "--output", str(out), "--jobs", "1", "--quiet"]) == 0
    assert len(seen) == 2 and all(np.array_equal(p[0][0], a) for p in seen)
    meta = json.loads(open(f"{out}.meta.json").read())
    assert meta["args"]["random_inputs"] == 7


def test_random_inputs_validate_to_a_scaled_bound():
    """On random inputs the payload's fp32 sums and numpy's differ in the last
    bits, so np.allclose's atol 1e-8 fails near-zero outputs: the explorer
    validates those samples to max |diff| <= 1e-4 max |ref| (1e-10 for
    float64), which still catches a dropped term."""
    from xtc_amd.search.explore import ExplorationConfig, random_inputs_tolerance
    from xtc_amd.targets.hip.evaluator import outputs_mismatch

    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (128, 512)).astype(np.float32)
    b = rng.uniform(-1, 1, (512, 128)).astype(np.float32)
    ref = np.dot(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    # fp32 sums in another order: k walked backwards, one term at a time
    got = np.zeros_like(ref)
    for k in range(511, -1, -1):
        got += np.outer(a[:, k], b[k, :])
    assert outputs_mismatch(ref, got, 1e-5, 1e-8) is not None  # np.allclose rejects the rounding
    assert outputs_mismatch(ref, got, 1e-5, 1e-8, 1e-4) is None
    dropped = got - np.outer(a[:, 17], b[17, :])  # one k missing
    assert "max |diff| / max |ref|" in outputs_mismatch(ref, dropped, 1e-5, 1e-8, 1e-4)
    nan_ref, nan_got = ref.copy(), got.copy()
    nan_ref[3, 4] = np.nan
    assert "NaN" in outputs_mismatch(nan_ref, got, 1e-5, 1e-8, 1e-4)
    nan_got[3, 4] = np.nan
    assert outputs_mismatch(nan_ref, nan_got, 1e-5, 1e-8, 1e-4) is None
    assert outputs_mismatch(ref, ref.copy(), 1e-5, 1e-8) is None

    assert random_inputs_tolerance(build_graph("matmul", [8, 8, 8], "bfloat16")) == 1e-4
    assert random_inputs_tolerance(build_graph("matmul", [8, 8, 8], "float32")) == 1e-4
    assert random_inputs_tolerance(build_graph("matmul", [8, 8, 8], "float64")) == 1e-10
    import xtc_amd.graphs.xtc.op as O

    x = O.tensor((8, 8), "bfloat16", name="X")
    y = O.tensor((8, 8), "bfloat16", name="Y")
    with O.graph(name="mm_bf16_out") as gb:
        O.matmul(x, y, name="Z")  # bf16 output: its rounding is coarser than the sums' differences
    assert random_inputs_tolerance(gb.graph) == 1e-2

    # the explorer hands the bound to the evaluator only for random inputs
    seen = []

    class Module:
        def get_evaluator(self, **kw):
            seen.append(kw)
            return type("E", (), {"evaluate": staticmethod(lambda: ([1e-3], 0, ""))})()

    g = build_graph("matmul", [8, 8, 8], "float64")
    for seed in (None, 3):
        ex = Exploration(g, ExplorationConfig(backend="hip", random_inputs=seed, validate=True))
        assert ex.evaluate_one(Module()) == ([1e-3], 0, "")
    assert "scaled_tolerance" not in seen[0] and seen[1]["scaled_tolerance"] == 1e-10


def test_exploration_static_helpers(capsys):
    """The reference's Exploration static API (explore.py:211-261, 813-862):
    graph builders with its tensor names, listings, named-operation dims."""
    g = Exploration.xtc_matmul_graph(4, 32, 512, "float32")
    assert [str(t) for t in g.inputs_types] == ["4x512xfloat32", "512x32xfloat32"] and g.name == "matmul"
    assert [str(t) for t in Exploration.xtc_conv2d_graph(1, 4, 4, 16, 5, 5, 3, 2, 2, "float32").outputs_types] == [
        "1x4x4x16xfloat32"]
    assert [str(t) for t in Exploration.xtc_relu_graph(10, "float64").inputs_types] == ["10xfloat64"]
    Exploration.list_operators()
    Exploration.list_optimizers()
    Exploration.list_strategies()
    out = capsys.readouterr().out.split()
    assert out[:3] == ["matmul", "conv2d", "relu"] and "random-forest-default" in out and "tile_hip" in out
    assert Exploration.get_operation_dims("conv2d", "ResNet18_01") == [1, 224, 224, 64, 7, 7, 3, 2, 2]
    assert Exploration.get_strategy_name("tile_oo") == "tile_oo"
