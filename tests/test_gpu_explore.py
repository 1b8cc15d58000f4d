# SPDX-License-Identifier: BSD-3-Clause
"""loop-explore on the GPU, through its command line (src/xtc/cli/explore.py).

Every sample is compiled, validated against the graph's numpy interpreter
(XTC's own np.allclose check on np_init inputs) and timed; the CSV keeps the
reference's layout.  Each run is a fresh process, as `loop-explore` is.
"""

from __future__ import annotations

import csv
import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent


def _explore(tmp_path, *flags):
    out = tmp_path / "e.csv"
    db = tmp_path / "e.jsonl"
    cmd = [sys.executable, "-u", "-m", "xtc_amd.cli.explore", "--operator", "matmul", "--dims", "512", "512", "512",
           "--dtype", "float32", "--strategy", "tile_hip", "--seed", "0", "--repeat", "2", "--min-repeat-ms", "10",
           "--jobs", "4", "--output", str(out), "--db-file", str(db), *flags]
    print("[explore]", " ".join(cmd[3:]), flush=True)
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr[-3000:]
    return list(csv.DictReader(open(out))), [json.loads(line) for line in open(db)], proc


def test_loop_explore_c1_random_validated(tmp_path):
    rows, recs, proc = _explore(tmp_path, "--search", "random", "--trials", "8", "--validate")
    assert len(recs) == 8
    assert all(r["results"][0] == 0 for r in recs), [r["error"] for r in recs]
    assert len(rows) == 8, proc.stderr[-2000:]
    for r in rows:
        t = float(r["time"])
        # 512^3 fp32: above the MFMA roofline (1.7 us), below a millisecond
        assert 1.7e-6 < t < 1e-3 and float(r["peak"]) > 0
        assert r["backend"] == "hip"


def test_loop_explore_random_inputs_validated(tmp_path):
    """--random-inputs: every sample runs on the same seeded uniform[-1,1)
    operands and is validated to max |diff| <= 1e-4 max |ref| (np.allclose's
    atol would reject the fp32 rounding of near-zero outputs)."""
    rows, recs, proc = _explore(tmp_path, "--search", "random", "--trials", "6", "--validate", "--random-inputs", "5")
    assert len(recs) == 6 and all(r["results"][0] == 0 for r in recs), [r["error"] for r in recs]
    assert len(rows) == 6
    meta = json.loads(open(tmp_path / "e.csv.meta.json").read())
    assert meta["args"]["random_inputs"] == 5 and meta["args"]["validate"] is True


def test_loop_explore_c1_iterative(tmp_path):
    rows, recs, proc = _explore(tmp_path, "--search", "iterative", "--trials", "6", "--batch", "2", "--optimizer",
                                "random-forest-default")
    assert len(recs) == 6 and all(r["results"][0] == 0 for r in recs), [r["error"] for r in recs]
    assert 1 <= len(rows) <= 6
    # the reference's closing line: best schedule, time and fraction of peak
    assert "Schedule: hip: [" in proc.stdout and "peak perf:" in proc.stdout


def test_loop_explore_descript_spec_validated(tmp_path):
    """--descript: a spec's free tile sizes, sampled under the HIP filter,
    compiled, run and validated on the device."""
    spec = tmp_path / "spec.yaml"
    spec.write_text("i: parallelize\nj: parallelize\nk:\ni#bm:\nj#bn:\nk#bk:\ni#wm:\nj#wn:\n")
    rows, recs, proc = _explore(tmp_path, "--descript", str(spec), "--trials", "6", "--validate")
    assert len(recs) == 6 and all(r["results"][0] == 0 for r in recs), [r["error"] for r in recs]
    assert len(rows) == 6 and list(rows[0])[:5] == ["bm", "bn", "bk", "wm", "wn"]
    assert all(r["strategy"][2] == "descript" for r in recs)
    assert all(1.7e-6 < float(r["time"]) < 1e-3 for r in rows)


def test_loop_explore_named_conv_with_split_k(tmp_path):
    """--op-name picks a reference layer (ResNet18_12: 7x7 outputs, 512
    channels, K 4608); tile_hip samples its split-K points, each validated."""
    out = tmp_path / "n.csv"
    cmd = [sys.executable, "-u", "-m", "xtc_amd.cli.explore", "--operator", "conv2d", "--op-name", "ResNet18_12",
           "--strategy", "tile_hip", "--search", "exhaustive", "--trials", "40", "--validate", "--repeat", "1",
           "--min-repeat-ms", "5", "--jobs", "4", "--quiet", "--output", str(out)]
    print("[explore]", " ".join(cmd[3:]), flush=True)
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr[-3000:]
    rows = list(csv.DictReader(open(out)))
    assert len(rows) >= 20 and {int(r["split_k"]) for r in rows} >= {1, 16, 32}
    times = {int(r["split_k"]): min(float(x["time"]) for x in rows if int(x["split_k"]) == int(r["split_k"]))
             for r in rows}
    # splitting the 4608-deep K over 16-32 slices is several times faster
    assert min(times[16], times[32]) * 2 < times[1]

