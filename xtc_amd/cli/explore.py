# SPDX-License-Identifier: BSD-3-Clause
"""`loop-explore` for the HIP backend (src/xtc/cli/explore.py:52-355).

  python -m xtc_amd.cli.explore --operator matmul --dims 4096 4096 4096 \
      --dtype float32 --backends hip --strategy tile_pprprp --search random \
      --trials 64 --seed 0 --output c2.csv

Flags follow the reference where they apply (operator, dims, dtype,
strategy, search, backends, trials, seed, threads, max-unroll, opt-level,
output, db-file, resume, append, graph-file, peak-flops, data, optimizer,
optimizer-list, optimizer-config, batch).  The
reference re-executes itself under `setarch -R` to disable ASLR for CPU
timing stability; GPU timing does not need it, so this driver runs in-process.
"""

from __future__ import annotations

import argparse
import logging
import os
import sys
from typing import Any

from ..search.explore import Exploration, ExplorationConfig
from ..search.strategies import Strategies

# default dims of the reference's OPERATORS table (src/xtc/search/explore.py:150-198)
DEFAULT_DIMS = {"matmul": [512, 512, 512], "conv2d": [1, 112, 112, 64, 7, 7, 3, 2, 2], "relu": [512 * 1024]}


def build_graph(operator: str, dims: list[int], dtype: str, pad: int = 0) -> Any:
    """Graphs of the reference's `--operator` choices, with the same tensor
    and node names and shapes (explore.py:218-256).  bfloat16 matmul/conv
    accumulate and store fp32 (out_dtype extension).  `pad` > 0 puts a
    pad2d producer on H and W in front of the conv (the C4 pattern); the
    padded input then has the reference's conv input shape."""
    import xtc_amd.graphs.xtc.op as O

    extra = {"out_dtype": "float32"} if dtype == "bfloat16" else {}
    if operator == "matmul":
        i, j, k = dims
        a = O.tensor((i, k), dtype, name="A")
        b = O.tensor((k, j), dtype, name="B")
        with O.graph(name="matmul") as gb:
            O.matmul(a, b, name="C", **extra)
        return gb.graph
    if operator == "conv2d":
        n, h, w, f, r, s, c, sh, sw = dims if len(dims) == 9 else (dims + [1, 1])[:9]
        ih, iw = h * sh + r - 1 - 2 * pad, w * sw + s - 1 - 2 * pad
        x = O.tensor((n, ih, iw, c), dtype, name="A")
        wt = O.tensor((r, s, c, f), dtype, name="B")
        with O.graph(name="conv2d") as gb:
            src = O.pad2d(x, padding=pad, axes=(1, 2), name="pad") if pad else x
            O.conv2d(src, wt, stride=(sh, sw), name="O", **extra)
        return gb.graph
    if operator == "relu":
        (i,) = dims
        x = O.tensor((i,), dtype, name="I")
        with O.graph(name="relu") as gb:
            O.relu(x, threshold=0, name="O")
        return gb.graph
    raise SystemExit(f"unknown operator {operator}")


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(prog="loop-explore", description=__doc__.split("\n\n")[0])
    p.add_argument("--operator", default="matmul", choices=["matmul", "conv2d", "relu"])
    p.add_argument("--graph-file", help="YAML graph (Graph.dump format) instead of --operator")
    p.add_argument("--dims", nargs="+", type=int, help="operator dimensions")
    p.add_argument("--pad", type=int, default=0, help="conv2d: pad2d producer on H and W")
    p.add_argument("--dtype", default="float32", choices=["float32", "bfloat16"])
    p.add_argument("--strategy", default="tile_hip", help=f"one of {Strategies.names(include_aliases=True)}")
    p.add_argument("--search", default="random", choices=["random", "exhaustive", "data", "default", "iterative"])
    p.add_argument("--optimizer", default="random-forest-default",
                   help="optimizer of --search iterative; --optimizer-list lists them")
    p.add_argument("--optimizer-list", action="store_true", help="print the optimizers and exit")
    p.add_argument("--optimizer-config", default="", help="YAML file overriding the optimizer's preset")
    p.add_argument("--batch", type=int, default=1, help="samples per optimizer proposal")
    p.add_argument("--data", help="CSV of samples for --search data")
    p.add_argument("--backends", nargs="+", default=["hip"], choices=["hip"])
    p.add_argument("--trials", type=int, default=64)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--threads", type=int, default=1, help="strategy threads (parallel outer axes)")
    p.add_argument("--max-unroll", type=int, default=None,
                   help="strategy unroll bound (default 2^22: the MFMA kernels always unroll their inner loops, "
                   "so the CPU bound of 256 would only exclude GPU-sized tiles)")
    p.add_argument("--vec-size", type=int, default=16)
    p.add_argument("--opt-level", type=int, default=2)
    p.add_argument("--repeat", type=int, default=5)
    p.add_argument("--number", type=int, default=1)
    p.add_argument("--min-repeat-ms", type=int, default=100)
    p.add_argument("--validate", action="store_true")
    p.add_argument("--pmu-counters", nargs="*", default=[],
                   help="counters per sample (gpu.time, gpu.clocks); gpu.time is added when missing and gives the "
                        "CSV time, every counter's values go to the --db-file record.  GPU hardware counters "
                        "(gpu.cycles, gpu.<rocprofiler counter>) are switched off here: explorations with them "
                        "stalled on MI355X")
    p.add_argument("--jobs", type=int, default=max(1, min(16, (os.cpu_count() or 2) // 2)))
    p.add_argument("--output", default="results.csv")
    p.add_argument("--db-file")
    p.add_argument("--resume", action="store_true")
    p.add_argument("--append", action="store_true")
    p.add_argument("--peak-flops", type=float, help="peak FMA/s (default: device MFMA peak)")
    p.add_argument("--debug", action="store_true")
    args = p.parse_args(argv)
    if args.optimizer_list:
        from ..search.optimizers import Optimizers

        print("\n".join(Optimizers.names()))
        return 0
    logging.basicConfig(level=logging.DEBUG if args.debug else logging.INFO, format="%(message)s")
    if args.pmu_counters:
        from ..search.explore import check_explore_counters

        try:
            check_explore_counters(args.pmu_counters)
        except ValueError as err:
            print(err, file=sys.stderr)
            return 2
    if "hip" in args.backends:
        from ..backends.hip.compiler import CompileService

        # the payload compiler's fork server starts before anything loads the
        # GPU libraries (XTC_HIP_PMU=1 registers the counter tool on load)
        CompileService.start_server()

    if args.graph_file:
        import xtc_amd.graphs.xtc.op as O

        with O.graph() as gb:
            gb.load(args.graph_file)
        graph = gb.graph
    else:
        graph = build_graph(args.operator, args.dims or DEFAULT_DIMS[args.operator], args.dtype, args.pad)
    max_unroll = args.max_unroll if args.max_unroll is not None else 1 << 22
    strat_kwargs = {"threads": args.threads, "max_unroll": max_unroll, "vec_size": args.vec_size}
    if Strategies.resolve_name(args.strategy) == "tile_hip":
        strat_kwargs = {}
    for backend in args.backends:
        cfg = ExplorationConfig(
            backend=backend,
            strategy=args.strategy,
            strategy_kwargs=strat_kwargs,
            search=args.search,
            trials=args.trials,
            seed=args.seed,
            optimizer=args.optimizer,
            optimizer_config=args.optimizer_config,
            batch=args.batch,
            opt_level=args.opt_level,
            data=args.data,
            repeat=args.repeat,
            number=args.number,
            min_repeat_ms=args.min_repeat_ms,
            validate=args.validate,
            pmu_counters=args.pmu_counters,
            jobs=args.jobs,
            output=args.output,
            db_file=args.db_file,
            resume=args.resume,
            append=args.append,
            peak_flops=args.peak_flops,
        )
        results = Exploration(graph, cfg).run()
        ok = [(min(t), s) for s, t, code, _ in results if code == 0 and t]
        if ok:
            best_t, best_s = min(ok)
            print(f"{backend}: best {best_s} {best_t * 1e6:.1f} us over {len(ok)}/{len(results)} samples", flush=True)
        else:
            print(f"{backend}: no successful sample ({len(results)} tried)", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
