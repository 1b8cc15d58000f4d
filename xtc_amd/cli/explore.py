# SPDX-License-Identifier: BSD-3-Clause
"""`loop-explore` for the HIP backend (src/xtc/cli/explore.py:52-355).

  python -m xtc_amd.cli.explore --operator matmul --dims 4096 4096 4096 \
      --dtype float32 --backends hip --strategy tile_pprprp --search random \
      --trials 64 --seed 0 --output c2.csv

Every flag of the reference is accepted, with the reference's meaning and
defaults: --opt-level 0-3 (or --test X) evaluates one schedule, 4 (the
default) searches; --descript takes a descript YAML spec in place of
--strategy; --op-name picks a named layer's dims (xtc_amd.artifacts);
--no-execute compiles without evaluating; --save-temps, --explore-dir, --dump
keep or print the payloads.  Differences: --backends has only `hip`;
--dtype is float32 or bfloat16 (bfloat16 operands, fp32 results);
--repeat defaults to 5; --huge-pages, --bare-ptr, --child, --mlir-prefix and
--use-tensors are accepted and change nothing here (device buffers, bare
pointers, no MLIR).  Extensions: --pad, --search default, --vec-size,
--pmu-counters.  The reference re-executes itself under `setarch -R` to
disable ASLR for CPU timing stability; GPU timing does not need it, so this
driver runs in-process.
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
DEFAULT_DIMS = {"matmul": [512, 1024, 128], "conv2d": [1, 112, 112, 64, 7, 7, 3, 2, 2], "relu": [512 * 1024]}


def build_graph(operator: str, dims: list[int], dtype: str, pad: int = 0, name: str | None = None) -> Any:
    """Graphs of the reference's `--operator` choices, with the same tensor
    and node names and shapes (explore.py:218-256).  bfloat16 matmul/conv
    accumulate and store fp32 (out_dtype extension).  `pad` > 0 puts a
    pad2d producer on H and W in front of the conv (the C4 pattern); the
    padded input then has the reference's conv input shape.  `name` is the
    graph's (function's) name, default to the operator."""
    import xtc_amd.graphs.xtc.op as O

    extra = {"out_dtype": "float32"} if dtype == "bfloat16" else {}
    if operator == "matmul":
        i, j, k = dims
        a = O.tensor((i, k), dtype, name="A")
        b = O.tensor((k, j), dtype, name="B")
        with O.graph(name=name or "matmul") as gb:
            O.matmul(a, b, name="C", **extra)
        return gb.graph
    if operator == "conv2d":
        n, h, w, f, r, s, c, sh, sw = dims if len(dims) == 9 else (dims + [1, 1])[:9]
        ih, iw = h * sh + r - 1 - 2 * pad, w * sw + s - 1 - 2 * pad
        x = O.tensor((n, ih, iw, c), dtype, name="A")
        wt = O.tensor((r, s, c, f), dtype, name="B")
        with O.graph(name=name or "conv2d") as gb:
            src = O.pad2d(x, padding=pad, axes=(1, 2), name="pad") if pad else x
            O.conv2d(src, wt, stride=(sh, sw), name="O", **extra)
        return gb.graph
    if operator == "relu":
        (i,) = dims
        x = O.tensor((i,), dtype, name="I")
        with O.graph(name=name or "relu") as gb:
            O.relu(x, threshold=0, name="O")
        return gb.graph
    raise SystemExit(f"unknown operator {operator}")


def _operation_dims(operator: str, name: str) -> list[int]:
    """Dims of a named operation: its loop sizes, then its params
    (src/xtc/search/explore.py:837-841)."""
    from ..artifacts import get_operation

    op = get_operation(operator, name)
    return [*op["dims"].values(), *op["params"].values()]


def _bool(p: argparse.ArgumentParser, name: str, default: bool, help: str) -> None:
    p.add_argument(name, action=argparse.BooleanOptionalAction, default=default, help=help)


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(prog="loop-explore", description=__doc__.split("\n\n")[0],
                                formatter_class=argparse.ArgumentDefaultsHelpFormatter)
    p.add_argument("--operator", default="matmul", choices=list(DEFAULT_DIMS),
                   help="operator to optimize, use --operator-list for available operators")
    p.add_argument("--operator-list", action="store_true", help="print available operators")
    p.add_argument("--graph-file", help="YAML graph (Graph.dump format) instead of --operator")
    p.add_argument("--op-name", help="named operation of --operator (its dims), use --op-name-list")
    p.add_argument("--op-name-list", action="store_true", help="print the named operations of --operator")
    p.add_argument("--func-name", help="graph (function) name, default to operator")
    p.add_argument("--strategy", default="tile_hip", help="tile strategy, use --strategy-list for the list")
    p.add_argument("--strategy-list", action="store_true", help="print available strategies")
    p.add_argument("--descript", help="path to a descript yaml specification; replaces --strategy")
    p.add_argument("--search", default="random", choices=["random", "exhaustive", "data", "default", "iterative"])
    p.add_argument("--backends", nargs="+", default=["hip"], choices=["hip"])
    p.add_argument("--optimizer", default="random-forest-default",
                   help="optimizer of --search iterative; --optimizer-list lists them")
    p.add_argument("--optimizer-list", action="store_true", help="print the optimizers and exit")
    p.add_argument("--data", help="CSV of samples for --search data")
    p.add_argument("--dims", nargs="+", type=int, help="operator dimensions, default to the operator's")
    p.add_argument("--pad", type=int, default=0, help="conv2d: pad2d producer on H and W")
    _bool(p, "--huge-pages", True, "accepted for compatibility: GPU buffers come from the device allocator")
    p.add_argument("--test", nargs="+", type=int, default=[], help="evaluate this sample only")
    p.add_argument("--opt-level", type=int, default=4, help="0-3: evaluate the strategy's default schedule; 4: search")
    p.add_argument("--dtype", default="float32", choices=["float32", "bfloat16"])
    p.add_argument("--trials", type=int, default=100)
    p.add_argument("--threads", type=int, default=1, help="strategy threads (parallel outer axes)")
    p.add_argument("--max-unroll", type=int, default=None,
                   help="strategy unroll bound (default 2^22: the MFMA kernels always unroll their inner loops, "
                   "so the CPU bound of 256 would only exclude GPU-sized tiles)")
    p.add_argument("--vec-size", type=int, default=16)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--output", default="results.csv")
    p.add_argument("--db-file", help="output json db, for instance: xtc-graphs-db.json")
    _bool(p, "--resume", False, "skip samples already in --output")
    _bool(p, "--append", False, "append to --output without deduplication")
    p.add_argument("--eval", default="eval", choices=["eval"], help="evaluation method")
    p.add_argument("--repeat", type=int, default=5,
                   help="timed repeats per sample, the minimum is kept (the reference's default is 1)")
    p.add_argument("--number", type=int, default=1)
    p.add_argument("--min-repeat-ms", type=int, default=100)
    _bool(p, "--validate", False, "check each sample's output against the graph's reference")
    _bool(p, "--save-temps", False, "keep every payload's source under --save-temps-dir")
    p.add_argument("--save-temps-dir", default="./save_temps_dir")
    p.add_argument("--explore-dir", default=None, help="directory of the payload libraries (default: a temporary one)")
    p.add_argument("--optimizer-config", default="", help="YAML file overriding the optimizer's preset")
    _bool(p, "--child", False, "accepted for compatibility (the explorer runs in-process)")
    _bool(p, "--bare-ptr", False, "accepted for compatibility: payloads always take bare device pointers")
    p.add_argument("--jobs", type=int, default=max(1, min(16, (os.cpu_count() or 2) // 2)),
                   help="parallel compile jobs")
    _bool(p, "--execute", True, "evaluate the samples (--no-execute: compile only)")
    p.add_argument("--peak-flops", type=float, help="peak FMA/s (default: device MFMA peak)")
    p.add_argument("--mlir-prefix", help="accepted for compatibility (no MLIR in this backend)")
    _bool(p, "--use-tensors", False, "accepted for compatibility (no MLIR in this backend)")
    p.add_argument("--batch", type=int, default=1, help="samples per optimizer proposal")
    p.add_argument("--pmu-counters", nargs="*", default=[],
                   help="counters per sample (gpu.time, gpu.clocks); gpu.time is added when missing and gives the "
                        "CSV time, every counter's values go to the --db-file record.  GPU hardware counters "
                        "(gpu.cycles, gpu.<rocprofiler counter>) are switched off here: explorations with them "
                        "stalled on MI355X")
    _bool(p, "--debug", False, "debug logging")
    _bool(p, "--debug-compile", False, "log the payload compile commands")
    _bool(p, "--debug-xtc", False, "debug logging of every xtc_amd module")
    _bool(p, "--debug-optimizer", False, "log the optimizer's steps")
    _bool(p, "--quiet", False, "no per-sample lines")
    _bool(p, "--dump", False, "print each payload's generated source")
    args = p.parse_args(argv)
    if args.resume and args.append:
        p.error("--resume and --append cannot be used together")
    logging.basicConfig(level=logging.DEBUG if args.debug else logging.INFO, format="%(message)s")
    if args.debug_xtc:
        logging.getLogger("xtc_amd").setLevel(logging.DEBUG)
    if args.debug_optimizer:
        logging.getLogger("xtc_amd.search.optimizers").setLevel(logging.INFO)
    if args.operator_list:
        print("\n".join(DEFAULT_DIMS))
        return 0
    if args.op_name_list:
        from ..artifacts import get_operation, list_operations

        for _, name in list_operations(args.operator):
            op = get_operation(args.operator, name)
            print(f"{name}: {op['dims']}, {op['params']}")
        return 0
    if args.strategy_list:
        print("\n".join(Strategies.names(include_aliases=True)))
        return 0
    if args.optimizer_list:
        from ..search.optimizers import Optimizers

        print("\n".join(Optimizers.names()))
        return 0
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
        if args.op_name:
            try:
                dims = _operation_dims(args.operator, args.op_name)
            except ValueError as err:
                p.error(str(err))
        else:
            dims = args.dims or DEFAULT_DIMS[args.operator]
        graph = build_graph(args.operator, dims, args.dtype, args.pad, name=args.func_name or args.operator)
    max_unroll = args.max_unroll if args.max_unroll is not None else 1 << 22
    strat_kwargs = {"threads": args.threads, "max_unroll": max_unroll, "vec_size": args.vec_size}
    if args.descript or Strategies.resolve_name(args.strategy) == "tile_hip":
        strat_kwargs = {}
    # the reference evaluates one schedule at opt-level 0-3 or with --test
    # (src/xtc/search/explore.py:784-800)
    search = "default" if args.opt_level in (0, 1, 2, 3) else args.search
    for backend in args.backends:
        cfg = ExplorationConfig(
            backend=backend,
            strategy=args.strategy,
            strategy_kwargs=strat_kwargs,
            search=search,
            trials=args.trials,
            seed=args.seed,
            optimizer=args.optimizer,
            optimizer_config=args.optimizer_config,
            batch=args.batch,
            opt_level=min(args.opt_level, 3),
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
            compile_kwargs={"debug": True} if args.debug_compile else {},
            test=args.test,
            execute=args.execute,
            quiet=args.quiet,
            dump=args.dump,
            save_temps=args.save_temps,
            save_temps_dir=args.save_temps_dir,
            explore_dir=args.explore_dir,
            descript=args.descript,
        )
        exploration = Exploration(graph, cfg)
        results = exploration.run()
        if args.quiet:
            continue
        if not args.execute:
            ok = sum(1 for _, _, code, _ in results if code == 0)
            print(f"{backend}: compiled {ok}/{len(results)} samples", flush=True)
            continue
        ok = [(min(t), s) for s, t, code, _ in results if code == 0 and t]
        if ok:
            best_t, best_s = min(ok)
            peak = exploration.peak_time_s / best_t if exploration.peak_time_s else 0.0
            print(f"Schedule: {backend}: {best_s}: time: {best_t * 1000:.2f} msecs, peak perf: {peak * 100:.2f}%",
                  flush=True)
        else:
            print(f"{backend}: no successful sample ({len(results)} tried)", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
