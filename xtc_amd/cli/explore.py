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
--dtype is float32, float64 (the reference's two) or bfloat16 (bfloat16
operands, fp32 results);
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

from ..search.explore import OPERATORS, Exploration, ExplorationConfig, build_graph, operation_dims

# default dims of the reference's OPERATORS table (src/xtc/search/explore.py:151-198)
DEFAULT_DIMS = {name: list(op["default_dims"]) for name, op in OPERATORS.items()}

__all__ = ["main", "build_graph", "DEFAULT_DIMS"]


_operation_dims = operation_dims


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
    p.add_argument("--dtype", default="float32", choices=["float32", "float64", "bfloat16"])
    p.add_argument("--trials", type=int, default=100)
    p.add_argument("--threads", type=int, default=1, help="strategy threads (parallel outer axes)")
    p.add_argument("--max-unroll", type=int, default=None,
                   help="strategy unroll bound (default 2^22: the MFMA kernels always unroll their inner loops, "
                   "so the CPU bound of 256 would only exclude GPU-sized tiles)")
    p.add_argument("--vec-size", type=int, default=16)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--random-inputs", type=int, default=None, metavar="SEED",
                   help="time (and validate) every sample on seeded uniform[-1,1) inputs, rounded to bfloat16 for "
                        "bfloat16 tensors, instead of the reference's np_init integers: on MI355X a bf16 GEMM's "
                        "clock depends on the power its operands draw. --validate then checks max |diff| <= "
                        "1e-4 max |ref| (1e-10 for float64, 1e-2 for a bfloat16 output) in place of np.allclose")
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
        Exploration.list_operations_dims(args.operator)
        return 0
    if args.strategy_list:
        Exploration.list_strategies()
        return 0
    if args.optimizer_list:
        Exploration.list_optimizers()
        return 0
    if args.pmu_counters:
        from ..search.explore import check_explore_counters

        try:
            check_explore_counters(args.pmu_counters)
        except ValueError as err:
            print(err, file=sys.stderr)
            return 2
    if args.op_name:
        try:
            _operation_dims(args.operator, args.op_name)
        except ValueError as err:
            p.error(str(err))
    if "hip" in args.backends:
        from ..backends.hip.compiler import CompileService

        # the payload compiler's fork server starts before anything loads the
        # GPU libraries (XTC_HIP_PMU=1 registers the counter tool on load)
        CompileService.start_server()
    config = ExplorationConfig.from_args(args)
    if args.graph_file:
        config.operator = None
    if args.random_inputs is not None:
        from ..search.explore import config_graph, random_parameters

        config.eval_parameters = random_parameters(config_graph(config), args.random_inputs)
    results = Exploration(config).run()
    if not args.quiet and not args.execute:
        ok = sum(1 for _, code, _, _ in results if code == 0)
        print(f"compiled {ok}/{len(results)} samples", flush=True)
    elif not args.quiet and not any(code == 0 and t > 0 for _, code, t, _ in results):
        print(f"no successful sample ({len(results)} tried)", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
