# SPDX-License-Identifier: BSD-3-Clause
"""Extracts the strategy golden vectors of the reference's search tests.

Reads, as text, /root/reference/tests/filecheck/search/test_*.py: the
strategy class and keyword arguments of the `Strategy(graph, ...)` call, the
graph helper used (matmul 21x32x12 or conv2d 2x4x4x32, 7x7x3, stride 2), the
printing helper (default schedules, exhaustive or random samples) and the
expected `schedule O<n>: [...]`, `sample <i>: [...]` and `stats {...}` lines
of its FileCheck comments.  Writes tests/golden/strategy_transcripts.json
(data only).  Run once in the build container; the fixture is committed.
"""

from __future__ import annotations

import ast
import json
import re
from pathlib import Path

SRC = Path("/root/reference/tests/filecheck/search")
OUT = Path(__file__).resolve().parent / "strategy_transcripts.json"


def _const(node: ast.AST) -> object:
    """Literal or integer arithmetic on literals (e.g. 8*1024)."""
    if isinstance(node, ast.BinOp) and isinstance(node.op, (ast.Mult, ast.Add, ast.Sub, ast.FloorDiv)):
        a, b = _const(node.left), _const(node.right)
        assert isinstance(a, int) and isinstance(b, int)
        return {ast.Mult: a * b, ast.Add: a + b, ast.Sub: a - b, ast.FloorDiv: a // b if b else 0}[type(node.op)]
    return ast.literal_eval(node)


def parse(path: Path) -> dict | None:
    text = path.read_text()
    tree = ast.parse(text)
    strategy = kwargs = graph = None
    calls = []
    for node in ast.walk(tree):
        if isinstance(node, ast.ImportFrom) and node.module == "xtc.search.strategies":
            for alias in node.names:
                if alias.asname == "Strategy":
                    strategy = alias.name
        if isinstance(node, ast.Call) and isinstance(node.func, ast.Name) and node.func.id == "Strategy":
            kwargs = {k.arg: _const(k.value) for k in node.keywords}
        if isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute):
            name = node.func.attr
            if name in ("get_graph_matmul", "get_graph_conv2d"):
                graph = name.replace("get_graph_", "")
            if name.startswith("print_"):
                args = [_const(a) for a in node.args[2:]]
                calls.append([name, args])
    if strategy is None or kwargs is None:
        return None
    checks = [re.sub(r"^#\s*CHECK(-NEXT)?:\s*", "", l) for l in text.splitlines() if re.match(r"^#\s*CHECK", l)]
    defaults = {int(m.group(1)): json.loads(m.group(2)) for l in checks if (m := re.match(r"schedule O(\d): (\[.*\])$", l))}
    samples = [json.loads(m.group(1)) for l in checks if (m := re.match(r"sample \d+: (\[.*\])$", l))]
    stats = [ast.literal_eval(m.group(1)) for l in checks if (m := re.match(r"stats (\{.*\})$", l))]
    return {
        "strategy": strategy,
        "kwargs": kwargs,
        "graph": graph,
        "calls": calls,
        "defaults": defaults,
        "samples": samples,
        "stats": stats[0] if stats else None,
    }


def main() -> None:
    out = {}
    for path in sorted(SRC.glob("test_*.py")):
        if "descript" in path.name:
            continue
        rec = parse(path)
        if rec is not None:
            out[path.name] = rec
    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"wrote {len(out)} transcripts to {OUT}")


if __name__ == "__main__":
    main()
