# SPDX-License-Identifier: BSD-3-Clause
"""Extracts the expected transcripts of the reference's graph tests.

Reads, as text, /root/reference/tests/filecheck/graphs/test_*.py and keeps
only the expected output of each: the patterns of its FileCheck `CHECK:` /
`CHECK-NEXT:` comment lines, in order.  Writes
tests/golden/graph_prints.json as {test name: [pattern lines]} (data only).

Also reads /root/reference/tests/filecheck/backends/padding/test_*.py (pad,
pad2d and unpad around matmul and conv2d) and keeps, per test, the printed
graph its CHECK lines expect (from `graph:` to the first blank line) and
whether it expects the validated run to end with `CODE: 0`, and the error
that backends/invalid/test_pad2d_invalid.py expects.  Writes
tests/golden/padding_graph_prints.json as {test name: {"graph": [lines],
"code0": bool}} plus {"test_pad2d_invalid": {"error": line}} (data only).

Run once in the build container; the fixtures are committed.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

SRC = Path("/root/reference/tests/filecheck/graphs")
OUT = Path(__file__).resolve().parent / "graph_prints.json"
PAD_SRC = Path("/root/reference/tests/filecheck/backends/padding")
PAD_INVALID = Path("/root/reference/tests/filecheck/backends/invalid/test_pad2d_invalid.py")
PAD_OUT = Path(__file__).resolve().parent / "padding_graph_prints.json"


def _patterns(path: Path) -> list[str]:
    return [m.group(1) for l in path.read_text().splitlines() if (m := re.match(r"^#\s*CHECK(?:-NEXT)?:(.*)$", l))]


def padding_prints() -> dict:
    out = {}
    for path in sorted(PAD_SRC.glob("test_*.py")):
        pats = [p.strip() for p in _patterns(path)]
        if "graph:" not in pats:
            continue
        start = pats.index("graph:")
        end = pats.index("", start) if "" in pats[start:] else len(pats)
        out[path.stem] = {"graph": pats[start:end], "code0": "CODE: 0" in pats}
    # the expected error of the invalid pad2d test: "<exception>: <message>"
    out[PAD_INVALID.stem] = {"error": [p.strip() for p in _patterns(PAD_INVALID)][0]}
    return out


def main() -> None:
    out = {}
    for path in sorted(SRC.glob("test_*.py")):
        out[path.stem] = [l.strip() for l in _patterns(path)]
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {len(out)} transcripts to {OUT}")
    pads = padding_prints()
    PAD_OUT.write_text(json.dumps(pads, indent=1) + "\n")
    print(f"wrote {len(pads)} padding graph prints to {PAD_OUT}")


if __name__ == "__main__":
    main()
