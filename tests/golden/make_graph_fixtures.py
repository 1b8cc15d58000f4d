# SPDX-License-Identifier: BSD-3-Clause
"""Extracts the expected transcripts of the reference's graph tests.

Reads, as text, /root/reference/tests/filecheck/graphs/test_*.py and keeps
only the expected output of each: the patterns of its FileCheck `CHECK:` /
`CHECK-NEXT:` comment lines, in order.  Writes
tests/golden/graph_prints.json as {test name: [pattern lines]} (data only).
Run once in the build container; the fixture is committed.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

SRC = Path("/root/reference/tests/filecheck/graphs")
OUT = Path(__file__).resolve().parent / "graph_prints.json"


def main() -> None:
    out = {}
    for path in sorted(SRC.glob("test_*.py")):
        lines = [m.group(1) for l in path.read_text().splitlines() if (m := re.match(r"^#\s*CHECK(?:-NEXT)?:(.*)$", l))]
        out[path.stem] = [l.strip() for l in lines]
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {len(out)} transcripts to {OUT}")


if __name__ == "__main__":
    main()
