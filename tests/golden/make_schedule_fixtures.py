# SPDX-License-Identifier: BSD-3-Clause
"""Extracts the expected outputs of the reference's schedule-description tests.

Reads, as text, /root/reference/tests/filecheck/schedules/{test_descript_pretty_print,
test_get_descript, test_low_level_validation, test_descript_parsing_errors}.py
and keeps, per FileCheck prefix, the patterns of the `CHECK-<PREFIX>:` and
`CHECK-<PREFIX>-NEXT:` comment lines in order.  Writes
tests/golden/schedule_prints.json as {file: {prefix: [patterns]}} (data
only).  Run once in the build container; the fixture is committed.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

SRC = Path("/root/reference/tests/filecheck/schedules")
FILES = ["test_descript_pretty_print", "test_get_descript", "test_low_level_validation", "test_descript_parsing_errors"]
OUT = Path(__file__).resolve().parent / "schedule_prints.json"


def main() -> None:
    out: dict[str, dict[str, list[str]]] = {}
    for name in FILES:
        per: dict[str, list[str]] = {}
        for line in (SRC / f"{name}.py").read_text().splitlines():
            m = re.match(r"^#\s*CHECK-([A-Z][A-Z-]*?)(?:-NEXT)?:(.*)$", line)
            if m:
                per.setdefault(m.group(1), []).append(m.group(2).rstrip())
        out[name] = per
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
