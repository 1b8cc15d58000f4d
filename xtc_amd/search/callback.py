# SPDX-License-Identifier: BSD-3-Clause
"""Result callbacks of an exploration (src/xtc/search/callback.py:22-166).

A callback is called once per evaluated sample with the result tuple
(sample, code, time, backend): code 0 for a timed sample, time its minimum
over the repeats in seconds.  CSVCallback writes the explorer's CSV,
DBCallback one JSON line per sample in the results-DB record format
(src/xtc/cli/query_results.py:25-123), MemoryCallback keeps the tuples.
"""

from __future__ import annotations

import csv
import hashlib
import json
import logging
import os
import platform
from abc import ABC, abstractmethod
from collections.abc import Sequence
from pathlib import Path
from typing import Any

__all__ = ["ResultCallBack", "CSVCallback", "DBCallback", "MemoryCallback", "DB_VERSION", "db_operator",
           "db_strategy"]

logger = logging.getLogger(__name__)

DB_VERSION = "v0.2"


def db_operator(graph: Any) -> list[Any]:
    """["xtc.graph", sha1 of the graph dict without its name, the dict]."""
    obj = graph.to_dict()
    obj.pop("name", None)
    return ["xtc.graph", hashlib.sha1(json.dumps(obj).encode()).hexdigest(), obj]


def db_strategy(name: str) -> list[Any]:
    return ["xtc.strategy", hashlib.sha1(json.dumps(name).encode()).hexdigest(), name]


class ResultCallBack(ABC):
    @abstractmethod
    def __call__(self, result: Sequence) -> None: ...


class MemoryCallback(ResultCallBack):
    """Keeps every result tuple in `results`."""

    def __init__(self) -> None:
        self.results: list[Sequence] = []

    def __call__(self, result: Sequence) -> None:
        self.results.append(result)


class CSVCallback(ResultCallBack):
    """One row per timed sample: the sample's values, X (the sample with ';'
    separators), time, peak (peak_time / time) and backend.

    * default: the file is rewritten, header first;
    * `append`: rows go after an existing file's, a header only for a new
      or empty file;
    * `resume`: as append, and a (backend, sample) pair already in the file
      (or written since) is skipped.
    Failed samples (code != 0) are not written."""

    def __init__(self, fname: str, peak_time: float, sample_names: list[str], *, resume: bool = False,
                 append: bool = False) -> None:
        self._fname = fname
        self._peak_time = peak_time
        self._names = list(sample_names)
        self._resume = resume
        # (backend, sample) pairs in the file: read back under resume, then every row written
        self.seen: set[tuple[str, tuple[int, ...]]] = set()
        path = Path(fname)
        existing = path.exists() and path.stat().st_size > 0
        if resume and existing:
            with open(path, newline="") as f:
                for row in csv.DictReader(f):
                    try:
                        self.seen.add((row["backend"], tuple(int(row[n]) for n in self._names)))
                    except (KeyError, TypeError, ValueError):
                        continue
        mode = "a" if (resume or append) else "w"
        self._f = open(path, mode, newline="")
        self._w = csv.writer(self._f)
        if mode == "w" or not existing:
            self._w.writerow(self._names + ["X", "time", "peak", "backend"])
            self._f.flush()

    def __call__(self, result: Sequence) -> None:
        sample, code, t, backend = result
        if code != 0:
            return
        key = (backend, tuple(int(v) for v in sample))
        if self._resume and key in self.seen:
            return
        x = str([int(v) for v in sample]).replace(",", ";")
        self._w.writerow([*sample, x, t, self._peak_time / t if t > 0 else 0.0, backend])
        self._f.flush()
        try:
            os.fsync(self._f.fileno())
        except OSError:
            logger.debug("no fsync for %s", self._fname)
        self.seen.add(key)

    def close(self) -> None:
        if not self._f.closed:
            self._f.close()

    def __del__(self) -> None:
        f = getattr(self, "_f", None)
        if f is not None and not f.closed:
            f.close()


class DBCallback(ResultCallBack):
    """Appends one JSON line per sample to `dbfile`: version, platform,
    compiler [xtc, version, target, threads, backend], operator (set by
    set_graph), strategy, schedule and results [code, [seconds]], with
    time 0 for a failed sample.  `record(result, extra)` adds fields of this
    backend's own (the kernel instance per node, the error text, counters)."""

    def __init__(self, dbfile: str, target: str, threads: int, strategy: str) -> None:
        from .. import __version__

        self._dbfile = dbfile
        self._platform = [platform.node().split(".")[0], platform.system(), platform.machine()]
        self._compiler = ["xtc", "v" + __version__, target, threads]
        self._strategy = db_strategy(strategy)
        self._operator: list[Any] | None = None

    def set_graph(self, graph: Any) -> None:
        self._operator = db_operator(graph)

    def record(self, result: Sequence, extra: dict[str, Any] | None = None) -> None:
        sample, code, t, backend = result
        rec = {
            "version": [DB_VERSION],
            "platform": self._platform,
            "compiler": [*self._compiler, backend],
            "operator": self._operator,
            "strategy": self._strategy,
            "schedule": [int(v) for v in sample],
            "results": [int(code), [float(t) if code == 0 else 0.0]],
            **(extra or {}),
        }
        with open(self._dbfile, "a") as f:
            f.write(json.dumps(rec) + "\n")

    def __call__(self, result: Sequence) -> None:
        self.record(result)

    def close(self) -> None:
        """Nothing to release: every record opens and closes the file."""
