# SPDX-License-Identifier: BSD-3-Clause
"""Compile / execute pipeline of a search (src/xtc/search/pipeline.py:16-117).

The reference runs batches: compile a batch of payloads on compile_jobs
threads, then execute it on execute_jobs threads, then the next batch.  On
this backend compiling is a C build on the host and executing a GPU run,
two resources that can be busy at once, so this pipeline keeps compiling
ahead while earlier tasks execute: up to compile_jobs + execute_jobs tasks
are compiled or compiling ahead of the oldest task not yet executed, tasks
execute in id order with at most execute_jobs at a time, and they come out
in id order, as the reference's do.
"""

from __future__ import annotations

import multiprocessing
import time
from collections import deque
from collections.abc import Callable, Generator, Iterable
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass
from typing import Any

__all__ = ["PipelineTask", "CompileExecutePipeline"]


@dataclass
class PipelineTask:
    """One payload through the pipeline: stamps are time.time() at the start
    of each stage, times its duration in seconds."""

    id: int
    payload: Any
    comp_stamp: float = 0
    comp_time: float = 0
    exec_stamp: float = 0
    exec_time: float = 0
    comp_result: Any = None
    exec_result: Any = None


class CompileExecutePipeline:
    """compile_func(payload) -> compiled, execute_func(compiled) -> result.
    compile_jobs < 1 means half the host's CPUs (at least 1), execute_jobs
    < 1 means 1, as in the reference."""

    def __init__(self, compile_func: Callable[[Any], Any], execute_func: Callable[[Any], Any],
                 compile_jobs: int = 0, execute_jobs: int = 0) -> None:
        self._compile_jobs = max(1, multiprocessing.cpu_count() // 2) if compile_jobs < 1 else compile_jobs
        self._execute_jobs = 1 if execute_jobs < 1 else execute_jobs
        self._compile_func = compile_func
        self._execute_func = execute_func

    def _compile(self, task: PipelineTask) -> PipelineTask:
        task.comp_stamp = time.time()
        task.comp_result = self._compile_func(task.payload)
        task.comp_time = time.time() - task.comp_stamp
        return task

    def _execute(self, task: PipelineTask) -> PipelineTask:
        task.exec_stamp = time.time()
        task.exec_result = self._execute_func(task.comp_result)
        task.exec_time = time.time() - task.exec_stamp
        return task

    def generate(self, payloads: Iterable[Any]) -> Generator[PipelineTask, None, None]:
        """Tasks in id order, each yielded once executed.  An exception of a
        compile or execute function is raised here, at its task's turn."""
        source = iter(enumerate(payloads))
        ahead = self._compile_jobs + self._execute_jobs
        compiling: deque[tuple[PipelineTask, Future]] = deque()
        executing: deque[tuple[PipelineTask, Future]] = deque()
        with ThreadPoolExecutor(self._compile_jobs) as cpool, ThreadPoolExecutor(self._execute_jobs) as epool:

            def refill() -> None:
                while len(compiling) + len(executing) < ahead:
                    nxt = next(source, None)
                    if nxt is None:
                        return
                    task = PipelineTask(id=nxt[0], payload=nxt[1])
                    compiling.append((task, cpool.submit(self._compile, task)))

            refill()
            while compiling or executing:
                while compiling and len(executing) < self._execute_jobs:
                    task, done = compiling.popleft()
                    done.result()
                    executing.append((task, epool.submit(self._execute, task)))
                    refill()
                task, done = executing.popleft()
                done.result()
                refill()
                yield task

    def run(self, payloads: Iterable[Any]) -> list[PipelineTask]:
        return list(self.generate(payloads))
