# SPDX-License-Identifier: BSD-3-Clause
"""Abstract interfaces of the XTC pipeline, restated for the HIP backend.

The class names, method names, signatures and return conventions are those of
the reference's `xtc.itf` package (src/xtc/itf/*), so that code written against
XTC's Backend -> Scheduler -> Compiler -> Module -> Evaluator/Executor
pipeline drives this backend unchanged.
"""

from . import back, comp, data, exec, graph, operator, runtime, schd, search

__all__ = ["back", "comp", "data", "exec", "graph", "operator", "runtime", "schd", "search"]
