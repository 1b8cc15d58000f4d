# SPDX-License-Identifier: BSD-3-Clause
"""`import xtc_amd.graphs.xtc.op as O` (src/xtc/graphs/xtc/op.py)."""

from .builder import graph_builder as graph  # noqa: F401
from .op_factory import *  # noqa: F401,F403
