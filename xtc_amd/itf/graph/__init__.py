# SPDX-License-Identifier: BSD-3-Clause
"""Graph, Node and Operation interfaces (src/xtc/itf/graph/)."""

from .graph import Graph
from .node import Node
from .operation import AccessesMaps, Operation

__all__ = ["Graph", "Node", "Operation", "AccessesMaps"]
