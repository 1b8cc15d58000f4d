# SPDX-License-Identifier: BSD-3-Clause
"""The XTC graph DSL: operators, expressions, nodes and graphs."""
