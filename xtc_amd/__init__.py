# SPDX-License-Identifier: BSD-3-Clause
"""MI355X (gfx950) execution backend for XTC.

Layout:
  itf/        XTC's interface ABCs (Backend, Scheduler, Compiler, Module, ...)
  graphs/xtc  the graph DSL (O.tensor, O.matmul, O.conv2d, O.pad2d, O.relu, ...)
  backends/hip  Backend -> Scheduler -> Compiler for the HIP kernels
  targets/hip   Module / Evaluator / Executor of compiled HIP payloads
  runtimes/hip  ctypes binding of libxtc_hip.so and the HIP AcceleratorDevice
  search/, cli/ strategies and the loop-explore driver
  csrc/       the HIP kernels and the C-ABI (include/xtc_hip.h)
"""

__version__ = "0.1.0"
