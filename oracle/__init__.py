# SPDX-License-Identifier: BSD-3-Clause
"""Test infrastructure: the CPU oracle of the XTC HIP backend.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker or the timed CPU
baseline.  Nothing in `xtc_amd/` imports it: the product path has no CPU
fallback.

Contents
--------
* `reference`  -- float64 numpy restatement of the operator semantics of the
  reference's graph interpreter (src/xtc/graphs/xtc/operators.py) and its
  I/O conventions (src/xtc/utils/numpy.py, src/xtc/utils/evaluation.py),
  plus the seeded inputs and the tolerance metric used by the parity tests.
* `cpu_backend` -- C restatement of the compiled MLIR `llvmir` CPU backend
  (tiled loop nest + OpenMP, src/xtc/backends/mlir/MlirCompilerPasses.py and
  MlirLLVMTarget.py) used as the CPU baseline; `cpu_baseline.load()` builds
  it with -march=native once per host into oracle/_build/<host>/.
* `Makefile` -- builds the reference's own host runtime (evaluate_perf,
  CNDArray, evaluate_flops) from its C sources into oracle/_ref/, used by
  `cpu_baseline` as the timing harness when present.

Pinning (each oracle function is checked against something that is not a
retyping of its own formula):
* matmul      -- integer known-answer tests (exact in fp32 while 81*K < 2^24),
                 closed forms (ones @ ones = K, identity, rank-1 u v^T), and the
                 reference's golden prints (tests/filecheck/graphs/test_matmul.py,
                 test_mlp.py, test_mlp_fc.py).
* conv2d      -- brute-force direct loop on small shapes, the reference golden
                 print of tests/filecheck/graphs/test_conv_relu.py, a 1x1
                 conv == matmul identity and integer known-answer tests.
* relu / pad  -- numpy.maximum / numpy.pad special cases and the reference
                 golden prints (test_relu.py, test_matmul_relu.py).
"""
